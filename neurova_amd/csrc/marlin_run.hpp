// Host entry of the Marlin-layout projections (defined in lb_marlin.hip),
// shared by the C-ABI translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lb {
namespace marlin {

// V_SILU_DONE: the SiLU-gated projection's plan and sums, with A given as the
// gated activations fp16(silu(g) * u) [M][K] (decode batches, M <= 32).
enum Variant { V_PLAIN = 0, V_SILU = 1, V_ARGMAX = 2, V_SILU_DONE = 3 };

// Validates, plans and launches one projection on `st`; `scratch` holds the
// split-K partials (and the argmax tile keys) the plan needs.  Returns an
// lb_status code; never allocates.
int run(Variant var, const uint16_t* a, const int32_t* b, uint16_t* c, const uint16_t* s, int64_t m, int64_t n,
        int64_t k, int32_t* workspace, int64_t workspace_len, int64_t groupsize, int64_t* argmax_state,
        int64_t* argmax_out, void* scratch, size_t scratch_bytes, hipStream_t st);

}  // namespace marlin
}  // namespace lb
