// Decode MLP, gate/up half: out = down( fp16(silu(g) * u) ), [g | u] =
// fp16(gate_up(x)), the arithmetic of the reference's production path
// (langburst/adapters/qwen36_impl/model.py:1460-1470: the gate_up Marlin
// projection, then `down.gemm_silu_packed`, loader.py:337-368).  The gate_up
// launch below pairs the gate and up chunks of the same neurons in each decode
// tile and stores fp16(silu(g) * u) instead of [g | u]; the down projection
// then runs over those activations (lb_marlin.hip, lb_marlin_mlp_fused).

#pragma once
#include "marlin_skinny.hpp"

namespace lb {
namespace mlp {

// The two-launch form's gate_up launch for decode batches: the tiles the
// plain gate_up projection plans (same k splits, so every g and u sums the
// same terms in the same order), with the gate and up chunks of the same
// neurons paired per tile, storing fp16(silu(g) * u) of the fp16 outputs
// (skinny::EPI_ACT) for the down projection instead of [g | u].  Scalar
// arguments, those the prologue and the split hand-off read first, so that
// they arrive preloaded in SGPRs (as for skinny::marlin_skinny_kernel); the
// tile count and the gate half's chunk count follow from N.
template <int AM, bool G, int CPW, int MR>
__global__ __launch_bounds__(skinny::kThreads) void mlp_gate_up_act_kernel(const uint16_t* a, const uint32_t* b,
                                                                           const uint16_t* s, int m, int n, int k,
                                                                           int splits, float* partial,
                                                                           int32_t* counters, uint32_t* act_out) {
  skinny::Params p{};
  p.a = a; p.b = b; p.s = s; p.partial = partial; p.counters = counters; p.act_out = act_out;
  p.m = m; p.n = n; p.k = k; p.splits = splits; p.kp_total = k >> 5;
  p.n_cg = n / (64 * CPW);
  p.gate_chunks = n / 128;
  skinny::skinny_tile<AM, skinny::EPI_ACT, G, CPW, MR>(p, blockIdx.x, blockIdx.y);
}

}  // namespace mlp
}  // namespace lb
