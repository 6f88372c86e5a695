// Whole decode MLP in one launch on gfx950:
//   out = down( fp16(silu(g) * u) ),  [g | u] = fp16(gate_up(x)),
// the arithmetic of the reference's production path, which runs it as two
// projections (langburst/adapters/qwen36_impl/model.py:1460-1470: the gate_up
// Marlin projection, then `down.gemm_silu_packed`, loader.py:337-368).
//
// Phase 1 runs the gate_up projection's decode tiles with gate and up chunks
// paired in each tile (skinny::EPI_ACT): the workgroup that completes a tile
// forms fp16(silu(g) * u) of its neurons with the same instruction sequence as
// the SiLU-gated A staging and publishes it (device-coherent stores).  Phase 2
// runs the down projection's decode tiles over those activations
// (skinny::A_HANDOFF, device-coherent loads).  Both phases use the tilings the
// separate projections use, so every output column sums the same fp32 terms
// in the same order: the result is bit-identical to the two launches.
//
// Hand-off without a grid barrier.  A gate_up tile covers 32 * CPW1 neurons,
// which lie in one scale group of the down projection's K, hence in exactly
// one of its k splits.  The workgroup that completed a tile counts it on that
// split's ready counter; a down workgroup issues its first weight batches,
// then waits until its split's counter holds every tile of the split's k
// range, then stages its activations.  Afterwards it counts its departure;
// the split's last departure zeroes both counters.
//
// The waits need every workgroup of the launch resident at once (a waiting
// workgroup must not hold the slot a producer needs); the host launches this
// kernel only when the instantiation's occupancy allows it and otherwise runs
// the two projections.  Each wait is bounded: a workgroup that has polled
// kSpinLimit times records a fault flag (workspace entry 1) and goes on, so a
// launch always ends.  The output of such a launch is not valid, and a late
// producer may still count a tile once its split's counters were reset: the
// host entry point runs this kernel only when the caller asks for it, and
// lb_marlin_mlp_fused_check reports the flag and zeroes the workspace.

#pragma once
#include "marlin_skinny.hpp"

namespace lb {
namespace mlp {

constexpr int kSpinLimit = 1 << 18;  // default polls; each waits for its device-scope load, then sleeps 128 cycles
constexpr int kLineInts = 32;        // one 128-byte line per counter
constexpr int kMaxSplits = 64;       // down k splits the counters cover
// workspace layout (int32): [1] fault flag; ready[s] at kReadyBase + kLineInts * s,
// departures[s] at kDepartBase + kLineInts * s
constexpr int kReadyBase = kLineInts;
constexpr int kDepartBase = kReadyBase + kLineInts * kMaxSplits;
constexpr int kSyncWorkspace = kDepartBase + kLineInts * kMaxSplits;

struct FusedParams {
  skinny::Params up;    // gate_up projection (EPI_ACT), N = 2 * intermediate
  skinny::Params down;  // down projection (A_HANDOFF), K = intermediate
  int32_t* ws;          // kSyncWorkspace entries, zero on entry and on exit
  int spin_limit;       // polls before a wait gives up (kSpinLimit unless a test lowers it)
};

// The down split whose k range holds scale group `grp`: split s covers groups
// [floor(G s / S), floor(G (s + 1) / S)) (skinny::split_range).
__device__ __forceinline__ int split_of_group(int grp, int groups, int splits) {
  return ((grp + 1) * splits + groups - 1) / groups - 1;
}

// Producer: every thread's activation stores are acknowledged, then one
// relaxed device-scope add (not waited for) counts the tile.
template <int CPW1>
__device__ __forceinline__ void count_ready(const FusedParams& f, int cg1) {
  wait_published();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int grp = cg1 * 32 * CPW1 / 128;
    const int s = split_of_group(grp, f.down.kp_total >> 2, f.down.splits);
    __hip_atomic_fetch_add(f.ws + kReadyBase + kLineInts * s, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Consumer: thread 0 polls the split's counter (bounded); the other waves wait
// at an LDS-only barrier, so their weight loads in flight stay in flight.
__device__ __forceinline__ void wait_ready(const FusedParams& f, int s, int expected) {
  if (threadIdx.x == 0) {
    int32_t* ready = f.ws + kReadyBase + kLineInts * s;
    int spins = 0;
    while (__hip_atomic_load(ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < expected) {
      if (++spins > f.spin_limit) {
        __hip_atomic_store(f.ws + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  lds_barrier();
}

// Workgroup w runs tile (w mod n_cg, w / n_cg) of each phase, the order in
// which the separate launches dispatch their (x, y) grids.
template <bool G1, int CPW1, bool G2, int CPW2>
__global__ __launch_bounds__(skinny::kThreads) void marlin_mlp_fused_kernel(FusedParams f) {
  const int w = blockIdx.x;
  if (w < f.up.n_cg * f.up.splits) {
    const int cg1 = w % f.up.n_cg;
    if (skinny::skinny_tile<skinny::A_PLAIN, skinny::EPI_ACT, G1, CPW1>(f.up, cg1, w / f.up.n_cg))
      count_ready<CPW1>(f, cg1);
  }
  if (w < f.down.n_cg * f.down.splits) {
    const int s = w / f.down.n_cg;
    const int groups = f.down.kp_total >> 2;
    const int g0 = (int)(((int64_t)groups * s) / f.down.splits);
    const int g1 = (int)(((int64_t)groups * (s + 1)) / f.down.splits);
    const int expected = (g1 - g0) * (128 / (32 * CPW1));  // gate_up tiles of the split
    skinny::skinny_tile<skinny::A_HANDOFF, skinny::EPI_STORE, G2, CPW2>(f.down, w % f.down.n_cg, s,
                                                                        [&]() { wait_ready(f, s, expected); });
    if (threadIdx.x == 0 && arrive(f.ws + kDepartBase + kLineInts * s) == f.down.n_cg - 1) {
      reset_counter(f.ws + kReadyBase + kLineInts * s);
      reset_counter(f.ws + kDepartBase + kLineInts * s);
    }
  }
}

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
