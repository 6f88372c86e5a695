// Host dispatch and C-ABI entry points for the Marlin-layout W4A16 path:
// GEMM (decode and prefill kernels), SiLU-gated A prologue, fused argmax,
// dense dequant, the streaming MLP and the two-launch decode MLP.

#include <stdlib.h>

#include <algorithm>


#include "marlin_gemm.hpp"
#include "marlin_run.hpp"
#include "marlin_mlp.hpp"
#include "marlin_skinny.hpp"

namespace lb {
namespace marlin {

// ---------------------------------------------------------------------------
// Dense dequant W[N, K] (test / utility path).  Closed-form position of
// weight (k, n) in the Marlin layout: row kb = k>>4, chunk n>>6, slot
// 4c+q (c = n&7, q = (k&7)>>1), word j = (n&63)>>4, nibble
// 4*(k&1) + 2*((n>>3)&1) + (k>>3 & 1).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t code_at(const uint32_t* b, int64_t n_total, int64_t k, int64_t n) {
  const int64_t kb = k >> 4;
  const int ki = (int)(k & 15);
  const int nn = (int)(n & 63);
  const int j = nn >> 4, c = nn & 7, h = (nn >> 3) & 1;
  const int q = (ki & 7) >> 1;
  const int nib = 4 * (ki & 1) + 2 * h + (ki >> 3);
  const uint32_t w = b[kb * 2 * n_total + (n >> 6) * 128 + (4 * c + q) * 4 + j];
  return (w >> (4 * nib)) & 15u;
}

__device__ __forceinline__ uint16_t scale_at(const uint16_t* s, int64_t n_total, int64_t grp, int64_t n, int grouped) {
  if (grouped) {
    const int nn = (int)(n & 63);
    return s[grp * n_total + (n >> 6) * 64 + 8 * (nn & 7) + (nn >> 3)];
  }
  const int r = (int)(n & 31);
  return s[(n & ~31LL) + 8 * ((r >> 1) & 3) + ((r >> 3) << 1) + (r & 1)];
}

__global__ void dequant_kernel(const uint32_t* __restrict__ b, const uint16_t* __restrict__ s, uint16_t* __restrict__ w,
                               int64_t n_total, int64_t k_total, int grouped) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n_total * k_total) return;
  const int64_t n = idx / k_total;
  const int64_t k = idx - n * k_total;
  const f16 q = (f16)((int)code_at(b, n_total, k, n) - 8);
  f16 v = q;
  if (grouped) v = q * __builtin_bit_cast(f16, scale_at(s, n_total, k >> 7, n, 1));
  w[idx] = __builtin_bit_cast(uint16_t, v);
}

// ---------------------------------------------------------------------------
// Streaming-MLP numerics (float32 weights (q-8)*s, float32 activations).
// One wave per (64-column chunk, k split); each lane reads its natural
// 16-byte slot (fully coalesced) and keeps 8 column sums per batch row.
// ---------------------------------------------------------------------------
constexpr int kF32Batch = 4;

template <bool XF32>
__global__ __launch_bounds__(64) void f32_gemv_kernel(const uint32_t* __restrict__ b, const uint16_t* __restrict__ s,
                                                      const void* __restrict__ xin, float* __restrict__ partial,
                                                      int m_total, int64_t n_total, int64_t k_total, int grouped,
                                                      int splits) {
  const int lane = threadIdx.x;
  const int64_t chunk = blockIdx.x;
  const int split = blockIdx.y;
  const int m0 = blockIdx.z * kF32Batch;
  const int pr = lane >> 5, slot = lane & 31, c = slot >> 2, q = slot & 3;
  const int64_t kp_total = k_total >> 5;
  const int64_t kp0 = kp_total * split / splits, kp1 = kp_total * (split + 1) / splits;
  float acc[kF32Batch][4][2];
#pragma unroll
  for (int mm = 0; mm < kF32Batch; ++mm)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[mm][j][0] = acc[mm][j][1] = 0.f;
  for (int64_t kp = kp0; kp < kp1; ++kp) {
    const int64_t kb = 2 * kp + pr;
    const u32x4 w = *reinterpret_cast<const u32x4*>(b + kb * 2 * n_total + chunk * 128 + slot * 4);
    const int64_t kbase = kb * 16 + 2 * q;  // k offsets {0, 1, 8, 9}
    float xv[kF32Batch][4];
#pragma unroll
    for (int mm = 0; mm < kF32Batch; ++mm) {
      const int m = min(m0 + mm, m_total - 1);
      const int64_t off = (int64_t)m * k_total + kbase;
      if (XF32) {
        const float* x = reinterpret_cast<const float*>(xin);
        xv[mm][0] = x[off]; xv[mm][1] = x[off + 1]; xv[mm][2] = x[off + 8]; xv[mm][3] = x[off + 9];
      } else {
        const uint16_t* x = reinterpret_cast<const uint16_t*>(xin);
        xv[mm][0] = h2f(x[off]); xv[mm][1] = h2f(x[off + 1]); xv[mm][2] = h2f(x[off + 8]); xv[mm][3] = h2f(x[off + 9]);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t word = w[j];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int64_t n = chunk * 64 + 16 * j + 8 * h + c;
        const float sc = h2f(scale_at(s, n_total, grouped ? (kb * 16) >> 7 : 0, n, grouped));
        // nibbles for column c+8h: k offsets 0 (nib 2h), 8 (nib 2h+1), 1 (nib 4+2h), 9 (nib 5+2h)
        const float w0 = (float)((int)((word >> (8 * h)) & 15u) - 8) * sc;
        const float w8 = (float)((int)((word >> (8 * h + 4)) & 15u) - 8) * sc;
        const float w1 = (float)((int)((word >> (16 + 8 * h)) & 15u) - 8) * sc;
        const float w9 = (float)((int)((word >> (20 + 8 * h)) & 15u) - 8) * sc;
#pragma unroll
        for (int mm = 0; mm < kF32Batch; ++mm)
          acc[mm][j][h] += w0 * xv[mm][0] + w1 * xv[mm][1] + w8 * xv[mm][2] + w9 * xv[mm][3];
      }
    }
  }
#pragma unroll
  for (int mm = 0; mm < kF32Batch; ++mm)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float v = quad_sum(acc[mm][j][h]);
        v += __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, __builtin_bit_cast(int, v)));
        if (lane < 32 && q == 0 && m0 + mm < m_total)
          partial[((int64_t)split * m_total + m0 + mm) * n_total + chunk * 64 + 16 * j + 8 * h + c] = v;
      }
}

__global__ void mlp_act_kernel(const float* __restrict__ gu, float* __restrict__ act, int m_total, int64_t inter,
                               int splits) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)m_total * inter) return;
  const int64_t m = idx / inter, i = idx - m * inter;
  float g = 0.f, u = 0.f;
  for (int sp = 0; sp < splits; ++sp) {
    const float* row = gu + ((int64_t)sp * m_total + m) * 2 * inter;
    g += row[i];
    u += row[inter + i];
  }
  act[idx] = (g / (1.0f + __expf(-g))) * u;
}

__global__ void f32_finalize_kernel(const float* __restrict__ partial, uint16_t* __restrict__ out, int64_t count,
                                    int splits) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= count) return;
  float v = 0.f;
  for (int sp = 0; sp < splits; ++sp) v += partial[(int64_t)sp * count + idx];
  out[idx] = f2h(v);
}

// ---------------------------------------------------------------------------
// Planning
// ---------------------------------------------------------------------------
constexpr size_t kAlign = 256;
inline size_t align_up(size_t v) { return (v + kAlign - 1) & ~(kAlign - 1); }

struct Plan {
  bool skinny = true;
  bool direct = false; // decode kernel without the whole-slice A staging: A fragments loaded per
                       // step (skinny::A_DIRECT), or, on 4-chunk tiles, an LDS ring (skinny::A_RING)
  int mr = 1;          // decode: 16-row blocks of the MFMA tile
  int mb = 1;        // GEMM: 16-row blocks per workgroup
  int n_mb = 1;
  int n_cg = 0;      // column tiles (decode: 64 * cpw columns; GEMM: 256)
  int cpw = 4;       // decode: chunks (64 columns) per workgroup
  int splits = 1;    // decode: K splits of every column tile (mixed plans: of the tiles past `whole`)
  int whole = 0;     // decode, mixed plan: the first `whole` tiles run over the whole K, unsplit
  int full_tiles = 0;   // GEMM: tiles computed whole
  int tail_tiles = 0;   // GEMM: tiles split over K ...
  int tail_splits = 1;  // ... this many ways
  int sk_wgs = 0;       // GEMM: > 0, the stream-K schedule over this many workgroups
  int64_t wgs = 0;      // GEMM workgroups
  size_t lds = 0;    // decode kernel dynamic LDS
  size_t x_bytes = 0; // decode kernel: staged activations
  size_t partial_bytes = 0;
  size_t keys_bytes = 0;
  size_t act_bytes = 0;  // A_DIRECT with SiLU-gated A: fp16(silu(g) * u) [M][K], after the partials
};

constexpr int kSkinnyWGsPerCU = 2;  // decode workgroups resident per CU (register-limited)
constexpr int kGemmMaxTailSplits = 16;
constexpr int kSkinnyMaxSplits = 8;  // decode: beyond this, narrower tiles instead
constexpr size_t kSkinnyMaxX = 48 * 1024;

using lbh::device_cus;

// GEMM tail split: the tiles left after the last full round of resident
// workgroups are split over K.  S minimises the tail's length in scale-group
// times, ceil(T*S / slots) * ceil(G / S), plus a charge per extra split for the
// partials written and summed by the last arrival: about kGemmSplitCharge
// group times for a 128-row tile (MB = 8), in proportion to the tile's rows,
// and not growing with K (fitted to M = 2048 sweeps of S = 2..12: K = 5120,
// N = 17408 runs fastest at S = 3, 290 against 294 us at S = 4; K = 17408,
// N = 5120 at S = 3, 309.5 against 318 us at S = 4).
constexpr int kGemmSplitCharge = 5;
inline int choose_tail_splits(int64_t tail, int64_t slots, int groups, int mb) {
  int best = 1;
  int64_t best_cost = 8 * (int64_t)groups;  // in eighths of a group time
  for (int s = 2; s <= kGemmMaxTailSplits && s <= groups; ++s) {
    const int64_t rounds = (tail * s + slots - 1) / slots;
    const int64_t cost = 8 * rounds * ((groups + s - 1) / s) + (int64_t)kGemmSplitCharge * mb * (s - 1);
    if (cost < best_cost) {
      best_cost = cost;
      best = s;
    }
  }
  return best;
}

// Decode tiling with `cpw` chunks per workgroup: the k split count, or 0
// when the tiling cannot run (some wave would get no scale group, or the
// staged A slice does not fit LDS without the workspace to split K).
// `direct`: A is not staged (skinny::A_DIRECT), so LDS sets no bound.
inline int skinny_splits(int64_t m, int64_t n, int64_t k, int64_t workspace_len, int cpw, bool direct = false) {
  const int n_cg = (int)(n / (64 * cpw));
  const int ksub = skinny::kWaves / cpw;
  const int groups = (int)(k / 128);
  // split counters: one per chunk for wide tiles (each wave hands off on its
  // own), one per tile otherwise
  const bool can_split = workspace_len >= 1 + (cpw == skinny::kWaves ? n / 64 : (int64_t)n_cg);
  // As many k splits as fit in one wave of resident workgroups: a second,
  // partial wave would cost a whole workgroup's time for a few tiles.
  int s = (kSkinnyWGsPerCU * device_cus()) / n_cg;
  // split-K partials (S * M * N fp32, written once and read once) stay
  // within half the weight bytes (K * N / 2): S * M <= K / 32
  const int s_traffic = (int)std::max<int64_t>(1, k / (32 * m));
  if (s > s_traffic) s = s_traffic;
  // the decode kernel stages its whole A slice in LDS
  // (whole scale groups: at most kSkinnyMaxX / (256 M) groups per split)
  const int64_t lds_groups = std::max<int64_t>(1, (int64_t)kSkinnyMaxX / (256 * m));
  const int s_lds = direct ? 1 : (int)((groups + lds_groups - 1) / lds_groups);
  if (s < s_lds) s = s_lds;
  if (s > groups / ksub) s = groups / ksub;  // every wave at least one group
  if (s > 256) s = 256;  // the kernel's split arithmetic is 32-bit: groups * S < 2^32
  if (s < 1) s = 1;
  if (!can_split) s = 1;
  if (groups / s < ksub) return 0;
  if (!direct && (size_t)((groups + s - 1) / s) * 128 * (size_t)m * 2 > kSkinnyMaxX) return 0;
  return s;
}

// Decode tilings (M <= 16 staged, M <= 32 direct): the chunks per workgroup
// and the k split count, or cpw = 0 when none runs.
struct Tiling {
  int cpw = 0, s = 0;
};

// Staged A (M <= 16): 4 chunks (one per wave) per workgroup, unless the
// narrow N then needs more than kSkinnyMaxSplits k splits to fill the chip:
// then 2 or 1 chunks, whose waves share the workgroup's k range.
inline Tiling staged_tiling(int64_t m, int64_t n, int64_t k, int64_t workspace_len) {
  Tiling t;
  for (int c = skinny::kWaves; c >= 1; c /= 2) {
    const int sc = skinny_splits(m, n, k, workspace_len, c);
    if (sc == 0) continue;
    if (t.cpw == 0 || sc < t.s) {
      t.cpw = c;
      t.s = sc;
    }
    if (t.s <= kSkinnyMaxSplits) break;
  }
  return t;
}

// Without the whole-slice staging: the split cap S * M <= K / 32 bites early
// at larger M; the widest tiling within kSkinnyMaxSplits splits that gives
// every CU a workgroup (4-chunk tiles, whose waves share A through the LDS
// ring) or 1.5 workgroups per CU (narrower tiles, each wave loading its own
// A), else the one with the most workgroups.
inline Tiling direct_tiling(int64_t m, int64_t n, int64_t k, int64_t workspace_len) {
  Tiling t;
  // From M = 12 (M = 8 at long K) with fewer 64-column chunks than CUs:
  // single-chunk tiles split to about one workgroup per CU instead of two
  // (M = 32, K = 5120: N = 5120 11.6 against 12.6 us, 14.2 at 1.5 per CU;
  // K = 17408, N = 5120: 22.3 against 23.5; M = 16: 15.2 against 16.3, N = 7168
  // 9.8 against 10.1; M = 12 even at K = 5120, 14.3 against 15.1 at K = 17408;
  // M = 8: 13.6 against 14.1 at K = 17408, 0.3 us slower at K = 5120, as at M
  // = 1 and 4)
  if ((m >= 12 || (m >= 8 && k > 8192)) && n / 64 < device_cus() && k / 128 >= skinny::kWaves) {
    const int64_t tiles = n / 64;
    int s = (int)std::max<int64_t>(1, device_cus() / tiles);
    s = std::min<int>(s, (int)std::max<int64_t>(1, k / (32 * m)));  // partials within half the weight bytes
    s = std::min<int>(s, (int)(k / 128 / skinny::kWaves));  // every wave a scale group
    if (workspace_len < 1 + tiles) s = 1;
    return Tiling{1, s};
  }
  int64_t most = -1;
  for (int c = skinny::kWaves; c >= 1; c /= 2) {
    const int sc = skinny_splits(m, n, k, workspace_len, c, true);
    if (sc == 0) continue;
    const int64_t w = (n / (64 * c)) * sc;
    const int64_t fill = c == skinny::kWaves ? device_cus() : 3 * (int64_t)device_cus() / 2;
    if (sc <= kSkinnyMaxSplits && w >= fill) return Tiling{c, sc};
    if (w > most) {
      most = w;
      t = Tiling{c, sc};
    }
  }
  return t;
}

// `am`: the A mode of the launch (gemm::A_PLAIN or gemm::A_SILU_PACKED);
// `argmax`: the fused-argmax variant; `allow_mixed`: the mixed whole-K plan
// may be used (grouped scales only).
//
// Which decode form (measured on the decode shapes of BASELINE.json): the direct
// form where the tiles are narrow (the waves of a workgroup then share
// little A, and staging the whole slice before the loop holds them up), or
// where LDS forces the staged form to more splits than one wave of resident
// workgroups (on 4-chunk tiles, A then goes through the LDS ring); the
// staged form where 4-chunk tiles share the slice.  The SiLU-gated direct
// form first forms fp16(silu(g) * u) in a launch of its own, which does not
// pay below 5 rows.  M = 17..32: the direct form on 64-column tiles (whole-K
// tiles where the chunks cover the CUs, below that about one workgroup per
// CU), the ring on 4-chunk tiles; 2-chunk tiles go to the prefill kernel.
constexpr int64_t kMixedMaxPerCu = 2;  // whole-K tiles per CU (more was not measured)
constexpr int64_t kMixedMaxM = 4;      // rows with the A slice staged (measured at M = 1..4)
constexpr int64_t kMixedDirectMaxM = 32;    // rows with A loaded per step, one whole-K tile per CU
constexpr int64_t kMixedDirectMaxM2 = 8;    // ... and with two whole-K tiles per CU

inline Plan make_plan(int64_t m, int64_t n, int64_t k, int64_t workspace_len, int am, bool argmax = false,
                      bool allow_mixed = true) {
  Plan pl;
  pl.n_cg = (int)(n / 256);
  const int groups = (int)(k / 128);
  // Whole-K plan, up to four rows of A, grouped scales, K <= 5120, and between
  // half a chunk (64 columns) and two chunks per CU: single-chunk tiles over
  // the whole K (the four waves' k shares summed in LDS, no split-K hand-off),
  // one or two per CU, and the chunks left over (at most CUs / 8) split over K
  // among at most one more workgroup per CU.  Measured (one process, graph
  // replay) against the split tiles: N = 16384 11.6 against 13.0 us, the
  // headline N = 17408 12.45 against 13.38 (M = 2, 3: 12.6 / 12.8 against
  // 13.8 / 13.9), gate/up N = 34816 21.2 against 21.9.  With one scale per
  // column it was slower (13.7 against 12.6 us): `allow_mixed` false.  At M = 4
  // 16 leftover chunks lose on 10 leftover splits (14.2 against 13.9 us) and
  // gain on 6 (13.2 against 13.4; gate/up 20.2 against 22.1), so M = 4 caps
  // the leftover splits at 6.  M = 5..32: the same tiles with A loaded per step
  // (the direct form; the slice no longer fits LDS), where the chunks give at
  // least 5/8 of the CUs one whole-K tile (N = 17408: M = 8 12.4 against 14.1
  // us, M = 16 15.0 against 16.0, M = 32 22.2 against 23.7 on the split tiles;
  // N = 14336: M = 8 10.5 against 13.5, M = 32 17.6 against 24.6; N = 10240:
  // M = 16 11.5 against 12.5; at half, N = 8192, M = 32 18.3 against 14.3) or
  // two per CU up to M = 8 (N = 34816, M = 8: 20.9 against 22.6 us; M = 16 even,
  // M = 32 39.2 against 31.2 on the ring tiles).
  const int64_t chunks_all = n / 64, cus_all = device_cus();
  const bool mixed_direct = m > kMixedMaxM && m <= kMixedDirectMaxM && chunks_all * 8 >= cus_all * 5 &&
                            (chunks_all < 2 * cus_all || m <= kMixedDirectMaxM2);
  if ((m <= kMixedMaxM || mixed_direct) && allow_mixed && !argmax && am == gemm::A_PLAIN) {
    const int64_t chunks = chunks_all, cus = cus_all;
    const int ksub = skinny::kWaves;  // 1-chunk tiles: the four waves share the k range
    // (measured at K <= 5120 and up to CUs / 8 leftover chunks; a longer K or
    // more leftover work per CU keeps the split tiles)
    int64_t per = std::min<int64_t>(chunks / cus, kMixedMaxPerCu), whole = per * cus;
    // Fewer chunks than CUs but at least half as many: one whole-K tile per
    // chunk and no split at all (K = 5120, M = 1: N = 14336 10.1 against 12.7
    // us, N = 10240 9.7 against 10.9, N = 8192 9.6 against 10.1; below half,
    // N = 7168 9.6 against 8.8 us, the split tiles stay).
    if (per == 0 && chunks * 2 >= cus) {
      per = 1;
      whole = chunks;
    }
    if (per >= 1 && (chunks - whole) * 8 <= cus && groups >= ksub && k <= 5120) {
      const int64_t left = chunks - whole;
      const int s = left > 0 ? (int)std::min<int64_t>(std::min<int64_t>(cus / left, groups / ksub), m >= 4 ? 6 : 256) : 1;
      if (left == 0 || (s >= 2 && workspace_len >= 1 + chunks)) {
        pl.skinny = true;
        pl.direct = mixed_direct;
        pl.mr = mixed_direct ? (int)((m + 15) / 16) : 1;
        pl.cpw = 1;
        pl.n_cg = (int)chunks;
        pl.whole = (int)whole;
        pl.splits = s;
        pl.x_bytes = mixed_direct ? 0 : (size_t)groups * 128 * (size_t)m * 2;
        pl.lds = std::max(mixed_direct ? 0 : pl.x_bytes + 16, (size_t)m * skinny::kCols * 4);
        pl.partial_bytes = left > 0 ? align_up((size_t)s * (size_t)m * (size_t)n * 4) : 0;
        pl.keys_bytes = align_up((size_t)m * (size_t)pl.n_cg * 8);
        return pl;
      }
    }
  }
  const Tiling ts = m <= skinny::kMaxM ? staged_tiling(m, n, k, workspace_len) : Tiling{};
  const Tiling td = (!argmax && m <= 16 * skinny::kMaxMR) ? direct_tiling(m, n, k, workspace_len)
                                                                         : Tiling{};
  bool direct = false;
  if (td.cpw > 0) {
    if (m > skinny::kMaxM) direct = td.cpw != 2;
    else if (ts.cpw == 0) direct = true;
    else if (am == gemm::A_SILU_PACKED && m <= 4) direct = false;
    else direct = td.cpw <= 2 || (ts.cpw == td.cpw && ts.s > td.s);
  }
  const Tiling tl = direct ? td : ts;
  const int cpw = tl.cpw, s = tl.s;
  if (cpw > 0) {
    pl.skinny = true;
    pl.direct = direct;
    pl.mr = direct ? (int)((m + 15) / 16) : 1;
    pl.cpw = cpw;
    pl.n_cg = (int)(n / (64 * cpw));
    pl.splits = s;
    const int max_groups = (groups + s - 1) / s;
    pl.x_bytes = direct ? 0 : (size_t)max_groups * 128 * (size_t)m * 2;  // staged A slice (at most kSkinnyMaxX)
    const size_t stage = direct ? 0 : pl.x_bytes + 16;                   // + the zero entry
    // the epilogue's fp32 tile [M][256] (direct plans on wide tiles store per wave)
    const size_t tile = (direct && cpw == skinny::kWaves) ? 0 : (size_t)m * skinny::kCols * 4;
    // A_RING: two batches of [M][128 k] in fragment order + the zero entry
    const size_t ring = (direct && cpw == skinny::kWaves) ? (size_t)(32 * m + 1) * 16 : 0;
    pl.lds = std::max(std::max(stage, tile), ring);
    pl.partial_bytes = pl.splits > 1 ? align_up((size_t)pl.splits * (size_t)m * (size_t)n * 4) : 0;
    if (direct && am == gemm::A_SILU_PACKED) pl.act_bytes = align_up((size_t)m * (size_t)k * 2);
  } else {
    pl.skinny = false;
    // 128-row tiles (two workgroups per CU) where M fills them; the SiLU-gated
    // variant keeps 64-row tiles (its A staging registers leave no room).
    pl.mb = (m >= 128 && am == gemm::A_PLAIN) ? 8 : (m > 32 ? 4 : 2);
    const int64_t bm = 16 * pl.mb;
    pl.n_mb = (int)((m + bm - 1) / bm);
    const int64_t tiles = (int64_t)pl.n_cg * pl.n_mb;
    const int64_t slots = (int64_t)gemm::wgs_per_cu(pl.mb, am) * device_cus();
    int64_t full = (tiles / slots) * slots;
    int64_t tail = tiles - full;
    int s = tail > 0 ? choose_tail_splits(tail, slots, groups, pl.mb) : 1;
    // Few rows: the kernel streams B and is bound by bandwidth, not by the
    // MFMAs the cost model above prices; split further so that every CU gets
    // a workgroup, as long as the fp32 partials (written and read once) stay
    // within half the weight bytes: S <= K / (32 * tile rows).
    if (tail > 0 && m <= 64) {
      const int s_fill = (int)((device_cus() + tail - 1) / tail);
      const int s_cap = (int)std::max<int64_t>(1, k / (32 * bm));
      const int s_mem = std::min(std::min(s_fill, s_cap), groups);
      if (s_mem > s) s = s_mem;
    }
    if (s > 1 && workspace_len < 1 + tail) s = 1;
    // partials are addressed through a 32-bit buffer resource
    while (s > 1 && (size_t)tail * s * 16 * pl.mb * gemm::kThreads * 4 >= ((size_t)1 << 31)) --s;
    if (s == 1) {
      full = tiles;
      tail = 0;
    }
    // Stream-K where 128-row tiles fill between half of one round of the
    // resident slots and all of it: every slot then runs the same number of
    // stages, and a tile is cut only where a workgroup's range ends.  M = 2048,
    // K = 17408, N = 5120 (320 tiles on 512 slots): 310 us against 321 us for
    // 960 third-tiles (1.875 rounds).  With a full round or more the split tail
    // stays ahead (K = 5120, N = 17408, 1088 tiles: 299 us against 323 us);
    // unequal ranges, wave priorities falling with progress and one workgroup
    // per CU were each slower (per-workgroup timestamps: the second workgroup
    // on a CU runs its equal range 15-20 % slower than the first).  Two
    // partial slots per workgroup.
    const size_t sk_bytes = (size_t)2 * slots * 16 * pl.mb * gemm::kThreads * 4;
    if (pl.mb == 8 && tiles < slots && tiles * 2 >= slots && workspace_len >= 1 + tiles &&
        sk_bytes < ((size_t)1 << 31) && (int64_t)groups * tiles < ((int64_t)1 << 31)) {
      pl.sk_wgs = (int)slots;
      pl.full_tiles = 0;
      pl.tail_tiles = (int)tiles;
      pl.tail_splits = 1;
      pl.wgs = slots;
      pl.partial_bytes = align_up(sk_bytes);
      pl.keys_bytes = align_up((size_t)m * (size_t)pl.n_cg * 8);
      return pl;
    }
    pl.full_tiles = (int)full;
    pl.tail_tiles = (int)tail;
    pl.tail_splits = s;
    pl.wgs = full + tail * s;
    pl.partial_bytes = tail > 0 ? align_up((size_t)tail * s * 16 * pl.mb * gemm::kThreads * 4) : 0;
  }
  pl.keys_bytes = align_up((size_t)m * (size_t)pl.n_cg * 8);
  return pl;
}

// Workspace entries a launch uses: [0] the argmax arrival counter, [1 + t]
// the split counters (decode: every column tile; GEMM: every tail tile).
inline int64_t counters_needed(const Plan& pl, bool argmax) {
  // plain stores on wide tiles count per 64-column chunk (see skinny::wave_epilogue)
  if (pl.skinny && pl.splits > 1) return 1 + (int64_t)pl.n_cg * (argmax ? 1 : pl.cpw == skinny::kWaves ? pl.cpw : 1);
  if (!pl.skinny && pl.tail_tiles > 0) return 1 + (int64_t)pl.tail_tiles;  // stream-K: every tile
  return argmax ? 1 : 0;
}

inline int normalize_group(int64_t g, int64_t k, int& grouped) {
  if (g <= 0 || g == k) {
    grouped = 0;
    return LB_OK;
  }
  if (g == 128) {
    grouped = 1;
    return LB_OK;
  }
  return LB_ERR_PROB_SHAPE;
}

int run(Variant var, const uint16_t* a, const int32_t* b, uint16_t* c, const uint16_t* s, int64_t m, int64_t n,
        int64_t k, int32_t* workspace, int64_t workspace_len, int64_t groupsize, int64_t* argmax_state,
        int64_t* argmax_out, void* scratch, size_t scratch_bytes, hipStream_t st) {
  if (m < 0 || n < 0 || k < 0) return LB_ERR_ARG;
  if (n % 256 != 0 || k % 128 != 0) return LB_ERR_PROB_SHAPE;
  int grouped = 0;
  if (normalize_group(groupsize, k, grouped) != LB_OK) return LB_ERR_PROB_SHAPE;
  if (m == 0 || n == 0 || k == 0) return LB_OK;
  if (m > 65535LL * 128 || n > (1LL << 30) || k > (1LL << 30)) return LB_ERR_ARG;
  if (!a || !b || !s) return LB_ERR_ARG;
  if (var == V_ARGMAX ? (!argmax_state || !argmax_out) : !c) return LB_ERR_ARG;
  if (!lbh::aligned(a, 16) || !lbh::aligned(b, 16) || !lbh::aligned(s, 16) || (c && !lbh::aligned(c, 2)))
    return LB_ERR_ALIGN;
  // The GEMM kernel addresses A, B and s through 32-bit buffer resources, the
  // decode kernel B and s with 32-bit offsets.
  const int64_t a_bytes = m * k * 2 * (var == V_SILU ? 2 : 1);
  if (m > skinny::kMaxM && (a_bytes >= (1LL << 31) || k * n / 2 >= (1LL << 31))) return LB_ERR_PROB_SHAPE;
  if (k * n / 2 >= (1LL << 32)) return LB_ERR_PROB_SHAPE;
  const bool gated = var == V_SILU || var == V_SILU_DONE;
  const Plan pl = make_plan(m, n, k, workspace_len, gated ? gemm::A_SILU_PACKED : gemm::A_PLAIN, var == V_ARGMAX,
                            grouped != 0);
  if (var == V_SILU_DONE && !pl.skinny) return LB_ERR_ARG;  // decode batches only
  if (workspace_len < counters_needed(pl, var == V_ARGMAX)) return LB_ERR_WORKSPACE;
  const size_t need = pl.partial_bytes + (var == V_ARGMAX ? pl.keys_bytes : 0) + (var == V_SILU ? pl.act_bytes : 0);
  if (need > 0 && (!scratch || scratch_bytes < need)) return LB_ERR_SCRATCH;
  if (need > 0 && !lbh::aligned(scratch, 16)) return LB_ERR_ALIGN;

  unsigned char* sc = reinterpret_cast<unsigned char*>(scratch);
  float* partial = pl.partial_bytes ? reinterpret_cast<float*>(sc) : nullptr;
  uint64_t* keys = var == V_ARGMAX ? reinterpret_cast<uint64_t*>(sc + pl.partial_bytes) : nullptr;

  if (pl.direct) {
    // A fragments loaded per step; the SiLU-gated A is formed once into
    // scratch first (the staged variant forms it in every tile).
    const uint16_t* av = a;
    if (var == V_SILU) {
      uint16_t* act = reinterpret_cast<uint16_t*>(sc + pl.partial_bytes);
      const int64_t items = m * (k / 8);
      hipLaunchKernelGGL(skinny::silu_pack_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, st, a, act,
                         (int)m, (int)k);
      av = act;
    }
    // (mixed plans: the whole-K tile count rides in the high bits of the split count)
    const int32_t sp = pl.whole > 0 ? (int32_t)((pl.whole << 16) | pl.splits) : pl.splits;
    const dim3 grid = pl.whole > 0 ? dim3((unsigned)(pl.whole + (int64_t)(pl.n_cg - pl.whole) * pl.splits), 1, 1)
                                   : dim3((unsigned)pl.n_cg, (unsigned)pl.splits, 1);
#define LB_SKD(AMV, GV, CV, MRV)                                                                                  \
  hipLaunchKernelGGL((skinny::marlin_skinny_kernel<AMV, skinny::EPI_STORE, GV, CV, MRV>), grid,                  \
                     dim3(skinny::kThreads), pl.lds, st, av, reinterpret_cast<const uint32_t*>(b), s, (int)m, (int)n, \
                     (int)k, sp, partial, workspace, c, nullptr, nullptr, nullptr)
#define LB_SKDG(AMV, CV, MRV)                               \
  do {                                                      \
    if (grouped) LB_SKD(AMV, true, CV, MRV);                \
    else LB_SKD(AMV, false, CV, MRV);                       \
  } while (0)
    if (pl.cpw == 4) {  // 4-chunk tiles: A through the LDS ring
      if (pl.mr == 1) LB_SKDG(skinny::A_RING, 4, 1);
      else LB_SKDG(skinny::A_RING, 4, 2);
    } else if (pl.mr == 1) {
      if (pl.cpw == 2) LB_SKDG(skinny::A_DIRECT, 2, 1);
      else LB_SKDG(skinny::A_DIRECT, 1, 1);
    } else {  // M = 17..32: 64-column tiles (make_plan)
      LB_SKDG(skinny::A_DIRECT, 1, 2);
    }
#undef LB_SKDG
#undef LB_SKD
    return lbh::launch_status();
  }

  if (pl.skinny) {
    skinny::Params p{};
    p.a = a; p.b = reinterpret_cast<const uint32_t*>(b); p.s = s; p.c = c;
    p.counters = workspace; p.partial = partial; p.tile_keys = keys;
    p.argmax_state = argmax_state; p.argmax_out = argmax_out;
    p.m = (int)m; p.n = (int)n; p.k = (int)k; p.splits = pl.splits;
    p.kp_total = (int)(k / 32); p.n_cg = pl.n_cg;
    const dim3 grid = pl.whole > 0 ? dim3((unsigned)(pl.whole + (int64_t)(pl.n_cg - pl.whole) * pl.splits), 1, 1)
                                   : dim3((unsigned)pl.n_cg, (unsigned)pl.splits, 1);
#define LB_SK(AMV, EPV, GV, CV) \
  hipLaunchKernelGGL((skinny::marlin_skinny_kernel<AMV, EPV, GV, CV>), grid, dim3(skinny::kThreads), pl.lds, st, \
                     p.a, p.b, p.s, p.m, p.n, p.k, (pl.whole << 16) | p.splits, p.partial, p.counters, p.c,        \
                     p.tile_keys, p.argmax_state, p.argmax_out)
#define LB_SKC(AMV, EPV, GV)                              \
  do {                                                    \
    if (pl.cpw == 4) LB_SK(AMV, EPV, GV, 4);              \
    else if (pl.cpw == 2) LB_SK(AMV, EPV, GV, 2);         \
    else LB_SK(AMV, EPV, GV, 1);                          \
  } while (0)
#define LB_SKG(AMV, EPV) do { if (grouped) LB_SKC(AMV, EPV, true); else LB_SKC(AMV, EPV, false); } while (0)
    if (var == V_PLAIN) LB_SKG(skinny::A_PLAIN, skinny::EPI_STORE);
    else if (var == V_SILU) LB_SKG(skinny::A_SILU_PACKED, skinny::EPI_STORE);
    else if (var == V_SILU_DONE) LB_SKG(skinny::A_PLAIN, skinny::EPI_STORE);
    else LB_SKG(skinny::A_PLAIN, skinny::EPI_ARGMAX);
#undef LB_SKG
#undef LB_SKC
#undef LB_SK
    return lbh::launch_status();
  }

  gemm::Params p{};
  p.a = a; p.b = reinterpret_cast<const uint32_t*>(b); p.s = s; p.c = c;
  p.counters = workspace; p.partial = partial; p.tile_keys = keys;
  p.argmax_state = argmax_state; p.argmax_out = argmax_out;
  p.m = (int)m; p.n = (int)n; p.k = (int)k; p.grouped = grouped;
  p.full_tiles = pl.full_tiles; p.tail_splits = pl.tail_splits; p.sk_wgs = pl.sk_wgs;
  p.partial_bytes = (uint32_t)pl.partial_bytes;
  p.kp_total = (int)(k / 32); p.n_cg = pl.n_cg; p.n_mb = pl.n_mb;
  dim3 grid((unsigned)pl.wgs, 1, 1);
#define LB_GM_SK(MBV, AMV, EPV, GV, SKV) \
  hipLaunchKernelGGL((gemm::marlin_gemm_kernel<MBV, AMV, EPV, GV, SKV>), grid, dim3(gemm::kThreads), 0, st, p)
#define LB_GM(MBV, AMV, EPV, GV)                                   \
  do {                                                             \
    if constexpr (MBV == 8 && AMV == gemm::A_PLAIN) {              \
      if (pl.sk_wgs > 0) LB_GM_SK(MBV, AMV, EPV, GV, true);        \
      else LB_GM_SK(MBV, AMV, EPV, GV, false);                     \
    } else {                                                       \
      LB_GM_SK(MBV, AMV, EPV, GV, false);                          \
    }                                                              \
  } while (0)
#define LB_GM_G(MBV, AMV, EPV)                      \
  do {                                              \
    if (grouped) LB_GM(MBV, AMV, EPV, true);        \
    else LB_GM(MBV, AMV, EPV, false);               \
  } while (0)
#define LB_GM_MB(AMV, EPV)                      \
  do {                                          \
    if (pl.mb == 8) LB_GM_G(8, AMV, EPV);       \
    else if (pl.mb == 4) LB_GM_G(4, AMV, EPV);  \
    else LB_GM_G(2, AMV, EPV);                  \
  } while (0)
  if (var == V_PLAIN) LB_GM_MB(gemm::A_PLAIN, gemm::EPI_STORE);
  else if (var == V_SILU) {  // 64-row tiles at most (see make_plan)
    if (pl.mb == 4) LB_GM_G(4, gemm::A_SILU_PACKED, gemm::EPI_STORE);
    else LB_GM_G(2, gemm::A_SILU_PACKED, gemm::EPI_STORE);
  }
  else LB_GM_MB(gemm::A_PLAIN, gemm::EPI_ARGMAX);
#undef LB_GM_MB
#undef LB_GM_G
#undef LB_GM
#undef LB_GM_SK
  return lbh::launch_status();
}

}  // namespace marlin
}  // namespace lb

using namespace lb;

extern "C" const char* lb_status_string(int status) {
  switch (status) {
    case LB_OK: return "ok";
    case LB_ERR_PROB_SHAPE: return "problem shape not supported";
    case LB_ERR_KERN_SHAPE: return "no kernel for this shape";
    case LB_ERR_ARG: return "invalid argument";
    case LB_ERR_ALIGN: return "misaligned pointer";
    case LB_ERR_WORKSPACE: return "workspace too small";
    case LB_ERR_SCRATCH: return "scratch too small";
    case LB_ERR_HIP: return "HIP runtime error";
    case LB_ERR_NOALLOC_LIMIT: return "problem needs more than the static no-allocation scratch";
    default: return "unknown status";
  }
}

extern "C" int lb_abi_version(void) { return 1; }

extern "C" size_t lb_marlin_scratch_bytes(int64_t prob_m, int64_t prob_n, int64_t prob_k, int64_t groupsize) {
  (void)groupsize;
  if (prob_m <= 0 || prob_n <= 0 || prob_k <= 0 || prob_n % 256 || prob_k % 128) return 0;
  // Plan with an unconstrained workspace: the largest scratch any plan uses.
  // Largest over the variants (the SiLU-gated one may use other tiles).
  // (with and without the mixed plan, which only grouped scales take)
  const marlin::Plan a = marlin::make_plan(prob_m, prob_n, prob_k, INT64_MAX, gemm::A_PLAIN);
  const marlin::Plan a2 = marlin::make_plan(prob_m, prob_n, prob_k, INT64_MAX, gemm::A_PLAIN, false, false);
  const marlin::Plan b = marlin::make_plan(prob_m, prob_n, prob_k, INT64_MAX, gemm::A_SILU_PACKED);
  const marlin::Plan c = marlin::make_plan(prob_m, prob_n, prob_k, INT64_MAX, gemm::A_PLAIN, true);
  return std::max(std::max(std::max(a.partial_bytes + a.keys_bytes, a2.partial_bytes + a2.keys_bytes),
                           b.partial_bytes + b.keys_bytes + b.act_bytes),
                  c.partial_bytes + c.keys_bytes);
}

extern "C" int lb_marlin_describe_plan(int64_t prob_m, int64_t prob_n, int64_t prob_k, int64_t groupsize,
                                       int32_t variant, int64_t workspace_len, int64_t* out) {
  if (!out || variant < 0 || variant > 2 || prob_m < 0 || prob_n < 0 || prob_k < 0) return LB_ERR_ARG;
  if (prob_n % 256 != 0 || prob_k % 128 != 0) return LB_ERR_PROB_SHAPE;
  int grouped = 0;
  if (marlin::normalize_group(groupsize, prob_k, grouped) != LB_OK) return LB_ERR_PROB_SHAPE;
  for (int i = 0; i < 10; ++i) out[i] = 0;
  if (prob_m == 0 || prob_n == 0 || prob_k == 0) return LB_OK;
  const bool argmax = variant == 2, gated = variant == 1;
  const marlin::Plan pl = marlin::make_plan(prob_m, prob_n, prob_k, workspace_len,
                                            gated ? gemm::A_SILU_PACKED : gemm::A_PLAIN, argmax, grouped != 0);
  if (pl.skinny) {
    out[0] = !pl.direct ? 0 : pl.cpw == skinny::kWaves ? 2 : 1;
    out[1] = pl.cpw;
    out[2] = pl.splits;
    out[3] = pl.mr;
    out[4] = pl.whole > 0 ? pl.whole + (int64_t)(pl.n_cg - pl.whole) * pl.splits : (int64_t)pl.n_cg * pl.splits;
    out[5] = (int64_t)pl.lds;
  } else {
    out[0] = pl.sk_wgs > 0 ? 4 : 3;
    out[1] = pl.mb;
    out[2] = pl.tail_splits;
    out[3] = pl.full_tiles;
    out[4] = pl.wgs;
    out[5] = 0;
  }
  out[6] = (int64_t)(pl.partial_bytes + (argmax ? pl.keys_bytes : 0) + (gated ? pl.act_bytes : 0));
  out[7] = marlin::counters_needed(pl, argmax);
  out[8] = (gated && pl.direct) ? 2 : 1;
  out[9] = marlin::device_cus();
  return LB_OK;
}

extern "C" int lb_marlin_gemm(const uint16_t* A, const int32_t* B, uint16_t* C, const uint16_t* s,
                              int64_t prob_m, int64_t prob_n, int64_t prob_k,
                              int32_t* workspace, int64_t workspace_len, int64_t groupsize,
                              void* scratch, size_t scratch_bytes, lb_stream_t stream) {
  return marlin::run(marlin::V_PLAIN, A, B, C, s, prob_m, prob_n, prob_k, workspace, workspace_len, groupsize,
                     nullptr, nullptr, scratch, scratch_bytes, (hipStream_t)stream);
}

extern "C" int lb_marlin_gemm_silu_packed(const uint16_t* mixed, const int32_t* B, uint16_t* C, const uint16_t* s,
                                          int64_t prob_m, int64_t prob_n, int64_t prob_k,
                                          int32_t* workspace, int64_t workspace_len, int64_t groupsize,
                                          void* scratch, size_t scratch_bytes, lb_stream_t stream) {
  return marlin::run(marlin::V_SILU, mixed, B, C, s, prob_m, prob_n, prob_k, workspace, workspace_len, groupsize,
                     nullptr, nullptr, scratch, scratch_bytes, (hipStream_t)stream);
}

extern "C" int lb_marlin_gemm_argmax(const uint16_t* A, const int32_t* B, const uint16_t* s,
                                     int64_t prob_m, int64_t prob_n, int64_t prob_k,
                                     int32_t* workspace, int64_t workspace_len, int64_t groupsize,
                                     int64_t* argmax_state, int64_t* argmax_out,
                                     int32_t* argmax_sync, int32_t epoch,
                                     void* scratch, size_t scratch_bytes, lb_stream_t stream) {
  (void)argmax_sync;
  if (epoch <= 0) return LB_ERR_ARG;
  return marlin::run(marlin::V_ARGMAX, A, B, nullptr, s, prob_m, prob_n, prob_k, workspace, workspace_len,
                     groupsize, argmax_state, argmax_out, scratch, scratch_bytes, (hipStream_t)stream);
}

extern "C" int lb_marlin_dequant(const int32_t* B, const uint16_t* s, uint16_t* w_nk,
                                 int64_t prob_n, int64_t prob_k, int64_t groupsize, lb_stream_t stream) {
  if (prob_n < 0 || prob_k < 0) return LB_ERR_ARG;
  if (prob_n % 256 || prob_k % 128) return LB_ERR_PROB_SHAPE;
  int grouped = 0;
  if (marlin::normalize_group(groupsize, prob_k, grouped) != LB_OK) return LB_ERR_PROB_SHAPE;
  if (prob_n == 0 || prob_k == 0) return LB_OK;
  if (!B || !s || !w_nk) return LB_ERR_ARG;
  const int64_t total = prob_n * prob_k;
  const int threads = 256;
  hipLaunchKernelGGL(marlin::dequant_kernel, dim3((unsigned)((total + threads - 1) / threads)), dim3(threads), 0,
                     (hipStream_t)stream, reinterpret_cast<const uint32_t*>(B), s, w_nk, prob_n, prob_k, grouped);
  return lbh::launch_status();
}

namespace {
struct MlpPlan {
  int s1, s2;
  size_t gu_bytes, act_bytes, down_bytes;
};
MlpPlan mlp_plan(int64_t batch, int64_t hidden, int64_t inter) {
  MlpPlan p{};
  const int64_t c1 = (2 * inter) / 64, c2 = hidden / 64;
  const int64_t kp1 = hidden / 32, kp2 = inter / 32;
  p.s1 = (int)std::max<int64_t>(1, std::min<int64_t>(kp1, (2048 + c1 - 1) / c1));
  p.s2 = (int)std::max<int64_t>(1, std::min<int64_t>(kp2, (2048 + c2 - 1) / c2));
  p.gu_bytes = marlin::align_up((size_t)p.s1 * batch * 2 * inter * 4);
  p.act_bytes = marlin::align_up((size_t)batch * inter * 4);
  p.down_bytes = marlin::align_up((size_t)p.s2 * batch * hidden * 4);
  return p;
}
}  // namespace

extern "C" size_t lb_marlin_mlp_scratch_bytes(int64_t batch, int64_t hidden, int64_t intermediate) {
  if (batch <= 0 || hidden <= 0 || intermediate <= 0) return 0;
  const MlpPlan p = mlp_plan(batch, hidden, intermediate);
  return p.gu_bytes + p.act_bytes + p.down_bytes;
}

extern "C" int lb_marlin_mlp_streaming(const int32_t* gate_up_qweight, const uint16_t* gate_up_scales,
                                       const int32_t* down_qweight, const uint16_t* down_scales,
                                       const uint16_t* x, uint16_t* out, float* accum, int32_t* sync,
                                       int64_t batch, int64_t hidden, int64_t intermediate,
                                       int64_t gate_group_size, int64_t down_group_size,
                                       void* scratch, size_t scratch_bytes, lb_stream_t stream) {
  (void)accum;
  (void)sync;
  if (batch < 0 || hidden <= 0 || intermediate <= 0) return LB_ERR_ARG;
  // the streaming kernel reads Marlin tiles of 64 output columns and 32-k steps
  if (hidden % 128 || intermediate % 128 || (2 * intermediate) % 256 || hidden % 256) return LB_ERR_PROB_SHAPE;
  int gg = 0, dg = 0;
  if (marlin::normalize_group(gate_group_size, hidden, gg) != LB_OK) return LB_ERR_PROB_SHAPE;
  if (marlin::normalize_group(down_group_size, intermediate, dg) != LB_OK) return LB_ERR_PROB_SHAPE;
  if (batch == 0) return LB_OK;
  if (!gate_up_qweight || !gate_up_scales || !down_qweight || !down_scales || !x || !out) return LB_ERR_ARG;
  if (!lbh::aligned(gate_up_qweight, 16) || !lbh::aligned(down_qweight, 16)) return LB_ERR_ALIGN;
  const MlpPlan pl = mlp_plan(batch, hidden, intermediate);
  if (!scratch || scratch_bytes < pl.gu_bytes + pl.act_bytes + pl.down_bytes) return LB_ERR_SCRATCH;
  hipStream_t st = (hipStream_t)stream;
  unsigned char* sc = reinterpret_cast<unsigned char*>(scratch);
  float* gu = reinterpret_cast<float*>(sc);
  float* act = reinterpret_cast<float*>(sc + pl.gu_bytes);
  float* dp = reinterpret_cast<float*>(sc + pl.gu_bytes + pl.act_bytes);
  const unsigned zb = (unsigned)((batch + marlin::kF32Batch - 1) / marlin::kF32Batch);
  hipLaunchKernelGGL((marlin::f32_gemv_kernel<false>), dim3((unsigned)(2 * intermediate / 64), pl.s1, zb), dim3(64), 0, st,
                     reinterpret_cast<const uint32_t*>(gate_up_qweight), gate_up_scales, (const void*)x, gu, (int)batch,
                     2 * intermediate, hidden, gg, pl.s1);
  const int64_t na = batch * intermediate;
  hipLaunchKernelGGL(marlin::mlp_act_kernel, dim3((unsigned)((na + 255) / 256)), dim3(256), 0, st, gu, act, (int)batch,
                     intermediate, pl.s1);
  hipLaunchKernelGGL((marlin::f32_gemv_kernel<true>), dim3((unsigned)(hidden / 64), pl.s2, zb), dim3(64), 0, st,
                     reinterpret_cast<const uint32_t*>(down_qweight), down_scales, (const void*)act, dp, (int)batch,
                     hidden, intermediate, dg, pl.s2);
  const int64_t no = batch * hidden;
  hipLaunchKernelGGL(marlin::f32_finalize_kernel, dim3((unsigned)((no + 255) / 256)), dim3(256), 0, st, dp, out, no,
                     pl.s2);
  return lbh::launch_status();
}

// ---------------------------------------------------------------------------
// Decode MLP: gate_up, then down over fp16(silu(g) * u) (marlin_mlp.hpp)
// ---------------------------------------------------------------------------
namespace {
struct FusedMlpPlan {
  marlin::Plan up, down;  // the tilings lb_marlin_gemm plans for the two projections
  bool act_path = false;  // gate_up stores fp16(silu(g) * u), no [g | u] round trip
  size_t partial = 0;     // scratch: [g | u] or the activations first, then either launch's own scratch
  size_t scratch = 0;
  int64_t ws_down = 0, ws_len = 0;  // workspace: the gate_up launch's counters, then the down launch's
};

// Counters a launch of `pl` may use (planned with an unbounded workspace).
int64_t fused_counters(const marlin::Plan& pl) {
  return std::max<int64_t>(1 + std::max<int64_t>(pl.n_cg, pl.tail_tiles), marlin::counters_needed(pl, false));
}

FusedMlpPlan fused_mlp_plan(int64_t batch, int64_t hidden, int64_t inter, bool g1, bool g2) {
  FusedMlpPlan p;
  // as run() plans each projection (the mixed decode plan only with grouped
  // scales), except that from M = 5 the gate/up launch keeps the 2- or 4-chunk
  // tiles that can pair gate and up chunks (its SiLU-gated store saves the
  // down launch's separate gating pass)
  p.up = marlin::make_plan(batch, 2 * inter, hidden, INT64_MAX, gemm::A_PLAIN, false,
                           g1 && batch <= marlin::kMixedMaxM);
  p.down = marlin::make_plan(batch, hidden, inter, INT64_MAX, gemm::A_SILU_PACKED, false, g2);
  // decode tiles of 2 or 4 chunks pair gate and up chunks; single-chunk tiles
  // and prefill tiles take the [g | u] round trip
  p.act_path = p.up.skinny && p.up.cpw >= 2 && p.down.skinny;
  p.partial = marlin::align_up((size_t)batch * (size_t)(2 * inter) * 2);
  p.scratch = p.partial + std::max(lb_marlin_scratch_bytes(batch, 2 * inter, hidden, g1 ? 128 : -1),
                                   lb_marlin_scratch_bytes(batch, hidden, inter, g2 ? 128 : -1));
  p.ws_down = fused_counters(p.up);
  p.ws_len = p.ws_down + fused_counters(p.down);
  return p;
}

int fused_mlp_check(int64_t batch, int64_t hidden, int64_t inter, int64_t gate_group, int64_t down_group, int& g1,
                    int& g2) {
  if (batch < 0 || hidden <= 0 || inter <= 0) return LB_ERR_ARG;
  if (hidden % 256 || inter % 128) return LB_ERR_PROB_SHAPE;
  if (batch > 65535LL * 128 || hidden > (1LL << 30) || inter > (1LL << 29)) return LB_ERR_ARG;
  if (marlin::normalize_group(gate_group, hidden, g1) != LB_OK) return LB_ERR_PROB_SHAPE;
  if (marlin::normalize_group(down_group, inter, g2) != LB_OK) return LB_ERR_PROB_SHAPE;
  return LB_OK;
}
}  // namespace

// Sizes cover grouped and per-column scales alike.
extern "C" size_t lb_marlin_mlp_fused_scratch_bytes(int64_t batch, int64_t hidden, int64_t intermediate) {
  int g1 = 0, g2 = 0;
  if (batch <= 0 || fused_mlp_check(batch, hidden, intermediate, 128, 128, g1, g2) != LB_OK) return 0;
  return std::max(fused_mlp_plan(batch, hidden, intermediate, true, true).scratch,
                  fused_mlp_plan(batch, hidden, intermediate, false, false).scratch);
}

extern "C" int64_t lb_marlin_mlp_fused_workspace_len(int64_t batch, int64_t hidden, int64_t intermediate) {
  int g1 = 0, g2 = 0;
  if (batch <= 0 || fused_mlp_check(batch, hidden, intermediate, 128, 128, g1, g2) != LB_OK) return 0;
  return std::max(fused_mlp_plan(batch, hidden, intermediate, true, true).ws_len,
                  fused_mlp_plan(batch, hidden, intermediate, false, false).ws_len);
}

extern "C" int lb_marlin_mlp_fused(const uint16_t* x, const int32_t* gate_up_qweight, const uint16_t* gate_up_scales,
                                   const int32_t* down_qweight, const uint16_t* down_scales, uint16_t* out,
                                   int64_t batch, int64_t hidden, int64_t intermediate, int64_t gate_group_size,
                                   int64_t down_group_size, int32_t* workspace, int64_t workspace_len,
                                   void* scratch, size_t scratch_bytes, lb_stream_t stream) {
  int g1 = 0, g2 = 0;
  const int st0 = fused_mlp_check(batch, hidden, intermediate, gate_group_size, down_group_size, g1, g2);
  if (st0 != LB_OK) return st0;
  if (batch == 0) return LB_OK;
  if (!x || !gate_up_qweight || !gate_up_scales || !down_qweight || !down_scales || !out || !workspace)
    return LB_ERR_ARG;
  if (!lbh::aligned(x, 16) || !lbh::aligned(gate_up_qweight, 16) || !lbh::aligned(gate_up_scales, 16) ||
      !lbh::aligned(down_qweight, 16) || !lbh::aligned(down_scales, 16) || !lbh::aligned(out, 2))
    return LB_ERR_ALIGN;
  const FusedMlpPlan pl = fused_mlp_plan(batch, hidden, intermediate, g1 != 0, g2 != 0);
  if (workspace_len < pl.ws_len) return LB_ERR_WORKSPACE;
  if (!scratch || scratch_bytes < pl.scratch) return LB_ERR_SCRATCH;
  if (!lbh::aligned(scratch, 256)) return LB_ERR_ALIGN;
  unsigned char* sc = reinterpret_cast<unsigned char*>(scratch);
  hipStream_t st = (hipStream_t)stream;
  const int64_t n_up = 2 * intermediate;
  const size_t rest = scratch_bytes - pl.partial;

  if (pl.act_path) {
    // gate_up -> fp16(silu(g) * u) [batch][intermediate] (at the start of
    // scratch), then the down projection over it with the SiLU-gated op's own
    // plan: the same sums as the two reference calls
    uint16_t* act = reinterpret_cast<uint16_t*>(sc);
    const marlin::Plan& u2 = pl.up;
    skinny::Params u{};
    u.a = x; u.b = reinterpret_cast<const uint32_t*>(gate_up_qweight); u.s = gate_up_scales; u.c = nullptr;
    u.counters = workspace;
    u.partial = u2.partial_bytes ? reinterpret_cast<float*>(sc + pl.partial) : nullptr;
    u.m = (int)batch; u.n = (int)n_up; u.k = (int)hidden; u.splits = u2.splits;
    u.kp_total = (int)(hidden / 32); u.n_cg = u2.n_cg;
    u.act_out = reinterpret_cast<uint32_t*>(act);
    u.gate_chunks = (int)(intermediate / 64);
    const size_t lds = std::max(u2.lds, (size_t)batch * skinny::kCols * 4);
    dim3 grid((unsigned)u2.n_cg, (unsigned)u2.splits, 1);
#define LB_ACT(AMV, GV, CV, MRV) \
  hipLaunchKernelGGL((mlp::mlp_gate_up_act_kernel<AMV, GV, CV, MRV>), grid, dim3(skinny::kThreads), lds, st, u.a, u.b, \
                     u.s, u.m, u.n, u.k, u.splits, u.partial, u.counters, u.act_out)
#define LB_ACTG(AMV, CV, MRV)                   \
  do {                                          \
    if (g1) LB_ACT(AMV, true, CV, MRV);         \
    else LB_ACT(AMV, false, CV, MRV);           \
  } while (0)
    if (!u2.direct) {  // staged (M <= 16)
      if (u2.cpw == 4) LB_ACTG(skinny::A_PLAIN, 4, 1);
      else LB_ACTG(skinny::A_PLAIN, 2, 1);
    } else if (u2.cpw == 4) {  // the LDS ring
      if (u2.mr == 1) LB_ACTG(skinny::A_RING, 4, 1);
      else LB_ACTG(skinny::A_RING, 4, 2);
    } else {  // direct A, 2-chunk tiles (M <= 16)
      LB_ACTG(skinny::A_DIRECT, 2, 1);
    }
#undef LB_ACTG
#undef LB_ACT
    const int e = lbh::launch_status();
    if (e != LB_OK) return e;
    return marlin::run(marlin::V_SILU_DONE, act, down_qweight, out, down_scales, batch, hidden, intermediate,
                       workspace + pl.ws_down, workspace_len - pl.ws_down, down_group_size, nullptr, nullptr,
                       sc + pl.partial, rest, st);
  }

  uint16_t* mixed = reinterpret_cast<uint16_t*>(sc);
  int e = marlin::run(marlin::V_PLAIN, x, gate_up_qweight, mixed, gate_up_scales, batch, n_up, hidden, workspace,
                      pl.ws_down, gate_group_size, nullptr, nullptr, sc + pl.partial, rest, st);
  if (e != LB_OK) return e;
  return marlin::run(marlin::V_SILU, mixed, down_qweight, out, down_scales, batch, hidden, intermediate,
                     workspace + pl.ws_down, workspace_len - pl.ws_down, down_group_size, nullptr, nullptr,
                     sc + pl.partial, rest, st);
}
