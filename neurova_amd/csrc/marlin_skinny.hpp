// Marlin-layout W4A16 projection for skinny batches (decode: M <= 16 per
// 16-row block) on gfx950.
//
// Reads the reference's Marlin layout (langburst/csrc/marlin_cuda_kernel.cu,
// packing in adapters/qwen36_tools/quantize.py:180-243) directly; no repack.
//
// Layout facts used (derived from quantize.py:50-76):
//   qweight int32 [K/16, 2N].  Row kb holds k = 16kb..16kb+15.  Each 64-column
//   "chunk" of a row is 128 int32 = 512 contiguous bytes = 32 16-byte slots.
//   Slot i (0..31), with c = i>>2 and q = i&3, holds 4 words j = 0..3; word j
//   covers columns 16j+c (nibbles 0,1,4,5) and 16j+c+8 (nibbles 2,3,6,7) of
//   the chunk at k-offsets {2q, 2q+8, 2q+1, 2q+9} (low nibble of bytes 0/2 =
//   k 2q/2q+1, high nibble = k 2q+8/2q+9; bytes 1/3 the same for column +8).
//   Group scales: 64-column chunk of row g stores column 8jj+i at 8i+jj, so
//   the 8 scales a slot needs are the 16 bytes at 8c.
//
// Kernel structure.  A workgroup owns 4 chunks (256 columns) and a range of
// k; wave w streams chunk w.  Per 32-k step a wave loads 1 KB of qweight with
// fully coalesced 16-byte loads (rows kb and kb+1), bounces it through a
// wave-private 1 KB LDS slot, and each lane reads the two adjacent slots its
// MFMA B fragment needs.  The fragment of v_mfma_f32_16x16x32_f16 (lane
// l = 16g + nl holds 8 k-values of column nl) is built in registers:
// k-group g = (row p = g>>1, slot pair q = 2(g&1), 2(g&1)+1), column
// nl = 8h + c, so its 8 halves are (q0 k0,k1)(q1 k0,k1)(q0 k8,k9)(q1 k8,k9)
// = physical k 4g'+{0,1,2,3} and 4g'+8+{0,1,2,3} of row p -- two contiguous
// 8-byte runs of the activation row, which is staged in LDS as
// [k/4][m][4 halves].  Dequant is the exact fp16 (q-8), then one fp16 multiply
// by the group scale: the same rounding as the reference's __hmul2.
//
// Split-K.  When the k range is split over S workgroups, each writes fp32
// partials to scratch [S][M][N]; the last workgroup to arrive on the
// column-group counter (workspace, zero on entry) sums them in split order
// (deterministic), writes the fp16 result and re-zeroes the counter.

#pragma once
#include "lb_common.hpp"

namespace lb {
namespace skinny {

constexpr int kWaves = 4;               // chunks (64 columns each) per workgroup
constexpr int kThreads = kWaves * kWave;
constexpr int kColsPerWG = 64 * kWaves;  // 256
constexpr int kMaxM = 16;                // rows per m-block (MFMA tile height)
constexpr int kPrefetch = 4;             // 1 KB steps in flight per batch (x2 double buffer)

enum AMode { A_PLAIN = 0, A_SILU_PACKED = 1 };
enum EpiMode { EPI_STORE = 0, EPI_ARGMAX = 1 };

struct Params {
  const uint16_t* a;     // x [M, K] (A_PLAIN) or mixed [M, 2K] (A_SILU_PACKED)
  const uint32_t* b;     // qweight [K/16, 2N]
  const uint16_t* s;     // scales
  uint16_t* c;           // out [M, N] (EPI_STORE)
  int32_t* counters;     // workspace: [0] argmax arrival counter, [1 + tile] split-K counters
  float* partial;        // scratch: [S][M][N] fp32 partials (S > 1)
  uint64_t* tile_keys;   // scratch: [M][n_cg] argmax keys (EPI_ARGMAX)
  int64_t* argmax_state; // [M]
  int64_t* argmax_out;   // [M]
  int m, n, k;
  int grouped;           // 1: group size 128, 0: one scale per column
  int splits;            // S
  int kp_total;          // K / 32
  int n_cg;              // N / 256
};

__device__ __forceinline__ float silu(float v) { return v / (1.0f + __expf(-v)); }

// Order-preserving key: larger value wins, then smaller column.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t col) {
  const uint32_t bits = __builtin_bit_cast(uint32_t, v);
  const uint32_t ord = (bits & 0x80000000u) ? ~bits : (bits ^ 0x80000000u);
  return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - col);
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  const int lane = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_bpermute(((lane ^ off) & 63) << 2, (int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_bpermute(((lane ^ off) & 63) << 2, (int)(uint32_t)(v >> 32));
    v = max_u64(v, ((uint64_t)hi << 32) | lo);
  }
  return v;
}

// Splits are whole scale groups (4 k-steps of 32) balanced over S.
__device__ __forceinline__ void split_range(const Params& p, int split, int& kp0, int& kp1) {
  const int groups = p.kp_total >> 2;
  const int g0 = (int)(((int64_t)groups * split) / p.splits);
  const int g1 = (int)(((int64_t)groups * (split + 1)) / p.splits);
  kp0 = g0 << 2;
  kp1 = g1 << 2;
}

template <int AM, int EPI>
__global__ __launch_bounds__(kThreads) void marlin_skinny_kernel(Params p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int cg = blockIdx.x;      // column group (256 columns)
  const int split = blockIdx.y;
  const int mb = blockIdx.z;      // 16-row block of A
  const int m0 = mb * kMaxM;
  const int mrows = min(kMaxM, p.m - m0);

  int kp0, kp1;
  split_range(p, split, kp0, kp1);
  const int nkp = kp1 - kp0;
  const int k0 = kp0 * 32;
  const int kr = nkp * 32;

  // ---- stage A rows [m0, m0+mrows) x [k0, k0+kr) as xs[k/4][m][4 halves] ----
  uint2* xs = reinterpret_cast<uint2*>(smem);
  uint4* bstage = reinterpret_cast<uint4*>(smem + (size_t)kr * mrows * 2);  // kWaves x 64 x 16 B
  {
    const int quads = kr >> 2;
    const int items = quads * mrows;
    for (int it = tid; it < items; it += kThreads) {
      const int mm = it / quads;
      const int kq = it - mm * quads;
      const int kk = k0 + (kq << 2);
      uint2 v;
      if (AM == A_PLAIN) {
        v = *reinterpret_cast<const uint2*>(p.a + (int64_t)(m0 + mm) * p.k + kk);
      } else {
        const uint16_t* row = p.a + (int64_t)(m0 + mm) * (2 * (int64_t)p.k);
        const uint2 g = *reinterpret_cast<const uint2*>(row + kk);
        const uint2 u = *reinterpret_cast<const uint2*>(row + p.k + kk);
        const uint32_t gw[2] = {g.x, g.y};
        const uint32_t uw[2] = {u.x, u.y};
        uint32_t ow[2];
#pragma unroll
        for (int w = 0; w < 2; ++w) {
          const float g0 = h2f((uint16_t)(gw[w] & 0xffffu)), g1 = h2f((uint16_t)(gw[w] >> 16));
          const float u0 = h2f((uint16_t)(uw[w] & 0xffffu)), u1 = h2f((uint16_t)(uw[w] >> 16));
          ow[w] = (uint32_t)f2h(silu(g0) * u0) | ((uint32_t)f2h(silu(g1) * u1) << 16);
        }
        v = make_uint2(ow[0], ow[1]);
      }
      xs[kq * mrows + mm] = v;
    }
  }
  __syncthreads();

  // ---- per-wave stream over one 64-column chunk ----
  const int chunk = cg * kWaves + wave;
  const int64_t row_words = 2 * (int64_t)p.n;  // int32 per qweight row
  // coalesced load: lane L takes slot (L & 31) of row 2*kp + (L >> 5)
  const uint32_t* bsrc = p.b + (int64_t)(lane >> 5) * row_words + (int64_t)chunk * 128 + (lane & 31) * 4;
  uint4* my_stage = bstage + wave * 64;

  // fragment coordinates: lane = 16g + 8h + c
  const int g = lane >> 4;
  const int hsel = (lane >> 3) & 1;
  const int cc = lane & 7;
  const int prow = g >> 1;     // which of the two k16 rows
  const int gq = g & 1;        // slot pair (q0, q1) = (2gq, 2gq+1)
  const int slot0 = prow * 32 + cc * 4 + gq * 2;
  const int mrow = lane & 15;  // A fragment row
  const bool a_live = mrow < mrows;

  f32x4 acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  f16x2 sc[4];  // per-tile scale (s, s) for this lane's column
#pragma unroll
  for (int j = 0; j < 4; ++j) sc[j] = (f16x2){(f16)1.0f, (f16)1.0f};

  // Software pipeline: a batch is one scale group (4 k-steps of 32, 4 KB per
  // wave); batch b+1 is in flight while batch b is consumed.
  u32x4 bufA[kPrefetch], bufB[kPrefetch];
  u32x4 sclA = (u32x4){0, 0, 0, 0}, sclB = (u32x4){0, 0, 0, 0};
  const uint16_t* ssrc = p.s + chunk * 64 + cc * 8;
  auto issue = [&](u32x4(&bf)[kPrefetch], u32x4& scl, int kp_first) {
    if (kp_first < kp1) {
#pragma unroll
      for (int d = 0; d < kPrefetch; ++d)
        bf[d] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(bsrc + (int64_t)(kp_first + d) * 2 * row_words));
      if (p.grouped) scl = *reinterpret_cast<const u32x4*>(ssrc + (int64_t)(kp_first >> 2) * p.n);
    }
  };
  auto consume = [&](const u32x4(&bf)[kPrefetch], const u32x4& scl, int kp_first) {
    if (p.grouped) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t w = scl[j];
        const uint32_t h = hsel ? (w >> 16) : (w & 0xffffu);
        sc[j] = as_h2(h | (h << 16));
      }
    }
#pragma unroll
    for (int d = 0; d < kPrefetch; ++d) {
      const int kp = kp_first + d;
      // bounce the coalesced 1 KB through this wave's LDS slot
      *reinterpret_cast<u32x4*>(&my_stage[lane]) = bf[d];
      __builtin_amdgcn_wave_barrier();
      const u32x4 w0 = *reinterpret_cast<const u32x4*>(&my_stage[slot0]);
      const u32x4 w1 = *reinterpret_cast<const u32x4*>(&my_stage[slot0 + 1]);
      // A fragment: x rows at k = 32kp + 16prow + 4gq + {0..3} and +8
      f16x8 afrag = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
      if (a_live) {
        const int kq = ((kp - kp0) << 3) + (prow << 2) + gq;
        const uint2 lo = xs[kq * mrows + mrow];
        const uint2 hi = xs[(kq + 2) * mrows + mrow];
        afrag = __builtin_bit_cast(f16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
      }
      const int sh = hsel * 8;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t v0 = w0[j] >> sh;
        const uint32_t v1 = w1[j] >> sh;
        f16x2 b0 = nib_lo_to_h2(v0);
        f16x2 b1 = nib_lo_to_h2(v1);
        f16x2 b2 = nib_hi_to_h2(v0);
        f16x2 b3 = nib_hi_to_h2(v1);
        if (p.grouped) {
          b0 *= sc[j];
          b1 *= sc[j];
          b2 *= sc[j];
          b3 *= sc[j];
        }
        const f16x8 bfrag = __builtin_bit_cast(f16x8, make_uint4(as_u32(b0), as_u32(b1), as_u32(b2), as_u32(b3)));
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(afrag, bfrag, acc[j], 0, 0, 0);
      }
      __builtin_amdgcn_wave_barrier();
    }
  };

  // kp0 and kp1 are multiples of kPrefetch (splits are whole groups)
  issue(bufA, sclA, kp0);
  for (int kpb = kp0; kpb < kp1; kpb += 2 * kPrefetch) {
    issue(bufB, sclB, kpb + kPrefetch);
    consume(bufA, sclA, kpb);
    if (kpb + kPrefetch >= kp1) break;
    issue(bufA, sclA, kpb + 2 * kPrefetch);
    consume(bufB, sclB, kpb + kPrefetch);
  }

  // ---- epilogue ----
  // acc[j][i] = C[m0 + 4*(lane>>4) + i][chunk*64 + 16j + (lane & 15)]
  const int crow0 = (lane >> 4) * 4;
  const int ccol = chunk * 64 + (lane & 15);
  __shared__ int s_prev;
  __shared__ uint64_t s_keys[kWaves][kMaxM];

  float final_v[4][4];
  bool have_final = false;

  if (p.splits > 1) {
    float* part = p.partial + ((int64_t)split * p.m) * p.n;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = crow0 + i;
        if (r < mrows) part[(int64_t)(m0 + r) * p.n + ccol + 16 * j] = acc[j][i];
      }
    __syncthreads();
    if (tid == 0) s_prev = arrive_release(p.counters + 1 + cg + mb * p.n_cg);
    __syncthreads();
    if (s_prev != p.splits - 1) return;  // not the last split of this tile
    acquire_device();
    // the last workgroup sums the partials in split order
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = crow0 + i;
        float sum = 0.f;
        if (r < mrows) {
          for (int sp = 0; sp < p.splits; ++sp)
            sum += __builtin_nontemporal_load(p.partial + ((int64_t)sp * p.m + m0 + r) * p.n + ccol + 16 * j);
        }
        final_v[j][i] = sum;
      }
    if (tid == 0) __hip_atomic_store(p.counters + 1 + cg + mb * p.n_cg, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    have_final = true;
  }
  if (!have_final) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) final_v[j][i] = acc[j][i];
  }

  // fp16 rounding (and the per-column scale after it, as the reference does)
  uint16_t outh[4][4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float colscale = 1.0f;
    if (!p.grouped) {
      const int n = ccol + 16 * j;
      const int base = n & ~31, r = n & 31;
      const int t = 8 * ((r >> 1) & 3) + ((r >> 3) << 1) + (r & 1);  // inverse of the per-column perm
      colscale = h2f(p.s[base + t]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f16 h = (f16)final_v[j][i];
      if (!p.grouped) h = h * (f16)colscale;
      outh[j][i] = __builtin_bit_cast(uint16_t, h);
    }
  }

  if (EPI == EPI_STORE) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = crow0 + i;
        if (r < mrows) p.c[(int64_t)(m0 + r) * p.n + ccol + 16 * j] = outh[j][i];
      }
    return;
  }

  // ---- argmax epilogue: per-row max key over this tile, then over tiles ----
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // rows crow0+i live in lanes with the same lane>>4; reduce over j and lane&15
    uint64_t best = 0;
    const int r = crow0 + i;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (r < mrows) best = max_u64(best, argmax_key(h2f(outh[j][i]), (uint32_t)(ccol + 16 * j)));
    }
    // reduce across the 16 lanes sharing r (xor 1,2,4,8)
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
      const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_bpermute(((lane ^ off) & 63) << 2, (int)(uint32_t)best);
      const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_bpermute(((lane ^ off) & 63) << 2, (int)(uint32_t)(best >> 32));
      best = max_u64(best, ((uint64_t)hi << 32) | lo);
    }
    if ((lane & 15) == 0 && r < kMaxM) s_keys[wave][r] = best;
  }
  __syncthreads();
  if (tid < mrows) {
    uint64_t best = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) best = max_u64(best, s_keys[w][tid]);
    p.tile_keys[(int64_t)(m0 + tid) * p.n_cg + cg] = best;
  }
  __syncthreads();
  int32_t* final_counter = p.counters;
  if (tid == 0) s_prev = arrive_release(final_counter);
  __syncthreads();
  const int total = p.n_cg * ((p.m + kMaxM - 1) / kMaxM);
  if (s_prev != total - 1) return;
  acquire_device();
  for (int r = wave; r < p.m; r += kWaves) {
    uint64_t best = 0;
    for (int t = lane; t < p.n_cg; t += kWave)
      best = max_u64(best, __builtin_nontemporal_load(p.tile_keys + (int64_t)r * p.n_cg + t));
    best = wave_max_u64(best);
    if (lane == 0) {
      p.argmax_state[r] = (int64_t)best;
      p.argmax_out[r] = (int64_t)(0xffffffffu - (uint32_t)(best & 0xffffffffu));
    }
  }
  if (tid == 0) __hip_atomic_store(final_counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace skinny
}  // namespace lb
