// Marlin-layout W4A16 GEMM for prefill batches (M > 16) on gfx950.
//
// Same fragment construction as the decode kernel (lb_marlin_skinny.hip):
// B fragments of v_mfma_f32_16x16x32_f16 are built in registers from the
// reference's Marlin layout (langburst/csrc/marlin_cuda_kernel.cu; packing in
// adapters/qwen36_tools/quantize.py:180-243), exact fp16 (q-8) times the fp16
// group scale.  Here each dequantised B fragment feeds MB MFMAs (MB 16-row
// blocks of A), so the VALU dequant cost is amortised over 16*MB rows.
//
// Workgroup tile: (16*MB rows) x 256 columns; wave w owns 64-column chunk w.
// Per 32-k step:
//   A  -- global rows (64 B each) -> registers -> LDS, rearranged so that the
//         A fragment of lane (g, m) is 16 contiguous bytes: frag[g][m] =
//         x[m][16p + 4g' + {0..3}] ++ x[m][16p + 4g' + 8 + {0..3}], g = 2p+g'.
//         Double-buffered, one __syncthreads per step.
//   B  -- each lane loads the two adjacent 16-byte slots its fragment needs
//         (slots 4c+2g', 4c+2g'+1 of row p) straight from global memory.
// Optional split-K over S workgroups with the same deterministic fixup as the
// decode kernel (fp32 partials in scratch, last arrival sums in split order).

#pragma once
#include "lb_common.hpp"

namespace lb {
namespace gemm {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWave;

enum AMode { A_PLAIN = 0, A_SILU_PACKED = 1 };
enum EpiMode { EPI_STORE = 0, EPI_ARGMAX = 1 };

struct Params {
  const uint16_t* a;
  const uint32_t* b;
  const uint16_t* s;
  uint16_t* c;
  int32_t* counters;     // [0] argmax arrival counter, [1 + tile] split-K counters
  float* partial;        // [S][M][N]
  uint64_t* tile_keys;   // [M][n_cg]
  int64_t* argmax_state;
  int64_t* argmax_out;
  int m, n, k;
  int grouped;
  int splits;
  int kp_total;
  int n_cg;
  int n_mb;
};

__device__ __forceinline__ float silu(float v) { return v / (1.0f + __expf(-v)); }

__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t col) {
  const uint32_t bits = __builtin_bit_cast(uint32_t, v);
  const uint32_t ord = (bits & 0x80000000u) ? ~bits : (bits ^ 0x80000000u);
  return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - col);
}
__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int lane, int off) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_bpermute(((lane ^ off) & 63) << 2, (int)(uint32_t)v);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_bpermute(((lane ^ off) & 63) << 2, (int)(uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ void split_range(const Params& p, int split, int& kp0, int& kp1) {
  const int groups = p.kp_total >> 2;
  const int g0 = (int)(((int64_t)groups * split) / p.splits);
  const int g1 = (int)(((int64_t)groups * (split + 1)) / p.splits);
  kp0 = g0 << 2;
  kp1 = g1 << 2;
}

// Loads the 32 halves (64 B) of A row `r`, k-step kp, half p (k 16p..16p+15)
// and returns the two fragment quads (g = 2p, g = 2p+1) as 2 x 16 bytes.
template <int AM>
__device__ __forceinline__ void load_a_half(const Params& p, int r, int kp, int ph, uint4& f0, uint4& f1) {
  if (r >= p.m) {
    f0 = make_uint4(0, 0, 0, 0);
    f1 = make_uint4(0, 0, 0, 0);
    return;
  }
  const int kk = kp * 32 + ph * 16;
  uint4 v0, v1;  // k kk..kk+7, kk+8..kk+15
  if (AM == A_PLAIN) {
    const uint4* src = reinterpret_cast<const uint4*>(p.a + (int64_t)r * p.k + kk);
    v0 = src[0];
    v1 = src[1];
  } else {
    const uint16_t* row = p.a + (int64_t)r * (2 * (int64_t)p.k);
    const uint4* gs = reinterpret_cast<const uint4*>(row + kk);
    const uint4* us = reinterpret_cast<const uint4*>(row + p.k + kk);
    uint4 gv[2] = {gs[0], gs[1]};
    uint4 uv[2] = {us[0], us[1]};
    uint4 ov[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint32_t gw[4] = {gv[t].x, gv[t].y, gv[t].z, gv[t].w};
      const uint32_t uw[4] = {uv[t].x, uv[t].y, uv[t].z, uv[t].w};
      uint32_t o[4];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float g0 = h2f((uint16_t)(gw[w] & 0xffffu)), g1 = h2f((uint16_t)(gw[w] >> 16));
        const float u0 = h2f((uint16_t)(uw[w] & 0xffffu)), u1 = h2f((uint16_t)(uw[w] >> 16));
        o[w] = (uint32_t)f2h(silu(g0) * u0) | ((uint32_t)f2h(silu(g1) * u1) << 16);
      }
      ov[t] = make_uint4(o[0], o[1], o[2], o[3]);
    }
    v0 = ov[0];
    v1 = ov[1];
  }
  // quads: v0 = (q0, q1), v1 = (q2, q3) where quad qd = k kk+4qd..+3
  // fragment g=2p   : quads 0 and 2 ; fragment g=2p+1 : quads 1 and 3
  f0 = make_uint4(v0.x, v0.y, v1.x, v1.y);
  f1 = make_uint4(v0.z, v0.w, v1.z, v1.w);
}

template <int MB, int AM, int EPI>
__global__ __launch_bounds__(kThreads) void marlin_gemm_kernel(Params p) {
  constexpr int BM = 16 * MB;
  // A fragments: [2 buffers][4 g][BM rows] x 16 B
  __shared__ __attribute__((aligned(16))) uint4 afr[2][4][BM];
  __shared__ int s_prev;
  __shared__ uint64_t s_keys[kWaves][BM];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int cg = blockIdx.x;
  const int split = blockIdx.y;
  const int mb = blockIdx.z;
  const int m0 = mb * BM;

  int kp0, kp1;
  split_range(p, split, kp0, kp1);

  const int chunk = cg * kWaves + wave;
  const int64_t row_words = 2 * (int64_t)p.n;
  const int g = lane >> 4;
  const int hsel = (lane >> 3) & 1;
  const int cc = lane & 7;
  const int prow = g >> 1;
  const int gq = g & 1;
  // B fragment source: slots 4cc + 2gq and +1 of row 2kp + prow of this chunk
  const uint32_t* bsrc = p.b + (int64_t)prow * row_words + (int64_t)chunk * 128 + (cc * 4 + gq * 2) * 4;
  const uint16_t* ssrc = p.s + chunk * 64 + cc * 8;
  const NibConsts nk = nib_consts();

  // A staging assignment: (row, half) pairs, BM*2 of them over 256 threads
  constexpr int kAItems = BM * 2;
  constexpr int kAPerThread = (kAItems + kThreads - 1) / kThreads;

  f32x4 acc[4][MB];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[j][i] = (f32x4){0.f, 0.f, 0.f, 0.f};
  f16x2 sc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) sc[j] = (f16x2){(f16)1.0f, (f16)1.0f};

  uint4 areg[kAPerThread][2];
  auto load_a = [&](int kp) {
#pragma unroll
    for (int t = 0; t < kAPerThread; ++t) {
      const int item = tid + t * kThreads;
      if (item < kAItems) load_a_half<AM>(p, m0 + (item >> 1), kp, item & 1, areg[t][0], areg[t][1]);
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int t = 0; t < kAPerThread; ++t) {
      const int item = tid + t * kThreads;
      if (item < kAItems) {
        const int r = item >> 1, ph = item & 1;
        afr[buf][2 * ph][r] = areg[t][0];
        afr[buf][2 * ph + 1][r] = areg[t][1];
      }
    }
  };

  u32x4 bcur0, bcur1, bnext0, bnext1;
  auto load_b = [&](int kp, u32x4& b0, u32x4& b1) {
    const u32x4* src = reinterpret_cast<const u32x4*>(bsrc + (int64_t)kp * 2 * row_words);
    b0 = __builtin_nontemporal_load(src);
    b1 = __builtin_nontemporal_load(src + 1);
  };

  if (kp0 < kp1) {
    load_a(kp0);
    load_b(kp0, bcur0, bcur1);
    store_a(0);
  }
  __syncthreads();

  int buf = 0;
  for (int kp = kp0; kp < kp1; ++kp) {
    const bool more = kp + 1 < kp1;
    if (more) {
      load_a(kp + 1);
      load_b(kp + 1, bnext0, bnext1);
    }
    if (p.grouped && (kp & 3) == 0) {
      const u32x4 sv = *reinterpret_cast<const u32x4*>(ssrc + (int64_t)(kp >> 2) * p.n);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t w = sv[j];
        const uint32_t h = hsel ? (w >> 16) : (w & 0xffffu);
        sc[j] = as_h2(h | (h << 16));
      }
    }
    f16x8 afrag[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) afrag[i] = __builtin_bit_cast(f16x8, afr[buf][g][i * 16 + (lane & 15)]);
    const int sh = hsel * 8;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t v0 = bcur0[j] >> sh;
      const uint32_t v1 = bcur1[j] >> sh;
      f16x2 b0 = nib_lo_to_h2(v0, nk);
      f16x2 b1 = nib_lo_to_h2(v1, nk);
      f16x2 b2 = nib_hi_to_h2(v0, nk);
      f16x2 b3 = nib_hi_to_h2(v1, nk);
      if (p.grouped) {
        b0 *= sc[j];
        b1 *= sc[j];
        b2 *= sc[j];
        b3 *= sc[j];
      }
      const f16x8 bfrag = __builtin_bit_cast(f16x8, make_uint4(as_u32(b0), as_u32(b1), as_u32(b2), as_u32(b3)));
#pragma unroll
      for (int i = 0; i < MB; ++i) acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(afrag[i], bfrag, acc[j][i], 0, 0, 0);
    }
    if (more) {
      store_a(buf ^ 1);
      bcur0 = bnext0;
      bcur1 = bnext1;
    }
    __syncthreads();
    buf ^= 1;
  }

  // ---- epilogue ----
  // acc[j][i][e] = C[m0 + 16i + 4*(lane>>4) + e][chunk*64 + 16j + (lane&15)]
  const int rbase = m0 + 4 * (lane >> 4);
  const int ccol = chunk * 64 + (lane & 15);

  if (p.splits > 1) {
    float* part = p.partial + (int64_t)split * p.m * p.n;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = rbase + 16 * i + e;
          if (r < p.m) publish(part + (int64_t)r * p.n + ccol + 16 * j, acc[j][i][e]);
        }
    wait_published();
    __syncthreads();
    int32_t* ctr = p.counters + 1 + cg + mb * p.n_cg;
    if (tid == 0) s_prev = arrive(ctr);
    __syncthreads();
    if (s_prev != p.splits - 1) return;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = rbase + 16 * i + e;
          float sum = 0.f;
          if (r < p.m) {
            for (int sp = 0; sp < p.splits; ++sp)
              sum += collect(p.partial + ((int64_t)sp * p.m + r) * p.n + ccol + 16 * j);
          }
          acc[j][i][e] = sum;
        }
    if (tid == 0) reset_counter(ctr);
  }

  float colscale[4] = {1.f, 1.f, 1.f, 1.f};
  if (!p.grouped) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = ccol + 16 * j;
      const int base = n & ~31, r = n & 31;
      colscale[j] = h2f(p.s[base + 8 * ((r >> 1) & 3) + ((r >> 3) << 1) + (r & 1)]);
    }
  }

  if (EPI == EPI_STORE) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = rbase + 16 * i + e;
          f16 h = (f16)acc[j][i][e];
          if (!p.grouped) h = h * (f16)colscale[j];
          if (r < p.m) p.c[(int64_t)r * p.n + ccol + 16 * j] = __builtin_bit_cast(uint16_t, h);
        }
    return;
  }

  // argmax: per-row best key over this workgroup's 256 columns
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int rl = 16 * i + 4 * (lane >> 4) + e;  // row within tile
      uint64_t best = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f16 h = (f16)acc[j][i][e];
        if (!p.grouped) h = h * (f16)colscale[j];
        best = max_u64(best, argmax_key((float)h, (uint32_t)(ccol + 16 * j)));
      }
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) best = max_u64(best, shfl_xor_u64(best, lane, off));
      if ((lane & 15) == 0) s_keys[wave][rl] = best;
    }
  __syncthreads();
  for (int rl = tid; rl < BM; rl += kThreads) {
    const int r = m0 + rl;
    if (r < p.m) {
      uint64_t best = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) best = max_u64(best, s_keys[w][rl]);
      publish(p.tile_keys + (int64_t)r * p.n_cg + cg, best);
    }
  }
  wait_published();
  __syncthreads();
  int32_t* final_counter = p.counters;
  if (tid == 0) s_prev = arrive(final_counter);
  __syncthreads();
  if (s_prev != p.n_cg * p.n_mb - 1) return;
  for (int r = wave; r < p.m; r += kWaves) {
    uint64_t best = 0;
    for (int t = lane; t < p.n_cg; t += kWave)
      best = max_u64(best, collect(p.tile_keys + (int64_t)r * p.n_cg + t));
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) best = max_u64(best, shfl_xor_u64(best, lane, off));
    if (lane == 0) {
      p.argmax_state[r] = (int64_t)best;
      p.argmax_out[r] = (int64_t)(0xffffffffu - (uint32_t)(best & 0xffffffffu));
    }
  }
  if (tid == 0) reset_counter(final_counter);
}

}  // namespace gemm
}  // namespace lb
