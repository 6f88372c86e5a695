// Marlin-layout W4A16 GEMM for prefill batches (M > 16) on gfx950.
//
// Same fragment construction as the decode kernel (marlin_skinny.hpp): B
// fragments of v_mfma_f32_16x16x32_f16 are built in registers from the
// reference's Marlin layout (langburst/csrc/marlin_cuda_kernel.cu; packing in
// adapters/qwen36_tools/quantize.py:180-243) -- one 16-byte slot per lane, the
// pair's other slot from lane ^ 8 by DPP -- as the exact fp16 (q-8) times the
// fp16 group scale (the reference's __hmul2 rounding).  Each dequantised B
// fragment feeds MB MFMAs (MB 16-row blocks of A), so the VALU dequant cost is
// amortised over 16*MB rows.
//
// Workgroup tile: (16*MB rows) x 256 columns; wave w owns 64-column chunk w.
// The k loop runs in stages of one scale group (128 k = 4 MFMA steps):
//   A  -- the stage's rows are read from global memory (16 B per item, one
//         row's 256 bytes by 16 consecutive threads) one stage ahead into
//         registers, then written to a double-buffered LDS tile in fragment
//         order (entry (d, g, r) = A[r][32d + 16(g>>1) + 4(g&1) + {0..3}] ++
//         the same + 8); one __syncthreads per stage.
//   B  -- each lane's slots and the group scales two stages ahead.
// The stage loop is unrolled by two so that buffer and slot indices are
// compile-time constants.  Optional split-K over S workgroups uses the same
// deterministic hand-off as the decode kernel (fp32 partials in scratch, the
// last arrival sums them in split order).

#pragma once
#include <type_traits>

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

// Raw buffer resource (gfx9 V#: stride 0, 32-bit data format).  Loads at or
// past num_records return zero: rows of the last M block beyond M use that.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

constexpr int kSteps = 4;  // 32-k steps per stage (one scale group of 128)

template <int MB, int AM, int EPI, bool GROUPED>
__global__ __launch_bounds__(kThreads) void marlin_gemm_kernel(Params p) {
  constexpr int BM = 16 * MB;
  // A stage in LDS, fragment order, double-buffered: entry (d, g, r) is 16 B:
  // A[r][32d + 16(g>>1) + 4(g&1) + {0..3}] ++ the same + 8.  Each (d, g) block
  // is padded by one entry so that the staging writes of one row, which go to
  // different (d, g) blocks, land in different banks.
  constexpr int kBlk = BM + 1;
  __shared__ __attribute__((aligned(16))) uint4 afr[2][kSteps * 4 * kBlk];
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
  const int st0 = kp0 / kSteps;         // first scale group (stage)
  const int nst = (kp1 - kp0) / kSteps; // stages of this split

  const int chunk = cg * kWaves + wave;
  const uint32_t row_bytes = 8u * (uint32_t)p.n;
  const int g = lane >> 4;
  const int hsel = (lane >> 3) & 1;
  const int cc = lane & 7;
  const int prow = g >> 1;
  const int gq = g & 1;
  const __amdgpu_buffer_rsrc_t rb = buffer_of(p.b, (uint32_t)p.k / 16u * row_bytes);
  const __amdgpu_buffer_rsrc_t rs = buffer_of(p.s, (GROUPED ? (uint32_t)(p.k / 128) : 1u) * (uint32_t)p.n * 2u);
  // each lane loads slot 4c + 2gq + h of row 2kp + prow; the pair's other slot
  // comes from lane ^ 8 (DPP row rotation)
  const uint32_t b_off = (uint32_t)prow * row_bytes + (uint32_t)chunk * 512u + (uint32_t)(cc * 4 + gq * 2 + hsel) * 16u;
  const uint32_t s_off = ((uint32_t)chunk * 64u + (uint32_t)cc * 8u) * 2u;
  const uint32_t psel = hsel ? 0x07030501u : 0x02060004u;
  const NibConsts nk = nib_consts();

  // ---- A staging: items (row r, octet o) of 8 halves, r-major so that 16
  // consecutive threads read one row's 256 contiguous bytes ----
  constexpr int kAItems = BM * 16;
  constexpr int kAPer = kAItems / kThreads;
  static_assert(kAItems % kThreads == 0, "A staging items");
  const int64_t a_row_halves = AM == A_SILU_PACKED ? 2 * (int64_t)p.k : (int64_t)p.k;
  const __amdgpu_buffer_rsrc_t ra = buffer_of(p.a, (uint32_t)((int64_t)p.m * a_row_halves * 2));
  uint4 areg[kAPer];
  uint4 ureg[AM == A_SILU_PACKED ? kAPer : 1];
  auto load_a = [&](int stage) {
#pragma unroll
    for (int t = 0; t < kAPer; ++t) {
      const int item = tid + t * kThreads;
      const int r = item >> 4, o = item & 15;
      const uint32_t off = (uint32_t)(((int64_t)(m0 + r) * a_row_halves + (int64_t)stage * 128 + 8 * o) * 2);
      areg[t] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 0));
      if (AM == A_SILU_PACKED)
        ureg[t] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ra, off + 2u * (uint32_t)p.k, 0, 0));
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int t = 0; t < kAPer; ++t) {
      const int item = tid + t * kThreads;
      const int r = item >> 4, o = item & 15;
      uint4 w = areg[t];
      if (AM == A_SILU_PACKED) {
        const uint4 u = ureg[t];
        const uint32_t gw[4] = {w.x, w.y, w.z, w.w};
        const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
        uint32_t ov[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float g0 = h2f((uint16_t)(gw[e] & 0xffffu)), g1 = h2f((uint16_t)(gw[e] >> 16));
          const float u0 = h2f((uint16_t)(uw[e] & 0xffffu)), u1 = h2f((uint16_t)(uw[e] >> 16));
          ov[e] = (uint32_t)f2h(silu(g0) * u0) | ((uint32_t)f2h(silu(g1) * u1) << 16);
        }
        w = make_uint4(ov[0], ov[1], ov[2], ov[3]);
      }
      // octet o = 4d + 2prow + half: halves 0..3 -> (d, g = 2prow), 4..7 -> (d, g = 2prow + 1)
      const int d = o >> 2, pr = (o >> 1) & 1, half = o & 1;
      uint2* dst0 = reinterpret_cast<uint2*>(&afr[buf][(d * 4 + 2 * pr) * kBlk + r]) + half;
      uint2* dst1 = reinterpret_cast<uint2*>(&afr[buf][(d * 4 + 2 * pr + 1) * kBlk + r]) + half;
      *dst0 = make_uint2(w.x, w.y);
      *dst1 = make_uint2(w.z, w.w);
    }
  };

  // ---- B ring: two stages of (4 slots + the group's scales) per lane ----
  u32x4 bst[2][kSteps];
  u32x4 sst[2];
  auto load_b = [&](int slot, int stage) {
#pragma unroll
    for (int d = 0; d < kSteps; ++d)
      bst[slot][d] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, b_off, (uint32_t)(stage * 8 + 2 * d) * row_bytes, 0));
    if (GROUPED)
      sst[slot] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, s_off, (uint32_t)stage * (uint32_t)p.n * 2u, 0));
  };

  f32x4 acc[4][MB];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[j][i] = (f32x4){0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int buf, int slot) {
    f16x2 sc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t h = GROUPED ? ((sst[slot][j] >> (16 * hsel)) & 0xffffu) : 0x3c00u;  // fp16 1.0
      sc[j] = as_h2(h | (h << 16));
    }
#pragma unroll
    for (int d = 0; d < kSteps; ++d) {
      f16x8 bfrag[4];
      const u32x4 own = bst[slot][d];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t partner = (uint32_t)__builtin_amdgcn_mov_dpp((int)own[j], 0x128, 0xf, 0xf, false);  // row_ror:8
        const uint32_t v0 = __builtin_amdgcn_perm(own[j], partner, psel);
        const uint32_t v1 = v0 >> 8;
        // exact fp16 (q - 8) times the fp16 group scale: the rounding of the reference's __hmul2
        const f16x2 b0 = nib_lo_to_h2(v0, nk) * sc[j];
        const f16x2 b1 = nib_lo_to_h2(v1, nk) * sc[j];
        const f16x2 b2 = nib_hi_to_h2(v0, nk) * sc[j];
        const f16x2 b3 = nib_hi_to_h2(v1, nk) * sc[j];
        bfrag[j] = __builtin_bit_cast(f16x8, make_uint4(as_u32(b0), as_u32(b1), as_u32(b2), as_u32(b3)));
      }
      const uint4* abase = &afr[buf][(d * 4 + g) * kBlk + (lane & 15)];
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        const f16x8 afrag = __builtin_bit_cast(f16x8, abase[16 * i]);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(afrag, bfrag[j], acc[j][i], 0, 0, 0);
      }
    }
  };

  // ---- pipeline: A one stage ahead (registers -> LDS), B two stages ahead ----
  if (nst > 0) {
    load_a(st0);
    load_b(0, st0);
    if (nst > 1) load_b(1, st0 + 1);
    store_a(0);
    __syncthreads();
    if (nst > 1) load_a(st0 + 1);
    // Stage s uses LDS buffer and B slot s & 1; unrolled by two so that both
    // are compile-time constants (no indexed register access).
    auto stage = [&](int s, auto par) {
      constexpr int c = decltype(par)::value;
      compute(c, c);
      if (s + 2 < nst) load_b(c, st0 + s + 2);
      if (s + 1 < nst) store_a(c ^ 1);  // buffer c ^ 1 was last read in stage s - 1
      __syncthreads();
      if (s + 2 < nst) load_a(st0 + s + 2);
    };
    for (int s = 0; s < nst; s += 2) {
      stage(s, std::integral_constant<int, 0>{});
      if (s + 1 >= nst) break;
      stage(s + 1, std::integral_constant<int, 1>{});
    }
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
  if (!GROUPED) {
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
          if (!GROUPED) h = h * (f16)colscale[j];
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
        if (!GROUPED) h = h * (f16)colscale[j];
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
