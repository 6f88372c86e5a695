// Rowwise symmetric 2..8-bit groupwise GEMV / pair-GEMV / skinny GEMM and
// single-row dequant on gfx950, plus their C-ABI entry points.
//
// Format (langburst/adapters/qwen36_tools/quantize.py:125-177): row r of
// qweight is an LSB-first bitstream, code c at bits [c*b, c*b+b); value
// (code - 2^(b-1)) * scale[r, c / group] (csrc/lowbit_gemv.cu:4-14, 16-70).
//
// Fast path (row stride % 4 == 0, group % 32 == 0, 16-byte aligned x): one
// wave per output row; a lane takes 32-code units, which are exactly `b`
// dwords, so every load is a dword-aligned vector load.  Codes become exact
// fp16 (code - z) pairs (1024 + code via the fp16 exponent trick, minus
// 1024 + z), multiplied into fp32 with v_dot2_f32_f16 against the fp16 x pair,
// and the unit sum is scaled once in fp32.  The wave reduces with DPP/swizzle.
// General path (any stride / group size): same wave-per-row mapping reading
// bytes like the reference's scalar decode.

#include "lb_common.hpp"

namespace lb {
namespace rowwise {

constexpr int kRowsPerWG = 4;
constexpr int kThreads = kRowsPerWG * kWave;
constexpr int kMaxBatchTile = 4;

struct Params {
  const uint8_t* q[2];
  const uint16_t* s[2];
  uint16_t* y[2];
  const uint16_t* x;
  int64_t x_stride;      // halves between x rows
  int64_t rows, packed_cols, scale_cols;
  int64_t cols, group;
  int batch;
  int unit_shift;        // LDS kernel: log2(group / 32)
};

// Code t (0..31) of a 32-code unit held in BITS dwords w[].
template <int BITS, int T>
__device__ __forceinline__ uint32_t unit_code(const uint32_t* w) {
  constexpr int bit = T * BITS;
  constexpr int d = bit >> 5;
  constexpr int s = bit & 31;
  constexpr uint32_t mask = (1u << BITS) - 1u;
  if constexpr (s + BITS <= 32) {
    return __builtin_amdgcn_ubfe(w[d], s, BITS);
  } else {
    return __builtin_amdgcn_alignbit(w[d + 1], w[d], s) & mask;
  }
}

// fp16 pair (code_t - z, code_{t+1} - z) for t even.
template <int BITS, int T>
__device__ __forceinline__ f16x2 unit_pair(const uint32_t* w) {
  constexpr float zb = 1024.0f + (float)(1 << (BITS - 1));
  if constexpr (BITS == 8) {
    // bytes T, T+1 of dword T/4 under exponent byte 0x64
    constexpr int d = T >> 2;
    constexpr int b0 = T & 3;
    constexpr uint32_t sel = (uint32_t)b0 | (4u << 8) | ((uint32_t)(b0 + 1) << 16) | (4u << 24);
    const uint32_t v = __builtin_amdgcn_perm(0x64646464u, w[d], sel);
    return as_h2(v) - (f16x2){(f16)zb, (f16)zb};
  } else if constexpr (BITS == 4) {
    // nibbles T, T+1 are the two nibbles of byte T/2
    constexpr int d = T >> 3;
    constexpr int by = (T >> 1) & 3;
    const uint32_t spread = __builtin_amdgcn_perm(w[d] >> 4, w[d], (uint32_t)by | (12u << 8) | ((uint32_t)(by + 4) << 16) | (12u << 24));
    const uint32_t v = (spread & 0x000f000fu) | 0x64006400u;
    return as_h2(v) - (f16x2){(f16)zb, (f16)zb};
  } else {
    const uint32_t lo = unit_code<BITS, T>(w);
    const uint32_t hi = unit_code<BITS, T + 1>(w);
    const uint32_t v = ((hi << 16) | lo) | 0x64006400u;
    return as_h2(v) - (f16x2){(f16)zb, (f16)zb};
  }
}

template <int BITS, int T>
__device__ __forceinline__ float unit_dot(const uint32_t* w, const uint32_t* xw, float acc) {
  acc = __builtin_amdgcn_fdot2(unit_pair<BITS, T>(w), as_h2(xw[T >> 1]), acc, false);
  if constexpr (T + 2 < 32) return unit_dot<BITS, T + 2>(w, xw, acc);
  return acc;
}

// Unit sum for a tail unit (codes past `valid` contribute zero).
template <int BITS>
__device__ __forceinline__ float unit_dot_tail(const uint32_t* w, const uint16_t* xrow, int64_t c0, int valid) {
  float acc = 0.f;
  constexpr int z = 1 << (BITS - 1);
#pragma unroll
  for (int t = 0; t < 32; ++t) {
    if (t < valid) {
      const int bit = t * BITS;
      const int d = bit >> 5, s = bit & 31;
      uint32_t v = (s + BITS <= 32) ? (w[d] >> s) : __builtin_amdgcn_alignbit(w[d + 1], w[d], s);
      v &= (1u << BITS) - 1u;
      acc += (float)((int)v - z) * h2f(xrow[c0 + t]);
    }
  }
  return acc;
}

template <int BITS, int NW, int BT>
__global__ __launch_bounds__(kThreads) void rowwise_fast_kernel(Params p) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerWG + wave;
  const int b0 = blockIdx.y * BT;
  if (row >= p.rows) return;
  const int64_t units = (p.cols + 31) >> 5;
  const int64_t full_units = p.cols >> 5;
  const int64_t row_dwords = p.packed_cols >> 2;

  float acc[NW][BT];
#pragma unroll
  for (int a = 0; a < NW; ++a)
#pragma unroll
    for (int b = 0; b < BT; ++b) acc[a][b] = 0.f;

  for (int64_t u = lane; u < units; u += kWave) {
    const int64_t c0 = u << 5;
    const int grp = (int)(c0 / p.group);
    uint32_t w[NW][BITS + 1];
#pragma unroll
    for (int a = 0; a < NW; ++a) {
      const uint32_t* src = reinterpret_cast<const uint32_t*>(p.q[a] + row * p.packed_cols) + u * BITS;
      if (u < full_units) {
#pragma unroll
        for (int d = 0; d < BITS; ++d) w[a][d] = __builtin_nontemporal_load(src + d);
      } else {
#pragma unroll
        for (int d = 0; d < BITS; ++d) w[a][d] = (u * BITS + d < row_dwords) ? src[d] : 0u;
      }
      w[a][BITS] = 0u;
    }
    float sc[NW];
#pragma unroll
    for (int a = 0; a < NW; ++a) sc[a] = h2f(p.s[a][row * p.scale_cols + grp]);
#pragma unroll
    for (int b = 0; b < BT; ++b) {
      if (b0 + b < p.batch) {
        const uint16_t* xrow = p.x + (int64_t)(b0 + b) * p.x_stride;
        if (u < full_units) {
          uint32_t xw[16];
          const uint4* xs = reinterpret_cast<const uint4*>(xrow + c0);
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const uint4 t4 = xs[v];
            xw[4 * v] = t4.x;
            xw[4 * v + 1] = t4.y;
            xw[4 * v + 2] = t4.z;
            xw[4 * v + 3] = t4.w;
          }
#pragma unroll
          for (int a = 0; a < NW; ++a) acc[a][b] += sc[a] * unit_dot<BITS, 0>(w[a], xw, 0.f);
        } else {
          const int valid = (int)(p.cols - c0);
#pragma unroll
          for (int a = 0; a < NW; ++a) acc[a][b] += sc[a] * unit_dot_tail<BITS>(w[a], xrow, c0, valid);
        }
      }
    }
  }
#pragma unroll
  for (int a = 0; a < NW; ++a)
#pragma unroll
    for (int b = 0; b < BT; ++b) {
      const float v = wave_sum(acc[a][b]);
      if (lane == 0 && b0 + b < p.batch) p.y[a][(int64_t)(b0 + b) * p.rows + row] = f2h(v);
    }
}

// ---------------------------------------------------------------------------
// Single-row GEMV with the activation row staged in LDS (batch 1, 2/3/4/8 bits,
// columns a multiple of 32).
//
// A 32-code unit (BITS dwords) is decoded into 16 fp16 pairs with one AND per
// pair: two codes that sit at the same bit offset `off` of the two 16-bit
// halves of a word (after at most one shift, bit-field insert, align or byte
// permute) are kept as they lie, which read as the fp16 subnormals
// (c * 2^off * 2^-24, c' * 2^off * 2^-24), exact.  The workgroup stages the
// activation row once, permuted into the same pair order, so v_dot2_f32_f16
// of a code pair and its activation pair adds the exact x * c * 2^(off-24)
// per code; pairs of one offset share an fp32 accumulator, and the unit's
// sum(x * c) is those sums times 2^(24-off) (exact).  The zero point's share
// z * sum(x) is staged per unit beside the activations and subtracted once,
// and the group scale multiplies the unit sum once, as in the fast path.
// (Scaling the activations by 2^-off instead, for one accumulator, would
// round those below 2^(off-14) to fp16 subnormals: not exact.)  Each wave
// computes R rows (of NW matrices) from one LDS read of the activations.
// ---------------------------------------------------------------------------
constexpr int kLdsWaves = 8;                       // waves (rows x R) per workgroup, unless the shape below says otherwise
constexpr int kLdsRows = 1;                        // rows per wave (one matrix)
constexpr int kLdsUnitBytes = 68;                  // 16 staged pair words + the unit's zero-point share
constexpr int64_t kLdsMaxBytes = 64 * 1024;
// activation units staged per thread of a workgroup of `threads` (the launch
// allows units * kLdsUnitBytes <= kLdsMaxBytes)
constexpr int stage_units(int threads) { return (int)((kLdsMaxBytes / kLdsUnitBytes + threads - 1) / threads); }
// Lane steps of codes prefetched before the activation staging (at most;
// one matrix per wave, about half for two).  Measured at K = 17408 against one
// step: 2 bits (5 steps) 10.65 -> 10.1 us, 3 bits (9 steps) 13.0 -> 12.0 us,
// in_proj_ba (K = 5120, 4 bits, 3 steps) 3.8 -> 3.0 us; 8 bits (32 bytes per
// lane step) 0.5 us slower with 3 or 5 steps, so it keeps one.
constexpr int kLdsPreMax = 9;
constexpr int kLdsPreMax8 = 1;

// Pair q (0..15) of a 32-code unit: codes (lo, hi) and their bit offset.  The
// decode below produces the pairs in this order.
__host__ __device__ constexpr int pair_lo(int bits, int q) {
  return bits == 2 ? 16 * (q >> 3) + (q & 7)
       : bits == 3 ? (q < 5 ? q : q < 9 ? q + 1 : q < 14 ? q + 2 : (q == 14 ? 5 : 10))
       : bits == 4 ? 8 * (q >> 2) + (q & 3)
       : 4 * (q >> 1) + (q & 1);
}
__host__ __device__ constexpr int pair_hi(int bits, int q) {
  return bits == 2 ? pair_lo(2, q) + 8 : bits == 3 ? pair_lo(3, q) + 16 : bits == 4 ? pair_lo(4, q) + 4 : pair_lo(8, q) + 2;
}
// Offset classes: b2 {0,2,4,6,8}, b3 {0,3,6}, b4 {0,4}, b8 {0}.
__host__ __device__ constexpr int n_classes(int bits) { return bits == 2 ? 5 : bits == 3 ? 3 : bits == 4 ? 2 : 1; }
__host__ __device__ constexpr int class_of_off(int bits, int off) {
  return bits == 2 ? off / 2 : bits == 3 ? off / 3 : bits == 4 ? off / 4 : off;
}
__host__ __device__ constexpr int off_of_class(int bits, int c) {
  return bits == 2 ? 2 * c : bits == 3 ? 3 * c : bits == 4 ? 4 * c : c;
}
__host__ __device__ constexpr int pair_off(int bits, int q) {
  return bits == 2 ? ((q & 7) < 5 ? 2 * (q & 7) : 2 * (q & 7) - 6)
       : bits == 3 ? (q == 2 || q == 4 || q == 11 || q == 13 ? 6
                      : q == 1 || q == 3 || q == 6 || q == 8 || q == 10 || q == 12 ? 3 : 0)
       : bits == 4 ? 4 * (q & 1)
       : 0;
}

template <int BITS>
__device__ __forceinline__ void decode_unit(const uint32_t* w, uint32_t (&b)[16]) {
  if constexpr (BITS == 2) {
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      const uint32_t x = w[d], xs = x >> 6;
      b[8 * d + 0] = x & 0x00030003u;
      b[8 * d + 1] = x & 0x000C000Cu;
      b[8 * d + 2] = x & 0x00300030u;
      b[8 * d + 3] = x & 0x00C000C0u;
      b[8 * d + 4] = x & 0x03000300u;
      b[8 * d + 5] = xs & 0x00300030u;
      b[8 * d + 6] = xs & 0x00C000C0u;
      b[8 * d + 7] = xs & 0x03000300u;
    }
  } else if constexpr (BITS == 3) {
    // unit bits [0,16) | [48,64), [16,32) | [64,80), [32,48) | [80,96), and
    // the four codes that straddle those ranges (5, 10, 21, 26); the middle
    // and last ranges are shifted so that every code sits at offset 0, 3 or 6
    // of its half (three offset classes instead of eight: 9 VALU fewer per
    // unit than decoding them in place)
    const uint32_t m0 = (w[0] & 0x0000ffffu) | (w[1] & 0xffff0000u), m0s = m0 >> 6;
    const uint32_t m1 = __builtin_amdgcn_alignbit(w[2], w[0], 18), m1s = __builtin_amdgcn_alignbit(w[2], w[0], 24);
    const uint32_t m2r = (w[1] & 0x0000ffffu) | (w[2] & 0xffff0000u), m2 = m2r >> 1, m2s = m2r >> 7;
    b[0] = m0 & 0x00070007u;
    b[1] = m0 & 0x00380038u;
    b[2] = m0 & 0x01c001c0u;
    b[3] = m0s & 0x00380038u;
    b[4] = m0s & 0x01c001c0u;
    b[5] = m1 & 0x00070007u;
    b[6] = m1 & 0x00380038u;
    b[7] = m1s & 0x00070007u;
    b[8] = m1s & 0x00380038u;
    b[9] = m2 & 0x00070007u;
    b[10] = m2 & 0x00380038u;
    b[11] = m2 & 0x01c001c0u;
    b[12] = m2s & 0x00380038u;
    b[13] = m2s & 0x01c001c0u;
    const uint32_t d0 = __builtin_amdgcn_perm(__builtin_amdgcn_alignbit(w[2], w[1], 31), w[0] >> 15, 0x05040100u);
    const uint32_t d1 = __builtin_amdgcn_perm(w[2] >> 14, __builtin_amdgcn_alignbit(w[1], w[0], 30), 0x05040100u);
    b[14] = d0 & 0x00070007u;
    b[15] = d1 & 0x00070007u;
  } else if constexpr (BITS == 4) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t x = w[d], xs = x >> 8;
      b[4 * d + 0] = x & 0x000f000fu;
      b[4 * d + 1] = x & 0x00f000f0u;
      b[4 * d + 2] = xs & 0x000f000fu;
      b[4 * d + 3] = xs & 0x00f000f0u;
    }
  } else {
    static_assert(BITS == 8, "2, 3, 4 or 8 bits");
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      b[2 * d + 0] = w[d] & 0x00ff00ffu;
      b[2 * d + 1] = (w[d] >> 8) & 0x00ff00ffu;
    }
  }
}

// Arguments as scalars, the ones the prologue needs first: gfx950 preloads
// the leading 16 dwords into SGPRs at wave launch (a struct argument is not
// preloaded), so the code prefetch below needs no kernarg fetch.
template <int BITS, int NW, int R, int UPL, int KPRE, int W, bool HT = false>
__global__ __launch_bounds__(W * kWave) void rowwise_lds_kernel(const uint8_t* q0, const uint8_t* q1,
                                                                  const uint16_t* s0, const uint16_t* s1,
                                                                  const uint16_t* x, int packed_cols, int scale_cols,
                                                                  int cols, int rows, int unit_shift, uint16_t* y0,
                                                                  uint16_t* y1) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int kThreadsWG = W * kWave;
  constexpr int kStageUnits = stage_units(kThreadsWG);
  const int units = cols >> 5;
  u32x4* xt = reinterpret_cast<u32x4*>(smem);                           // [4][units] pair words
  float* corr = reinterpret_cast<float*>(smem + (size_t)units * 64);    // [units]
  const int tid = threadIdx.x;
  constexpr int z = 1 << (BITS - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;

  // ---- per-row bases; the first kPre lane steps of codes and scales are
  // issued right after the activation row's loads, before the staging ----
  const int64_t row0 = ((int64_t)blockIdx.x * W + wave) * R;
  const uint8_t* const qm[2] = {q0, q1};
  const uint16_t* const sm[2] = {s0, s1};
  // per-row bases, wave-uniform; 32-bit offsets from them in the loop
  const uint32_t* qrow[NW][R];
  const uint16_t* srow[NW][R];
#pragma unroll
  for (int a = 0; a < NW; ++a)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t row = row0 + r < rows ? row0 + r : rows - 1;
      qrow[a][r] = reinterpret_cast<const uint32_t*>(qm[a] + row * packed_cols);
      srow[a][r] = sm[a] + row * scale_cols;
    }
  constexpr int kStepWords = UPL * BITS;
  // KPRE lane steps of codes (the host picks enough to cover the row where the
  // registers allow): the whole row is requested at once, so no lane waits a
  // second memory round trip for the row's last units
  constexpr int kPre = KPRE;
  auto load_step = [&](int u0, uint32_t (&w)[NW][R][kStepWords], float (&sc)[UPL][NW][R])
      __attribute__((always_inline)) {
#pragma unroll
    for (int a = 0; a < NW; ++a)
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint32_t* src = qrow[a][r] + (uint32_t)u0 * BITS;
#pragma unroll
        for (int d = 0; d < kStepWords; ++d) w[a][r][d] = __builtin_nontemporal_load(src + d);
        // (UPL = 2: the pair shares one group's scale, sc[0])
#pragma unroll
        for (int j = 0; j < (UPL == 2 ? 1 : UPL); ++j) sc[j][a][r] = h2f(srow[a][r][(uint32_t)(u0 + j) >> unit_shift]);
      }
  };
  // ---- the activation row's loads first (at most kStageUnits units per
  // thread), then the codes, so that the staging waits only for the row and
  // not for the code stream behind it ----
  uint4 xl[kStageUnits][4];
#pragma unroll
  for (int su = 0; su < kStageUnits; ++su) {
    const int u = min(tid + su * kThreadsWG, units - 1);
    const uint4* xs = reinterpret_cast<const uint4*>(x + (int64_t)u * 32);
#pragma unroll
    for (int v = 0; v < 4; ++v) xl[su][v] = xs[v];
  }
  __builtin_amdgcn_sched_barrier(0);
  // HT (two units per lane step, the host checks the shape): the last of the
  // KPRE steps holds at most 32 units (K = 17408: 544 units, four steps and
  // 32) and runs as half units, one 16-code word per lane, lanes 2k and 2k + 1
  // taking the two words of one unit: about a third of a full step's
  // instructions.
  static_assert(!HT || UPL == 2, "half-unit last step: two units per lane step only");
  constexpr int half_step = HT ? kPre - 1 : -1;
  uint32_t wpre[kPre][NW][R][kStepWords];
  float spre[kPre][UPL][NW][R];
#pragma unroll
  for (int i = 0; i < kPre; ++i) {
    if (i == half_step) {
      // word (lane & 1) of unit i * 128 + lane / 2
      const int u = min(i * UPL * kWave + (lane >> 1), units - 1);
#pragma unroll
      for (int a = 0; a < NW; ++a)
#pragma unroll
        for (int r = 0; r < R; ++r) {
          wpre[i][a][r][0] = __builtin_nontemporal_load(qrow[a][r] + (uint32_t)u * BITS + (lane & 1));
          spre[i][0][a][r] = h2f(srow[a][r][(uint32_t)u >> unit_shift]);
        }
      continue;
    }
    // steps past the row load its last step (in bounds; not used)
    const int u0 = min(UPL * lane + i * UPL * kWave, units - UPL);
    load_step(u0, wpre[i], spre[i]);
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- stage the activation row in pair order, and each unit's z * sum(x) ----
#pragma unroll
  for (int su = 0; su < kStageUnits; ++su) {
    const int u = tid + su * kThreadsWG;
    if (u >= units) break;
    uint32_t xd[16];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      xd[4 * v] = xl[su][v].x;
      xd[4 * v + 1] = xl[su][v].y;
      xd[4 * v + 2] = xl[su][v].z;
      xd[4 * v + 3] = xl[su][v].w;
    }
    uint32_t pw[16];
    float sx = 0.f;  // sum of the unit's activations
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int lo = pair_lo(BITS, q), hi = pair_hi(BITS, q);
      const uint32_t sel = (uint32_t)(2 * (lo & 1)) | ((uint32_t)(2 * (lo & 1) + 1) << 8) |
                           ((uint32_t)(4 + 2 * (hi & 1)) << 16) | ((uint32_t)(5 + 2 * (hi & 1)) << 24);
      const uint32_t v = __builtin_amdgcn_perm(xd[hi >> 1], xd[lo >> 1], sel);
      pw[q] = v;
      sx = __builtin_amdgcn_fdot2(as_h2(v), (f16x2){(f16)1.0f, (f16)1.0f}, sx, false);
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) xt[v * units + u] = (u32x4){pw[4 * v], pw[4 * v + 1], pw[4 * v + 2], pw[4 * v + 3]};
    corr[u] = (float)z * sx;
  }
  lds_barrier();  // LDS only: the code loads stay in flight

  // ---- R rows of each of NW matrices per wave ----
  float acc[NW][R];
#pragma unroll
  for (int a = 0; a < NW; ++a)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[a][r] = 0.f;
  // With UPL = 2 (2 bits, even unit count, group >= 64 codes) a lane takes
  // two adjacent units of one scale group per step, so each code load is 16
  // contiguous bytes: wider loads per instruction move the weight stream
  // faster.  The pair is summed as one unit of 64 codes: one set of offset
  // class sums, one z * sum(x) correction, one scale multiply (85 instead
  // of 94 VALU per step).  A lane adds its steps in increasing order.
  auto step = [&](int u0, const uint32_t (&w)[NW][R][kStepWords], const float (&sc)[UPL][NW][R])
      __attribute__((always_inline)) {
    if constexpr (UPL == 2) {
      constexpr int NC = n_classes(BITS);
      float tc[NW][R][NC];
#pragma unroll
      for (int a = 0; a < NW; ++a)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int c = 0; c < NC; ++c) tc[a][r][c] = 0.f;
      float cu = 0.f;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int u = u0 + j;
        uint32_t xq[16];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const u32x4 t4 = xt[v * units + u];
          xq[4 * v] = t4[0];
          xq[4 * v + 1] = t4[1];
          xq[4 * v + 2] = t4[2];
          xq[4 * v + 3] = t4[3];
        }
        cu += corr[u];
#pragma unroll
        for (int a = 0; a < NW; ++a)
#pragma unroll
          for (int r = 0; r < R; ++r) {
            uint32_t b[16];
            decode_unit<BITS>(&w[a][r][j * BITS], b);
#pragma unroll
            for (int q = 0; q < 16; ++q) {
              const int c = class_of_off(BITS, pair_off(BITS, q));
              tc[a][r][c] = __builtin_amdgcn_fdot2(as_h2(b[q]), as_h2(xq[q]), tc[a][r][c], false);
            }
          }
      }
#pragma unroll
      for (int a = 0; a < NW; ++a)
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float t = -cu;
#pragma unroll
          for (int c = 0; c < NC; ++c) t = __builtin_fmaf(tc[a][r][c], (float)(1 << (24 - off_of_class(BITS, c))), t);
          acc[a][r] = __builtin_fmaf(t, sc[0][a][r], acc[a][r]);
        }
      return;
    }
#pragma unroll
    for (int j = 0; j < UPL; ++j) {
      const int u = u0 + j;
      uint32_t xq[16];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const u32x4 t4 = xt[v * units + u];
        xq[4 * v] = t4[0];
        xq[4 * v + 1] = t4[1];
        xq[4 * v + 2] = t4[2];
        xq[4 * v + 3] = t4[3];
      }
      const float cu = corr[u];
#pragma unroll
      for (int a = 0; a < NW; ++a)
#pragma unroll
        for (int r = 0; r < R; ++r) {
          uint32_t b[16];
          decode_unit<BITS>(&w[a][r][j * BITS], b);
          constexpr int NC = n_classes(BITS);
          float tc[NC];
#pragma unroll
          for (int c = 0; c < NC; ++c) tc[c] = 0.f;
#pragma unroll
          for (int q = 0; q < 16; ++q) {
            const int c = class_of_off(BITS, pair_off(BITS, q));
            tc[c] = __builtin_amdgcn_fdot2(as_h2(b[q]), as_h2(xq[q]), tc[c], false);
          }
          float t = -cu;
#pragma unroll
          for (int c = 0; c < NC; ++c) t = __builtin_fmaf(tc[c], (float)(1 << (24 - off_of_class(BITS, c))), t);
          acc[a][r] = __builtin_fmaf(t, sc[j][a][r], acc[a][r]);  // explicit: one rounding in every instantiation
        }
    }
  };
  // the half-unit last step: pairs 8h .. 8h + 7 of the unit (LDS planes 2h,
  // 2h + 1); the unit's z * sum(x) is taken once, by its h = 0 lane
  auto half_unit_step = [&](int i, const uint32_t (&w)[NW][R][kStepWords], const float (&sc)[UPL][NW][R])
      __attribute__((always_inline)) {
    const int h = lane & 1;
    const int u = i * UPL * kWave + (lane >> 1);
    const bool valid = u < units;
    const int uc = valid ? u : units - 1;
    uint32_t xq[8];
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const u32x4 t4 = xt[(2 * h + v) * units + uc];
      xq[4 * v] = t4[0];
      xq[4 * v + 1] = t4[1];
      xq[4 * v + 2] = t4[2];
      xq[4 * v + 3] = t4[3];
    }
    const float cu = h == 0 ? corr[uc] : 0.f;
#pragma unroll
    for (int a = 0; a < NW; ++a)
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint32_t wd[BITS] = {w[a][r][0]};
        uint32_t b[16];
        decode_unit<BITS>(wd, b);  // pairs 0..7 of a one-word unit
        constexpr int NC = n_classes(BITS);
        float tc[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) tc[c] = 0.f;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const int c = class_of_off(BITS, pair_off(BITS, q));
          tc[c] = __builtin_amdgcn_fdot2(as_h2(b[q]), as_h2(xq[q]), tc[c], false);
        }
        float t = -cu;
#pragma unroll
        for (int c = 0; c < NC; ++c) t = __builtin_fmaf(tc[c], (float)(1 << (24 - off_of_class(BITS, c))), t);
        if (valid) acc[a][r] = __builtin_fmaf(t, sc[0][a][r], acc[a][r]);
      }
  };
#pragma unroll
  for (int i = 0; i < kPre; ++i) {
    const int u0 = UPL * lane + i * UPL * kWave;
    if (i == half_step) {
      half_unit_step(i, wpre[i], spre[i]);
      continue;
    }
    if (u0 < units) step(u0, wpre[i], spre[i]);
  }
  for (int u0 = UPL * lane + kPre * UPL * kWave; u0 < units; u0 += UPL * kWave) {
    uint32_t w[NW][R][kStepWords];
    float sc[UPL][NW][R];
    load_step(u0, w, sc);
    step(u0, w, sc);
  }
  uint16_t* const ym[2] = {y0, y1};
#pragma unroll
  for (int a = 0; a < NW; ++a)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float v = wave_sum(acc[a][r]);
      if (lane == 0 && row0 + r < rows) ym[a][row0 + r] = f2h(v);
    }
}

// Any stride / group size: bytes as in the reference's qb_lowbit_value.
template <int NW, int BT>
__global__ __launch_bounds__(kThreads) void rowwise_general_kernel(Params p, int bits) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerWG + wave;
  const int b0 = blockIdx.y * BT;
  if (row >= p.rows) return;
  const uint32_t mask = (1u << bits) - 1u;
  const int z = 1 << (bits - 1);
  float acc[NW][BT];
#pragma unroll
  for (int a = 0; a < NW; ++a)
#pragma unroll
    for (int b = 0; b < BT; ++b) acc[a][b] = 0.f;
  for (int64_t c = lane; c < p.cols; c += kWave) {
    const int64_t bit = c * bits;
    const int64_t byte_i = bit >> 3;
    const int shift = (int)(bit & 7);
    const int64_t grp = c / p.group;
#pragma unroll
    for (int a = 0; a < NW; ++a) {
      const uint8_t* qrow = p.q[a] + row * p.packed_cols;
      uint32_t word = qrow[byte_i];
      if (shift + bits > 8) word |= (uint32_t)qrow[byte_i + 1] << 8;
      const float wq = (float)((int)((word >> shift) & mask) - z) * h2f(p.s[a][row * p.scale_cols + grp]);
#pragma unroll
      for (int b = 0; b < BT; ++b)
        if (b0 + b < p.batch) acc[a][b] += wq * h2f(p.x[(int64_t)(b0 + b) * p.x_stride + c]);
    }
  }
#pragma unroll
  for (int a = 0; a < NW; ++a)
#pragma unroll
    for (int b = 0; b < BT; ++b) {
      const float v = wave_sum(acc[a][b]);
      if (lane == 0 && b0 + b < p.batch) p.y[a][(int64_t)(b0 + b) * p.rows + row] = f2h(v);
    }
}

__global__ void row_dequant_kernel(const uint8_t* __restrict__ q, const uint16_t* __restrict__ s,
                                   const int64_t* __restrict__ row_ptr, uint16_t* __restrict__ out,
                                   int64_t rows, int64_t packed_cols, int64_t scale_cols,
                                   int64_t cols, int64_t group, int bits) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= cols) return;
  const int64_t row = row_ptr[0];
  if (row < 0 || row >= rows) {
    out[c] = 0;
    return;
  }
  const uint8_t* qrow = q + row * packed_cols;
  const int64_t bit = c * bits;
  const int64_t byte_i = bit >> 3;
  const int shift = (int)(bit & 7);
  uint32_t word = qrow[byte_i];
  if (shift + bits > 8) word |= (uint32_t)qrow[byte_i + 1] << 8;
  const int v = (int)((word >> shift) & ((1u << bits) - 1u)) - (1 << (bits - 1));
  out[c] = f2h((float)v * h2f(s[row * scale_cols + c / group]));
}

template <int NW, int BT>
int launch_bt(const Params& p, int bits, bool fast, hipStream_t st) {
  dim3 grid((unsigned)((p.rows + kRowsPerWG - 1) / kRowsPerWG), (unsigned)((p.batch + BT - 1) / BT));
  if (!fast) {
    hipLaunchKernelGGL((rowwise_general_kernel<NW, BT>), grid, dim3(kThreads), 0, st, p, bits);
    return lbh::launch_status();
  }
  switch (bits) {
#define LB_CASE(B) \
  case B: hipLaunchKernelGGL((rowwise_fast_kernel<B, NW, BT>), grid, dim3(kThreads), 0, st, p); break;
    LB_CASE(2) LB_CASE(3) LB_CASE(4) LB_CASE(5) LB_CASE(6) LB_CASE(7) LB_CASE(8)
#undef LB_CASE
    default: return LB_ERR_ARG;
  }
  return lbh::launch_status();
}

// One bit width of the one-row kernel on workgroups of W waves of R rows.
template <int B, int NW, int W, int R>
int launch_lds_bits(const Params& p, hipStream_t st) {
  const int64_t rows_per_wg = (int64_t)W * R;
  dim3 grid((unsigned)((p.rows + rows_per_wg - 1) / rows_per_wg));
  const size_t lds = (size_t)(p.cols >> 5) * kLdsUnitBytes;
  // 2 bits: two units per lane step (16-byte code loads) where every lane's
  // pair lies inside the row and inside one scale group (group >= 64 codes:
  // the kernel then sums the pair as one).  Measured at K = 17408: 2 bits 4 %
  // faster; 3 bits mixed (g64 faster, g128 slower); 4 bits 15 % slower, so
  // 3-8 bits keep one.
  const bool pairs = ((p.cols >> 5) & 1) == 0 && p.unit_shift > 0;
  // Lane steps prefetched before the staging: enough to cover the row (one
  // flood of requests, no second round trip for the row's tail), up to
  // kLdsPreMax, so that the workgroups of a BASELINE.json rowwise launch stay
  // resident at once.
  const int upl = (B == 2 && pairs) ? 2 : 1;
  const int64_t steps = ((p.cols >> 5) + upl * kWave - 1) / (upl * kWave);
  const int cap = B == 8 ? kLdsPreMax8 : (NW == 1 ? kLdsPreMax : 5);
  const int64_t want = std::min<int64_t>(steps, cap);
  const int kp = want <= 1 ? 1 : want <= 2 ? 2 : want <= 3 ? 3 : want <= 5 ? 5 : 9;
  // two units per lane step: a last step of at most 32 units, when the
  // prefetched steps are exactly the row's, runs as half units (K = 17408,
  // N = 5120: 8.76 -> 8.4 us)
  const int64_t tail = (p.cols >> 5) % (upl * kWave);
  const bool ht = upl == 2 && tail > 0 && tail <= kWave / 2 && steps == kp && kp > 1;
#define LB_LAUNCH_T(U, KP, HTV)                                                                                    \
  hipLaunchKernelGGL((rowwise_lds_kernel<B, NW, R, U, KP, W, HTV>), grid, dim3(W * kWave), lds, st, p.q[0], p.q[1], \
                     p.s[0], p.s[1], p.x, (int)p.packed_cols, (int)p.scale_cols, (int)p.cols, (int)p.rows,           \
                     p.unit_shift, p.y[0], p.y[1])
#define LB_LAUNCH(U, KP) LB_LAUNCH_T(U, KP, false)
#define LB_LKP(U)                          \
  do {                                     \
    if (kp == 1) LB_LAUNCH(U, 1);          \
    else if (kp == 2) LB_LAUNCH(U, 2);     \
    else if (kp == 3) LB_LAUNCH(U, 3);     \
    else if (kp == 5) LB_LAUNCH(U, 5);     \
    else LB_LAUNCH(U, 9);                  \
  } while (0)
  if constexpr (B == 8) {
    LB_LAUNCH(1, kLdsPreMax8);
  } else if constexpr (B == 2) {
    if (pairs && ht) {
      if (kp == 2) LB_LAUNCH_T(2, 2, true);
      else if (kp == 3) LB_LAUNCH_T(2, 3, true);
      else if (kp == 5) LB_LAUNCH_T(2, 5, true);
      else LB_LAUNCH_T(2, 9, true);
    } else if (pairs) {
      LB_LKP(2);
    } else {
      LB_LKP(1);
    }
  } else {
    LB_LKP(1);
  }
#undef LB_LKP
#undef LB_LAUNCH
#undef LB_LAUNCH_T
  return lbh::launch_status();
}

// Workgroup shape of the one-row kernel.  A workgroup stages the whole
// activation row in LDS, so fewer, wider workgroups stage it fewer times;
// the shapes below give the BASELINE.json configs one workgroup per CU where that
// measured faster (one process, graph replay, against 8 waves of one row):
//   8 bits, 5120 x 17408:  10 waves of 2 rows (256 workgroups) 18.5 us against 21.2 us;
//   4 bits, 4096 x 4096:   16 waves of 1 row  (256 workgroups)  3.66 us against 3.95 us.
// 2 and 3 bits keep 8 waves of one row (2.5 workgroups per CU): every other
// shape measured slower there (10 waves of 1 or 2 rows by 11-15 %, 16 waves by
// 25-30 %, 8 waves of 2 rows by 27-38 %).
template <int NW>
int launch_lds(const Params& p, int bits, hipStream_t st) {
  if constexpr (NW == 1) {
    const int64_t cus = lbh::device_cus();
    if (bits == 8 && p.rows >= 20 * cus) return launch_lds_bits<8, 1, 10, 2>(p, st);
    if (bits == 4 && p.rows >= 16 * cus) return launch_lds_bits<4, 1, 16, 1>(p, st);
  }
  constexpr int R = NW == 1 ? kLdsRows : (kLdsRows + 1) / 2;
  switch (bits) {
    case 2: return launch_lds_bits<2, NW, kLdsWaves, R>(p, st);
    case 3: return launch_lds_bits<3, NW, kLdsWaves, R>(p, st);
    case 4: return launch_lds_bits<4, NW, kLdsWaves, R>(p, st);
    case 8: return launch_lds_bits<8, NW, kLdsWaves, R>(p, st);
    default: return LB_ERR_ARG;
  }
}

int launch(Params p, int nw, int bits, hipStream_t st) {
  const bool fast = (p.packed_cols % 4 == 0) && lbh::aligned(p.q[0], 4) && (nw == 1 || lbh::aligned(p.q[1], 4)) &&
                    (p.group % 32 == 0) && (p.x_stride % 8 == 0) && lbh::aligned(p.x, 16);
  // one activation row, whole units, staged in LDS
  const int64_t gu = p.group / 32;  // units per group
  const bool lds = fast && p.batch == 1 && p.cols % 32 == 0 && (bits == 2 || bits == 3 || bits == 4 || bits == 8) &&
                   (p.cols >> 5) * kLdsUnitBytes <= kLdsMaxBytes && (gu & (gu - 1)) == 0 &&
                   p.packed_cols * (p.rows > 0 ? 1 : 0) <= (int64_t)0xffffffff / 2 &&
                   p.rows < (int64_t(1) << 31) && p.scale_cols < (int64_t(1) << 31);  // int kernel arguments
  if (lds) {
    p.unit_shift = 0;
    while ((int64_t(1) << p.unit_shift) < gu) ++p.unit_shift;
  }
  if (lds) return nw == 1 ? launch_lds<1>(p, bits, st) : launch_lds<2>(p, bits, st);
  if (p.batch <= 1) {
    return nw == 1 ? launch_bt<1, 1>(p, bits, fast, st) : launch_bt<2, 1>(p, bits, fast, st);
  }
  if (p.batch == 2) return nw == 1 ? launch_bt<1, 2>(p, bits, fast, st) : launch_bt<2, 2>(p, bits, fast, st);
  return nw == 1 ? launch_bt<1, kMaxBatchTile>(p, bits, fast, st) : launch_bt<2, kMaxBatchTile>(p, bits, fast, st);
}

// Argument checks shared by the rowwise entry points; mirrors check_lowbit_args
// (csrc/lowbit_gemv.cu:250-268) on raw sizes.
int check(const void* q, const void* s, int64_t rows, int64_t packed_cols, int64_t scale_cols,
          int64_t cols, int64_t group, int64_t bits) {
  if (!q || !s) return LB_ERR_ARG;
  if (rows < 0 || cols <= 0 || group <= 0) return LB_ERR_ARG;
  if (bits < 2 || bits > 8) return LB_ERR_ARG;
  const int64_t n_groups = (cols + group - 1) / group;
  const int64_t packed_need = (cols * bits + 7) / 8;
  if (scale_cols < n_groups || packed_cols < packed_need) return LB_ERR_ARG;
  return LB_OK;
}

bool rows_per_cta_ok(int64_t r) { return r == 4 || r == 8 || r == 16; }

}  // namespace rowwise
}  // namespace lb

using namespace lb;

extern "C" int lb_lowbit_gemv(const uint8_t* qweight, int64_t rows, int64_t packed_cols,
                              const uint16_t* scales, int64_t scale_cols,
                              const uint16_t* x, uint16_t* y,
                              int64_t cols, int64_t group_size, int64_t bits, int64_t rows_per_cta,
                              lb_stream_t stream) {
  int st = rowwise::check(qweight, scales, rows, packed_cols, scale_cols, cols, group_size, bits);
  if (st) return st;
  if (!rowwise::rows_per_cta_ok(rows_per_cta) || !x || (!y && rows > 0)) return LB_ERR_ARG;
  if (rows == 0) return LB_OK;
  rowwise::Params p{};
  p.q[0] = qweight; p.s[0] = scales; p.y[0] = y;
  p.q[1] = qweight; p.s[1] = scales; p.y[1] = y;
  p.x = x; p.x_stride = cols; p.rows = rows; p.packed_cols = packed_cols; p.scale_cols = scale_cols;
  p.cols = cols; p.group = group_size; p.batch = 1;
  return rowwise::launch(p, 1, (int)bits, (hipStream_t)stream);
}

extern "C" int lb_lowbit_gemv_pair(const uint8_t* qweight_a, const uint16_t* scales_a,
                                   const uint8_t* qweight_b, const uint16_t* scales_b,
                                   int64_t rows, int64_t packed_cols, int64_t scale_cols,
                                   const uint16_t* x, uint16_t* y_a, uint16_t* y_b,
                                   int64_t cols, int64_t group_size, int64_t bits, int64_t rows_per_cta,
                                   lb_stream_t stream) {
  int st = rowwise::check(qweight_a, scales_a, rows, packed_cols, scale_cols, cols, group_size, bits);
  if (st) return st;
  st = rowwise::check(qweight_b, scales_b, rows, packed_cols, scale_cols, cols, group_size, bits);
  if (st) return st;
  if (!rowwise::rows_per_cta_ok(rows_per_cta) || !x || ((!y_a || !y_b) && rows > 0)) return LB_ERR_ARG;
  if (rows == 0) return LB_OK;
  rowwise::Params p{};
  p.q[0] = qweight_a; p.s[0] = scales_a; p.y[0] = y_a;
  p.q[1] = qweight_b; p.s[1] = scales_b; p.y[1] = y_b;
  p.x = x; p.x_stride = cols; p.rows = rows; p.packed_cols = packed_cols; p.scale_cols = scale_cols;
  p.cols = cols; p.group = group_size; p.batch = 1;
  return rowwise::launch(p, 2, (int)bits, (hipStream_t)stream);
}

extern "C" int lb_lowbit_gemm(const uint8_t* qweight, int64_t rows, int64_t packed_cols,
                              const uint16_t* scales, int64_t scale_cols,
                              const uint16_t* x, int64_t batch, int64_t x_stride, uint16_t* y,
                              int64_t cols, int64_t group_size, int64_t bits, int64_t rows_per_cta,
                              lb_stream_t stream) {
  int st = rowwise::check(qweight, scales, rows, packed_cols, scale_cols, cols, group_size, bits);
  if (st) return st;
  if (!rowwise::rows_per_cta_ok(rows_per_cta) || batch < 0 || x_stride < cols) return LB_ERR_ARG;
  if (rows == 0 || batch == 0) return LB_OK;
  if (!x || !y || batch > 65535 * (int64_t)rowwise::kMaxBatchTile) return LB_ERR_ARG;
  rowwise::Params p{};
  p.q[0] = qweight; p.s[0] = scales; p.y[0] = y;
  p.q[1] = qweight; p.s[1] = scales; p.y[1] = y;
  p.x = x; p.x_stride = x_stride; p.rows = rows; p.packed_cols = packed_cols; p.scale_cols = scale_cols;
  p.cols = cols; p.group = group_size; p.batch = (int)batch;
  return rowwise::launch(p, 1, (int)bits, (hipStream_t)stream);
}

extern "C" int lb_lowbit_row_dequant(const uint8_t* qweight, int64_t rows, int64_t packed_cols,
                                     const uint16_t* scales, int64_t scale_cols,
                                     const int64_t* row_index, uint16_t* out,
                                     int64_t cols, int64_t group_size, int64_t bits,
                                     lb_stream_t stream) {
  int st = rowwise::check(qweight, scales, rows, packed_cols, scale_cols, cols, group_size, bits);
  if (st) return st;
  if (!row_index || !out) return LB_ERR_ARG;
  const int threads = 256;
  const int64_t blocks = (cols + threads - 1) / threads;
  hipLaunchKernelGGL(rowwise::row_dequant_kernel, dim3((unsigned)blocks), dim3(threads), 0, (hipStream_t)stream,
                     qweight, scales, row_index, out, rows, packed_cols, scale_cols, cols, group_size, (int)bits);
  return lbh::launch_status();
}
