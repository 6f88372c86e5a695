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

int launch(Params p, int nw, int bits, hipStream_t st) {
  const bool fast = (p.packed_cols % 4 == 0) && lbh::aligned(p.q[0], 4) && (nw == 1 || lbh::aligned(p.q[1], 4)) &&
                    (p.group % 32 == 0) && (p.x_stride % 8 == 0) && lbh::aligned(p.x, 16);
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
