/*
 * CPU restatement (plain C) of the scalar pieces of LangBurst's low-bit
 * projection path.  TEST INFRASTRUCTURE, NOT PRODUCT CODE: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load this library.
 *
 * Paths below are relative to /root/reference/langburst.
 *   orc_rowwise_value   <- csrc/lowbit_gemv.cu:4-14 (qb_lowbit_value)
 *   orc_rowwise_gemm    <- csrc/lowbit_gemv.cu:145-224 (fp32 terms, fp16 out)
 *   orc_marlin_code     <- csrc/marlin_mlp_stream.cu:109-133 (inverse-perm reader)
 *   orc_marlin_scale    <- csrc/marlin_mlp_stream.cu:91-107
 *   orc_marlin_gemm     <- csrc/marlin_cuda_kernel.cu:131-159 (fp16 dequant),
 *                          :92-104 (fp32 MMA accumulate), :651-659 (fp16 store)
 * The inverse permutation is regenerated from the generator definition in
 * adapters/qwen36_tools/quantize.py:50-76, independently of the numpy oracle.
 * Sums are accumulated in double (the exact sum of the fp32 terms the
 * reference accumulates in fp32), then rounded once to fp16.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* IEEE binary16 <-> binary32, round-to-nearest-even, with subnormals. */
float orc_half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      float f = (float)man * (1.0f / 16777216.0f); /* man * 2^-24 */
      memcpy(&bits, &f, 4);
      bits |= sign;
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float out;
  memcpy(&out, &bits, 4);
  return out;
}

uint16_t orc_float_to_half(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t absx = x & 0x7fffffffu;
  if (absx >= 0x7f800000u) { /* inf or nan */
    return (uint16_t)(sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u : 0u));
  }
  if (absx >= 0x477ff000u) { /* rounds to >= 65520 -> inf */
    return (uint16_t)(sign | 0x7c00u);
  }
  if (absx < 0x38800000u) { /* below 2^-14: subnormal half (or zero) */
    float af;
    memcpy(&af, &absx, 4);
    /* value in units of 2^-24, rounded to nearest even */
    double scaled = (double)af * 16777216.0;
    double fl = floor(scaled);
    double rem = scaled - fl;
    uint32_t m = (uint32_t)fl;
    if (rem > 0.5 || (rem == 0.5 && (m & 1u))) m++;
    return (uint16_t)(sign | m);
  }
  uint32_t exp = ((absx >> 23) - 112u);
  uint32_t man = absx & 0x7fffffu;
  uint32_t hm = man >> 13;
  uint32_t rest = man & 0x1fffu;
  uint32_t h = (exp << 10) | hm;
  if (rest > 0x1000u || (rest == 0x1000u && (hm & 1u))) h++;
  return (uint16_t)(sign | h);
}

int orc_rowwise_value(const uint8_t* row, int64_t row_bytes, int c, int bits) {
  const int64_t bit_pos = (int64_t)c * bits;
  const int64_t byte_i = bit_pos >> 3;
  const int shift = (int)(bit_pos & 7);
  uint32_t word = row[byte_i];
  if (shift + bits > 8 && byte_i + 1 < row_bytes) word |= (uint32_t)row[byte_i + 1] << 8;
  return (int)((word >> shift) & ((1u << bits) - 1u)) - (1 << (bits - 1));
}

/* y[b, r] = fp16( sum_c (q*s) * x[b, c] ) */
void orc_rowwise_gemm(const uint8_t* qweight, int64_t rows, int64_t packed_cols,
                      const uint16_t* scales, int64_t scale_cols,
                      const uint16_t* x, int64_t batch, int64_t x_stride,
                      int64_t cols, int64_t group_size, int bits, uint16_t* y) {
  for (int64_t b = 0; b < batch; ++b) {
    for (int64_t r = 0; r < rows; ++r) {
      const uint8_t* qrow = qweight + r * packed_cols;
      double acc = 0.0;
      for (int64_t c = 0; c < cols; ++c) {
        const int q = orc_rowwise_value(qrow, packed_cols, (int)c, bits);
        const float s = orc_half_to_float(scales[r * scale_cols + c / group_size]);
        const float w = (float)q * s; /* exact in fp32 */
        acc += (double)w * (double)orc_half_to_float(x[b * x_stride + c]);
      }
      y[b * rows + r] = orc_float_to_half((float)acc);
    }
  }
}

static int g_inv_ready = 0;
static int g_inv_perm[1024];
static int g_inv_scale_perm[64];
static int g_inv_scale_perm_single[32];

static void orc_init_tables(void) {
  if (g_inv_ready) return;
  int perm[1024];
  int n = 0;
  for (int i = 0; i < 32; ++i) {
    int perm1[8];
    int t = 0;
    const int col = i / 4;
    for (int block = 0; block < 2; ++block) {
      const int rows4[4] = {2 * (i % 4), 2 * (i % 4) + 1, 2 * (i % 4 + 4), 2 * (i % 4 + 4) + 1};
      for (int rr = 0; rr < 4; ++rr) perm1[t++] = 16 * rows4[rr] + col + 8 * block;
    }
    for (int j = 0; j < 4; ++j)
      for (int e = 0; e < 8; ++e) perm[n++] = perm1[e] + 256 * j;
  }
  static const int interleave[8] = {0, 2, 4, 6, 1, 3, 5, 7};
  int perm2[1024];
  for (int blk = 0; blk < 128; ++blk)
    for (int e = 0; e < 8; ++e) perm2[blk * 8 + e] = perm[blk * 8 + interleave[e]];
  for (int j = 0; j < 1024; ++j) g_inv_perm[perm2[j]] = j;
  int sp[64];
  for (int i = 0; i < 8; ++i)
    for (int j = 0; j < 8; ++j) sp[i * 8 + j] = i + 8 * j;
  for (int j = 0; j < 64; ++j) g_inv_scale_perm[sp[j]] = j;
  static const int off[8] = {0, 1, 8, 9, 16, 17, 24, 25};
  int sps[32];
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 8; ++j) sps[i * 8 + j] = 2 * i + off[j];
  for (int j = 0; j < 32; ++j) g_inv_scale_perm_single[sps[j]] = j;
  g_inv_ready = 1;
}

/* Copies the regenerated inverse tables out (for pinning against the hashes). */
void orc_marlin_inverse_tables(int32_t* inv_perm, int32_t* inv_scale, int32_t* inv_scale_single) {
  orc_init_tables();
  for (int i = 0; i < 1024; ++i) inv_perm[i] = g_inv_perm[i];
  for (int i = 0; i < 64; ++i) inv_scale[i] = g_inv_scale_perm[i];
  for (int i = 0; i < 32; ++i) inv_scale_single[i] = g_inv_scale_perm_single[i];
}

int orc_marlin_code(const int32_t* qweight, int64_t prob_n, int64_t in_col, int64_t out_col) {
  orc_init_tables();
  const int64_t kblock = in_col >> 4, kinner = in_col & 15;
  const int64_t nblock = out_col >> 4, ninner = out_col & 15;
  const int64_t pre = nblock * 256 + kinner * 16 + ninner;
  const int64_t base = (pre / 1024) * 1024;
  const int64_t fin = base + g_inv_perm[pre - base];
  const uint32_t word = (uint32_t)qweight[kblock * (prob_n * 2) + (fin >> 3)];
  return (int)((word >> (4 * (fin & 7))) & 0xfu);
}

uint16_t orc_marlin_scale(const uint16_t* scales, int64_t prob_n, int64_t group, int64_t out_col, int per_column) {
  orc_init_tables();
  if (per_column) {
    const int64_t base = (out_col / 32) * 32;
    return scales[base + g_inv_scale_perm_single[out_col - base]];
  }
  const int64_t flat = group * prob_n + out_col;
  const int64_t base = (flat / 64) * 64;
  return scales[base + g_inv_scale_perm[flat - base]];
}

/* C[m, n] for the rows listed in row_idx (or all rows when row_idx == NULL). */
void orc_marlin_gemm(const uint16_t* a, int64_t prob_m, const int32_t* qweight, const uint16_t* scales,
                     int64_t prob_n, int64_t prob_k, int64_t group_size,
                     const int64_t* row_idx, int64_t n_rows, uint16_t* c) {
  orc_init_tables();
  const int per_column = (group_size <= 0 || group_size == prob_k);
  const int64_t rows = row_idx ? n_rows : prob_m;
  for (int64_t n = 0; n < prob_n; ++n) {
    /* dequantise column n once: w = fp16(fp16(q-8) * s) */
    static float wcol[1 << 17];
    if (prob_k > (1 << 17)) return;
    for (int64_t k = 0; k < prob_k; ++k) {
      const int q = orc_marlin_code(qweight, prob_n, k, n) - 8;
      if (per_column) {
        wcol[k] = (float)q;
      } else {
        const float s = orc_half_to_float(orc_marlin_scale(scales, prob_n, k / group_size, n, 0));
        wcol[k] = orc_half_to_float(orc_float_to_half((float)q * s));
      }
    }
    const float sc = per_column ? orc_half_to_float(orc_marlin_scale(scales, prob_n, 0, n, 1)) : 1.0f;
    for (int64_t ri = 0; ri < rows; ++ri) {
      const int64_t m = row_idx ? row_idx[ri] : ri;
      double acc = 0.0;
      for (int64_t k = 0; k < prob_k; ++k)
        acc += (double)wcol[k] * (double)orc_half_to_float(a[m * prob_k + k]);
      uint16_t h = orc_float_to_half((float)acc);
      if (per_column) h = orc_float_to_half(orc_half_to_float(h) * sc);
      c[ri * prob_n + n] = h;
    }
  }
}
