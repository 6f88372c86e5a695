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
//   A  -- plain A goes from global memory straight into a double-buffered LDS
//         tile by buffer-to-LDS DMA, one dword per lane, in fragment order;
//         the SiLU-gated A is loaded into registers, gated, and written to LDS.
//   B  -- each lane's four slots and the group's scales, in registers.
// The loads of stage s + 1 are issued a share per MFMA step during stage s;
// one s_waitcnt and one barrier end each stage.  The stage loop is unrolled by
// two so that buffer and slot indices are compile-time constants.
//
// Schedules.  Stream-K: as many workgroups as are resident at once each take
// an equal contiguous range of the (tile, scale group) stages in tile-major
// order, so that no CU idles through a partial last round; a tile whose
// stages span several workgroups is finished by the last of them to arrive.
// Split-tail: the first `full_tiles` workgroups each compute one tile whole
// -- as many tiles as fill every resident slot a whole number of times -- and
// the remaining tiles are split over K among `tail_splits` workgroups each.
// Either way, workgroups with part of a tile publish fp32 partials to
// scratch; the last to arrive at the tile's counter sums them in k order
// (deterministic) and finishes.

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
  int32_t* counters;     // [0] argmax arrival counter, [1 + t] counters of split tail tile t
  float* partial;        // [tail tile][split][accumulator register][thread] fp32x4
  uint32_t partial_bytes;
  uint64_t* tile_keys;   // [M][n_cg]
  int64_t* argmax_state;
  int64_t* argmax_out;
  int m, n, k;
  int grouped;
  int full_tiles;        // tiles computed whole, by workgroups 0 .. full_tiles - 1
  int tail_splits;       // the remaining tiles are split over K among this many workgroups each
  int sk_wgs;            // > 0: stream-K schedule over this many workgroups (full_tiles, tail_splits unused)
  int kp_total;
  int n_cg;
  int n_mb;
};

// Workgroups per CU each variant is compiled for (register-limited); the host
// plans the tail split with the same figures.
__host__ __device__ constexpr int wgs_per_cu(int mb, int am) { return mb >= 8 ? 2 : (am == A_SILU_PACKED ? 2 : 3); }

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

// buffer_of (lb_common.hpp): loads at or past num_records return zero; rows
// of the last M block beyond M use that.

constexpr int kSteps = 4;  // 32-k steps per stage (one scale group of 128)


// s_waitcnt vmcnt(N) as the builtin, so that the compiler's own wait
// placement knows which of its loads have completed (an assembly wait is
// opaque to it and it would wait again, for newer loads too).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is six bits");
  __builtin_amdgcn_s_waitcnt(((N & 0x30) << 10) | (N & 0xf) | (0x7 << 4) | (0xf << 8));
}


// An empty volatile asm that reads and rewrites a register value: the value
// is computed before this point and not moved past it.
template <class T>
__device__ __forceinline__ void pin_vgpr(T& x) {
  asm volatile("" : "+v"(x));
}

// SK: the stream-K schedule (p.sk_wgs workgroups), else the split-tail one.
template <int MB, int AM, int EPI, bool GROUPED, bool SK>
__global__ __launch_bounds__(kThreads, wgs_per_cu(MB, AM)) void marlin_gemm_kernel(Params p) {
  constexpr int BM = 16 * MB;
  // Plain A is staged by LDS DMA (buffer loads straight into LDS, no
  // registers); the SiLU-gated A goes through registers to be computed.
  constexpr bool kDma = AM == A_PLAIN;
  // DMA layout: one 256-byte LDS row per A row, the stage's 128 k in natural
  // order as 16 chunks of 8 halves, chunk c stored at position c ^ (r & 15)
  // (so that the 16 rows of a fragment read fall in 16 different positions:
  // no bank conflicts).  A
  // 16-byte-per-lane DMA writes four rows (1 KB) per instruction: lane L
  // writes position L & 15 of row L >> 4 and fetches the chunk that belongs
  // there.  A fragment -- A[r][32d + 16(g>>1) + 4(g&1) + {0..3}] ++ the same
  // + 8 -- is the (g&1) half of chunks 4d + 2(g>>1) and 4d + 2(g>>1) + 1: two
  // 8-byte reads.  Register layout: entry (d, g, r) at ((4d + g) * kBlk + r),
  // each (d, g) block padded by one entry so that the staging writes of one
  // row, which go to different blocks, land in different banks.
  constexpr int kRowU4 = 16;
  constexpr int kBlk = BM + 1;
  constexpr int kBufU4 = kDma ? BM * kRowU4 : kSteps * 4 * kBlk;
  // two separate arrays (not one [2][...]): the compiler's wait placement then
  // tells the buffer-to-LDS DMA into one buffer from reads of the other, and
  // waits for a DMA only before reads of the buffer it writes
  __shared__ __attribute__((aligned(16))) uint4 afr0[kBufU4];
  __shared__ __attribute__((aligned(16))) uint4 afr1[kBufU4];
  auto afr = [&](int buf) __attribute__((always_inline)) -> uint4* { return buf ? afr1 : afr0; };
  __shared__ int s_prev;
  __shared__ uint64_t s_keys[kWaves][BM];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int groups = p.kp_total >> 2;

  // One work unit: stages [st0, st0 + nst) of tile `tile`; `part`: not the
  // whole tile (`split`: its index among the tile's splits under the
  // split-tail schedule).
  auto unit = [&](const int tile_in, const int st0_in, const int nst_in, const bool part, const int split_in)
                  __attribute__((always_inline)) {
  // wave-uniform (the compiler's uniformity analysis does not follow them
  // through the lambda: without this the stage offsets go through VGPRs)
  const int tile = __builtin_amdgcn_readfirstlane(tile_in);
  const int st0 = __builtin_amdgcn_readfirstlane(st0_in);
  const int nst = __builtin_amdgcn_readfirstlane(nst_in);
  const int split = __builtin_amdgcn_readfirstlane(split_in);
  const int mb = tile / p.n_cg;
  const int cg = tile - mb * p.n_cg;
  const int m0 = mb * BM;

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
  uint4 areg[kDma ? 1 : kAPer];
  uint4 ureg[AM == A_SILU_PACKED ? kAPer : 1];
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  constexpr int kRowsPerWave = BM / kWaves;
  // DMA source of lane L in a four-row instruction: tile row b + (L >> 4), b
  // a multiple of 4, chunk (L & 15) ^ (row & 15) = ((L & 15) ^ (L >> 4)) ^
  // (b & 12).  The whole row offset is in the vector offset, which the
  // descriptor's range check covers: rows at or past M read zeros and are
  // never stored.  The stage offset (< 2K bytes) is the scalar offset.
  static_assert(kRowsPerWave % 4 == 0, "DMA row blocks");
  const uint32_t a_row_bytes = (uint32_t)p.k * 2u;
  const int lrow = lane >> 4;
  const uint32_t dma_row0 = (uint32_t)(m0 + wave_u * kRowsPerWave + lrow) * a_row_bytes;
  // rows [t0, t0 + N) of this wave's share of stage `stage` into LDS buffer `buf`
  auto dma_rows = [&](int stage, int buf, int t0, auto n) __attribute__((always_inline)) {
    static_assert(decltype(n)::value % 4 == 0, "four rows per DMA");
    char* dst = reinterpret_cast<char*>(afr(buf)) + (wave_u * kRowsPerWave + t0) * 256;
    // opaque per call, so that the per-instruction offsets are recomputed
    // (one scalar multiply and one vector add) instead of all kept live
    uint32_t rows4 = 4u * a_row_bytes;
    asm volatile("" : "+s"(rows4));
    // the lane's chunk within a block starting at row b = 0 (mod 16), recomputed per call
    const uint32_t x16 = (uint32_t)((lane & 15) ^ lrow) * 16u;
#pragma unroll
    for (int jj = 0; jj < decltype(n)::value / 4; ++jj) {  // constant trip count: fully unrolled
      const int j = t0 / 4 + jj;
      const uint32_t b12 = (uint32_t)((wave_u * kRowsPerWave + 4 * j) & 12) << 4;
      const uint32_t voff = dma_row0 + (x16 ^ b12) + (uint32_t)j * rows4;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (__attribute__((address_space(3))) void*)(dst + jj * 4 * 256), 16,
                                               voff, (uint32_t)stage * 256u, 0, 0);
    }
  };
  auto dma_a = [&](int stage, int buf) __attribute__((always_inline)) {
    dma_rows(stage, buf, 0, std::integral_constant<int, kRowsPerWave>{});
  };
  auto load_a = [&](int stage) __attribute__((always_inline)) {
    if (kDma) return;
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
  auto store_a = [&](int buf) __attribute__((always_inline)) {
    if (kDma) return;
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
      uint2* dst0 = reinterpret_cast<uint2*>(&afr(buf)[(d * 4 + 2 * pr) * kBlk + r]) + half;
      uint2* dst1 = reinterpret_cast<uint2*>(&afr(buf)[(d * 4 + 2 * pr + 1) * kBlk + r]) + half;
      *dst0 = make_uint2(w.x, w.y);
      *dst1 = make_uint2(w.z, w.w);
    }
  };

  // ---- B ring: two stages of (4 slots + the group's scales) per lane ----
  u32x4 bst[2][kSteps];
  u32x4 sst[2];
  auto load_b = [&](int slot, int stage) __attribute__((always_inline)) {
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

  // dequantise step d of B slot `slot` into four fp16 fragments: exact fp16
  // (q - 8) times the fp16 group scale, the rounding of the reference's __hmul2
  auto dequant = [&](int slot, int d, const f16x2 (&sc)[4], f16x8 (&bf)[4]) __attribute__((always_inline)) {
    const u32x4 own = bst[slot][d];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t partner = (uint32_t)__builtin_amdgcn_mov_dpp((int)own[j], 0x128, 0xf, 0xf, false);  // row_ror:8
      const uint32_t v0 = __builtin_amdgcn_perm(own[j], partner, psel);
      const uint32_t v1 = v0 >> 8;
      const f16x2 b0 = nib_lo_to_h2(v0, nk) * sc[j];
      const f16x2 b1 = nib_lo_to_h2(v1, nk) * sc[j];
      const f16x2 b2 = nib_hi_to_h2(v0, nk) * sc[j];
      const f16x2 b3 = nib_hi_to_h2(v1, nk) * sc[j];
      bf[j] = __builtin_bit_cast(f16x8, make_uint4(as_u32(b0), as_u32(b1), as_u32(b2), as_u32(b3)));
    }
  };
  auto compute = [&](int buf, int slot, auto hook) __attribute__((always_inline)) {
    f16x2 sc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t h = GROUPED ? ((sst[slot][j] >> (16 * hsel)) & 0xffffu) : 0x3c00u;  // fp16 1.0
      sc[j] = as_h2(h | (h << 16));
    }
#pragma unroll
    for (int d = 0; d < kSteps; ++d) {
      f16x8 bfrag[4];
      dequant(slot, d, sc, bfrag);
      hook(d);
      const uint4* abase = &afr(buf)[(d * 4 + g) * kBlk + (lane & 15)];
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        const f16x8 afrag = __builtin_bit_cast(f16x8, abase[16 * i]);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(afrag, bfrag[j], acc[j][i], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);  // bound the registers live across steps
    }
  };

  auto no_hook = [](int) __attribute__((always_inline)) {};

  // ---- interleaved dequant (plain A) ----
  // One step's dequant split into 8 phases of one or two VALU instructions
  // per B word, so that step d + 1's dequant can be spread over the MFMAs of
  // step d (VALU instructions between a wave's MFMAs run in their shadow),
  // one word after another:
  //   0: DPP partner, byte perm    1: >> 8, low nibbles of v0
  //   2: high of v0, low of v1     3: high of v1, bias of (lo v0)
  //   4: bias of (lo v1), (hi v0)  5: bias of (hi v1), scale (lo v0)
  //   6: scale (lo v1), (hi v0)    7: scale (hi v1)
  struct DqTmp {
    uint32_t v0[4], v1[4], lo0[4], hi0[4], lo1[4], hi1[4];
    f16x2 b[4][4];
  };
  // Each phase's results pass through an empty volatile asm: that pins them
  // to their slot (left alone, the compiler sinks the f16 arithmetic to the
  // end of the step, where it runs exposed after the last MFMA).
  auto dq_word = [&](DqTmp& q, int d, const f16x2 (&sc)[4], int ph, int j) __attribute__((always_inline)) {
    const f16x2 k1032 = {(f16)1032.0f, (f16)1032.0f};
    const f16x2 k16 = {(f16)0.0625f, (f16)0.0625f}, k72 = {(f16)-72.0f, (f16)-72.0f};
    switch (ph) {
      case 0: {
        const uint32_t own = bst[0][d][j];
        const uint32_t partner = (uint32_t)__builtin_amdgcn_mov_dpp((int)own, 0x128, 0xf, 0xf, false);  // row_ror:8
        q.v0[j] = __builtin_amdgcn_perm(own, partner, psel);
        pin_vgpr(q.v0[j]);
        break;
      }
      case 1:
        q.v1[j] = q.v0[j] >> 8;
        q.lo0[j] = and_or(q.v0[j], nk.lo_mask, nk.magic);
        pin_vgpr(q.v1[j]);
        pin_vgpr(q.lo0[j]);
        break;
      case 2:
        q.hi0[j] = and_or(q.v0[j], nk.hi_mask, nk.magic);
        q.lo1[j] = and_or(q.v1[j], nk.lo_mask, nk.magic);
        pin_vgpr(q.hi0[j]);
        pin_vgpr(q.lo1[j]);
        break;
      case 3:
        q.hi1[j] = and_or(q.v1[j], nk.hi_mask, nk.magic);
        q.b[j][0] = as_h2(q.lo0[j]) - k1032;
        pin_vgpr(q.hi1[j]);
        pin_vgpr(q.b[j][0]);
        break;
      case 4:
        q.b[j][1] = as_h2(q.lo1[j]) - k1032;
        q.b[j][2] = as_h2(q.hi0[j]) * k16 + k72;
        pin_vgpr(q.b[j][1]);
        pin_vgpr(q.b[j][2]);
        break;
      case 5:
        q.b[j][3] = as_h2(q.hi1[j]) * k16 + k72;
        q.b[j][0] = q.b[j][0] * sc[j];
        pin_vgpr(q.b[j][3]);
        pin_vgpr(q.b[j][0]);
        break;
      case 6:
        q.b[j][1] = q.b[j][1] * sc[j];
        q.b[j][2] = q.b[j][2] * sc[j];
        pin_vgpr(q.b[j][1]);
        pin_vgpr(q.b[j][2]);
        break;
      default:
        q.b[j][3] = q.b[j][3] * sc[j];
        pin_vgpr(q.b[j][3]);
        break;
    }
  };
  auto dq_pack = [&](const DqTmp& q, f16x8 (&bf)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      bf[j] = __builtin_bit_cast(f16x8, make_uint4(as_u32(q.b[j][0]), as_u32(q.b[j][1]), as_u32(q.b[j][2]),
                                                   as_u32(q.b[j][3])));
  };
  // A fragment (d, g) of row 16i + r, r = lane & 15: the (g&1) halves of
  // chunks c = 4d + 2(g>>1) and c + 1, stored at positions c ^ r and
  // (c ^ r) ^ 1 (c is even).  c ^ r = 4(d ^ (r >> 2)) + ((2(g>>1) ^ r) & 3),
  // so step d's byte offset is a per-lane base XOR 64d (bits 6-7, which the
  // rest of the base leaves clear), plus 4096 i; the chunk + 1 half is at the
  // offset XOR 16.
  const uint32_t a_off0 = (uint32_t)((lane & 15) * 256 + 8 * (g & 1) + 64 * ((lane & 15) >> 2) +
                                     16 * ((2 * (g >> 1) ^ lane) & 3));
  // The group scales of the stage whose B slots are in registers, as f16x2.
  auto scales_of = [&](f16x2 (&sc)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t h = GROUPED ? ((sst[0][j] >> (16 * hsel)) & 0xffffu) : 0x3c00u;  // fp16 1.0
      sc[j] = as_h2(h | (h << 16));
    }
  };
  // Step 0 of the first stage, dequantised up front (every later stage's step
  // 0 is dequantised during the previous stage's last step).
  auto dequant_first = [&](const f16x2 (&sc)[4], f16x8 (&bcur)[4]) __attribute__((always_inline)) {
    DqTmp q;
#pragma unroll
    for (int ph = 0; ph < 8; ++ph)
#pragma unroll
      for (int j = 0; j < 4; ++j) dq_word(q, 0, sc, ph, j);
    dq_pack(q, bcur);
  };
  // One stage of plain-A compute.  On entry `bcur` holds step 0's B
  // fragments and `sc` the stage's scales.  Step d's MFMAs (row block i's A
  // fragment read two blocks ahead) each carry a share of the dequant of step
  // d + 1 -- for the last step, of the next stage's step 0, whose slot and
  // scales were loaded by hook(0) -- so that no dequant runs outside the
  // MFMAs' shadow.  `hook(d)` issues loads once step d's slot has been
  // dequantised: hook(0) at the top of the stage, after its first A reads.
  auto compute_interleaved = [&](int buf, auto hook, f16x2 (&sc)[4], f16x8 (&bcur)[4])
      __attribute__((always_inline)) {
    // 32 (word, phase) pairs per step, spread over the 4*MB MFMA slots word
    // by word (a word's phases are dependent, one slot apart at least; one
    // word's temporaries live at a time)
    constexpr int kPhPerSlot = 8 / MB > 0 ? 8 / MB : 1;
    // steps as compile-time constants (a plain loop over d is not always
    // unrolled, and a runtime d would index the B registers dynamically)
    auto step = [&](auto dc) __attribute__((always_inline)) {
      constexpr int d = decltype(dc)::value;
      constexpr int dn = (d + 1) % kSteps;  // slot dequantised during this step
      const char* abuf = reinterpret_cast<const char*>(afr(buf));
      // recomputed per step (two XORs) rather than eight offsets kept live
      uint32_t off_base = a_off0;
      pin_vgpr(off_base);
      const uint32_t off_lo = off_base ^ (uint32_t)(64 * d), off_hi = off_lo ^ 16u;
      auto read_a = [&](int i) __attribute__((always_inline)) {
        const int o = i * 16 * 256;
        const uint2 lo = *reinterpret_cast<const uint2*>(abuf + off_lo + o);
        const uint2 hi = *reinterpret_cast<const uint2*>(abuf + off_hi + o);
        // keeps one block's reads from merging with the next block's into a
        // two-address read (whose halves land interleaved: register moves)
        asm volatile("" ::: "memory");
        return __builtin_bit_cast(f16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
      };
      DqTmp q;
      f16x8 ar[MB];
      ar[0] = read_a(0);
      if (MB > 1) ar[1] = read_a(1);
      if (d == 0) hook(0);
      if (d == kSteps - 1) scales_of(sc);  // the next stage's
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        if (i + 2 < MB) ar[i + 2] = read_a(i + 2);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ar[i], bcur[j], acc[j][i], 0, 0, 0);
#pragma unroll
          for (int t = 0; t < kPhPerSlot; ++t) {
            const int pw = (i * 4 + j) * kPhPerSlot + t;
            if (pw < 32) dq_word(q, dn, sc, pw & 7, pw >> 3);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      dq_pack(q, bcur);
      if (d + 1 < kSteps) hook(d + 1);
      __builtin_amdgcn_sched_barrier(0);
    };
    static_assert(kSteps == 4, "four MFMA steps per stage");
    step(std::integral_constant<int, 0>{});
    step(std::integral_constant<int, 1>{});
    step(std::integral_constant<int, 2>{});
    step(std::integral_constant<int, 3>{});
  };

  // ---- pipeline (DMA A): the loads of stage s + 1 are issued during stage
  // s -- A into the LDS buffer stage s - 1 used, each B slot into the
  // registers of the slot just dequantised.  A, the scales and B slots 0 and
  // 1 land before the barrier that ends stage s; slots 2 and 3 are waited for
  // where stage s + 1 dequantises them ----
  if (kDma && nst > 0) {
    dma_a(st0, 0);
    load_b(0, st0);
    wait_vmcnt<0>();
    __syncthreads();
    f16x2 sc[4];
    f16x8 bcur[4];
    scales_of(sc);
    dequant_first(sc, bcur);
    // Every stage issues the next stage's loads -- the last one re-reads its
    // own stage into the buffer and registers nobody reads afterwards -- so
    // that the loop body has no load-skipping branches and the compiler's
    // wait placement stays exact.
    auto stage = [&](int s, auto par) __attribute__((always_inline)) {
      constexpr int c = decltype(par)::value;
      const int nx = st0 + (s + 1 < nst ? s + 1 : s);
      // issue order: scale, B slot 0, A rows 0 .. R/2 (top of the stage);
      // B slot 1, A rows R/2 .. R (after step 1's dequant); B slots 2, 3.
      // Slot 0 and the scales are dequantised in step 3, slots 1 .. 3 in
      // steps 0 .. 2 of the next stage.
      auto hook = [&](int d) __attribute__((always_inline)) {
        if (GROUPED && d == 0)
          sst[0] = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, s_off, (uint32_t)nx * (uint32_t)p.n * 2u, 0));
        // step d's B slot is reloaded with stage s + 1's right after its
        // dequant, so one set of B registers serves both stages
        bst[0][d] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, b_off, (uint32_t)(nx * 8 + 2 * d) * row_bytes, 0));
        static_assert(kRowsPerWave % 2 == 0, "rows per half");
        if (d < 2) dma_rows(nx, c ^ 1, d * (kRowsPerWave / 2), std::integral_constant<int, kRowsPerWave / 2>{});
      };
      compute_interleaved(c, hook, sc, bcur);
      // everything but B slots 2 and 3 of stage s + 1 has landed: this
      // wave's A rows of buffer c ^ 1 among them; the barrier makes every
      // wave's rows visible and retires buffer c
      wait_vmcnt<2>();
      __syncthreads();
    };
    int s = 0;
    for (; s + 1 < nst; s += 2) {
      stage(s, std::integral_constant<int, 0>{});
      stage(s + 1, std::integral_constant<int, 1>{});
    }
    if (s < nst) stage(s, std::integral_constant<int, 0>{});
    // the last stage's extra DMA must land before the workgroup's LDS is released
    wait_vmcnt<0>();
  }
  // ---- pipeline (register A): A one stage ahead, B two stages ahead ----
  if (!kDma && nst > 0) {
    load_a(st0);
    load_b(0, st0);
    if (nst > 1) load_b(1, st0 + 1);
    store_a(0);
    __syncthreads();
    if (nst > 1) load_a(st0 + 1);
    // Stage s uses LDS buffer and B slot s & 1; unrolled by two so that both
    // are compile-time constants (no indexed register access).
    auto stage = [&](int s, auto par) __attribute__((always_inline)) {
      constexpr int c = decltype(par)::value;
      compute(c, c, no_hook);
      if (s + 2 < nst) load_b(c, st0 + s + 2);
      if (s + 1 < nst) store_a(c ^ 1);  // buffer c ^ 1 was last read in stage s - 1
      __syncthreads();
      if (s + 2 < nst) load_a(st0 + s + 2);
    };
    // pairs of stages, then an odd last one: no exit from the middle of the
    // loop body, so the compiler's wait placement sees one state per edge
    int s = 0;
    for (; s + 1 < nst; s += 2) {
      stage(s, std::integral_constant<int, 0>{});
      stage(s + 1, std::integral_constant<int, 1>{});
    }
    if (s < nst) stage(s, std::integral_constant<int, 0>{});
  }

  // ---- epilogue ----
  // acc[j][i][e] = C[m0 + 16i + 4*(lane>>4) + e][chunk*64 + 16j + (lane&15)]
  const int rbase = m0 + 4 * (lane >> 4);
  const int ccol = chunk * 64 + (lane & 15);

  if (part) {
    // A tile computed in parts.  Its contributors, in k order: `narr`
    // workgroups, this one at position `own`.  Split-tail schedule: tail tile
    // t's splits, partial slots t * S + split.  Stream-K: workgroup i owns two
    // partial slots, 2i for the segment its range begins with and 2i + 1 for
    // the one it ends with; a tile's contributors are consecutive workgroups
    // i0 .. i1, where only i0 can reach the tile with its ending segment.
    constexpr int kQ = 4 * MB;
    constexpr uint32_t kRegBytes = kThreads * 16u;
    int narr, own, ctr_idx, slot_base, first_alt = 0;
    if constexpr (SK) {
      const int64_t work = (int64_t)p.n_cg * p.n_mb * groups, wgs = p.sk_wgs;
      const int64_t ts = (int64_t)tile * groups;
      // the workgroup whose range holds stage s: the last i with i * work / wgs <= s
      const int64_t i0 = ((ts + 1) * wgs - 1) / work;
      const int64_t i1 = ((ts + groups) * wgs - 1) / work;
      narr = (int)(i1 - i0 + 1);
      own = (int)(blockIdx.x - i0);
      first_alt = (i0 * work / wgs) < ts ? 1 : 0;
      slot_base = 2 * (int)i0;
      ctr_idx = 1 + tile;
    } else {
      narr = p.tail_splits;
      own = split;
      slot_base = (tile - p.full_tiles) * narr;
      ctr_idx = 1 + tile - p.full_tiles;
    }
    // partial slot of contributor sp
    auto slot_of = [&](int sp) __attribute__((always_inline)) -> uint32_t {
      return SK ? (uint32_t)(slot_base + 2 * sp + (sp == 0 ? first_alt : 0)) : (uint32_t)(slot_base + sp);
    };
    const __amdgpu_buffer_rsrc_t rp = buffer_of(p.partial, p.partial_bytes);
    const uint32_t lane_off = (uint32_t)tid * 16u;
    const uint32_t own_off = slot_of(own) * (uint32_t)kQ * kRegBytes + lane_off;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < MB; ++i)
        publish16(rp, own_off + (uint32_t)(j * MB + i) * kRegBytes, acc[j][i]);
    wait_published();
    __syncthreads();
    int32_t* ctr = p.counters + ctr_idx;
    if (tid == 0) s_prev = arrive(ctr);
    __syncthreads();
    if (s_prev != narr - 1) return;
    after_last_arrival();
    // The last arrival sums the splits in split order, one column block of
    // MB registers at a time.  Tiles below 128 rows: it reads its own split
    // back with the others, so that its registers are free for the loads, and
    // issues the loads of up to kCollect splits of a block together: a block
    // costs one memory round trip per kCollect splits instead of one per split
    // (M = 64, K = 17408, N = 5120: 37.5 -> 34.7 us).  128-row tiles keep one
    // split per round trip, their own from registers: there the batched form
    // measured 1-2 % slower over the whole launch.  Both sum the same values
    // in split order.
    constexpr bool kReload = MB < 8;
    constexpr int kCollect = 3;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f32x4 sum[MB];
#pragma unroll
      for (int i = 0; i < MB; ++i) sum[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
      if constexpr (kReload) {
        for (int sp0 = 0; sp0 < narr; sp0 += kCollect) {
          f32x4 v[kCollect][MB];
#pragma unroll
          for (int u = 0; u < kCollect; ++u)
            if (sp0 + u < narr) {
              const uint32_t off = slot_of(sp0 + u) * (uint32_t)kQ * kRegBytes + lane_off;
#pragma unroll
              for (int i = 0; i < MB; ++i) v[u][i] = collect16(rp, off + (uint32_t)(j * MB + i) * kRegBytes);
            }
#pragma unroll
          for (int u = 0; u < kCollect; ++u)
            if (sp0 + u < narr) {
#pragma unroll
              for (int i = 0; i < MB; ++i) sum[i] += v[u][i];
            }
        }
      } else {
        for (int sp = 0; sp < narr; ++sp) {
          if (sp == own) {
#pragma unroll
            for (int i = 0; i < MB; ++i) sum[i] += acc[j][i];
          } else {
            const uint32_t off = slot_of(sp) * (uint32_t)kQ * kRegBytes + lane_off;
            f32x4 v[MB];
#pragma unroll
            for (int i = 0; i < MB; ++i) v[i] = collect16(rp, off + (uint32_t)(j * MB + i) * kRegBytes);
#pragma unroll
            for (int i = 0; i < MB; ++i) sum[i] += v[i];
          }
        }
      }
#pragma unroll
      for (int i = 0; i < MB; ++i) acc[j][i] = sum[i];
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
  after_last_arrival();
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
  };

  if constexpr (SK) {
    // Stream-K: workgroup i takes stages [i * W / P, (i + 1) * W / P) of the
    // W = tiles x groups stages in tile-major order, P = sk_wgs (every
    // workgroup resident at once), and runs them tile segment by segment.
    const int64_t work = (int64_t)p.n_cg * p.n_mb * groups;
    const int64_t w1 = work * (blockIdx.x + 1) / p.sk_wgs;
    for (int64_t w = work * blockIdx.x / p.sk_wgs; w < w1;) {
      const int tile = (int)(w / groups);
      const int st0 = (int)(w - (int64_t)tile * groups);
      const int nst = (int)(w1 - w < (int64_t)(groups - st0) ? w1 - w : (int64_t)(groups - st0));
      unit(tile, st0, nst, nst != groups, 0);
      w += nst;
    }
  } else {
  // Split-tail schedule.  When every tile is split over K, each XCD
  // (workgroups go to the 8 XCDs round-robin) takes a contiguous range of
  // work units: a tile's splits and its neighbours share A rows and B columns
  // in that XCD's L2 (measured 2-3 % faster there; slower by 10 % where whole
  // tiles dominate, which keep the plain order).
  int bid = blockIdx.x;
  if (p.full_tiles == 0) {
    const int w8 = (int)gridDim.x & ~7;
    if (bid < w8) bid = (bid & 7) * (w8 >> 3) + (bid >> 3);
  }
  int tile = bid, split = 0, nsplit = 1;
  if (bid >= p.full_tiles) {
    nsplit = p.tail_splits;
    const int u = bid - p.full_tiles;
    tile = p.full_tiles + u / nsplit;
    split = u - (u / nsplit) * nsplit;
  }
  const int st0 = (int)(((int64_t)groups * split) / nsplit);           // first scale group (stage)
  const int nst = (int)(((int64_t)groups * (split + 1)) / nsplit) - st0;  // stages of this unit
  unit(tile, st0, nst, nsplit > 1, split);
  }
}

}  // namespace gemm
}  // namespace lb
