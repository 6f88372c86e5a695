// Shared device/host helpers for the gfx950 low-bit projection kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/langburst_lowbit.h"

namespace lb {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ __forceinline__ f16x2 as_h2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }
__device__ __forceinline__ uint32_t as_u32(f16x2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(f16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (f16)f); }

// Two 4-bit codes sitting in bits [0,4) and [16,20) of `w` (after masking) become
// the fp16 pair (code - 8): OR-ing the exponent of 1024 turns the nibble into the
// mantissa of 1024 + code; subtracting 1032 is exact.  Codes in bits [4,8) and
// [20,24) give 1024 + 16*code, scaled by 1/16 and offset by -72 with one exact fma.
// The mask-and-OR is a single v_and_or_b32 (mask in an SGPR, the exponent
// pattern in a VGPR: gfx9 VOP3 takes no literals and one scalar operand).
__device__ __forceinline__ uint32_t and_or(uint32_t w, uint32_t smask, uint32_t vbits) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(w), "s"(smask), "v"(vbits));
  return r;
}
struct NibConsts {
  uint32_t lo_mask, hi_mask;  // SGPR
  uint32_t magic;             // VGPR 0x64006400
};
__device__ __forceinline__ NibConsts nib_consts() {
  NibConsts c;
  asm("s_mov_b32 %0, 0x000f000f" : "=s"(c.lo_mask));
  asm("s_mov_b32 %0, 0x00f000f0" : "=s"(c.hi_mask));
  asm("v_mov_b32 %0, 0x64006400" : "=v"(c.magic));
  return c;
}
__device__ __forceinline__ f16x2 nib_lo_to_h2(uint32_t w, const NibConsts& k) {
  return as_h2(and_or(w, k.lo_mask, k.magic)) - (f16x2){(f16)1032.0f, (f16)1032.0f};
}
__device__ __forceinline__ f16x2 nib_hi_to_h2(uint32_t w, const NibConsts& k) {
  return as_h2(and_or(w, k.hi_mask, k.magic)) * (f16x2){(f16)0.0625f, (f16)0.0625f} + (f16x2){(f16)-72.0f, (f16)-72.0f};
}
// Biased forms: 1024 + code (bits [0,4) / [16,20)) and 1024 + 16*code
// (bits [4,8) / [20,24)), one v_and_or_b32 each; the caller removes the bias.
__device__ __forceinline__ f16x2 nib_lo_biased(uint32_t w, const NibConsts& k) {
  return as_h2(and_or(w, k.lo_mask, k.magic));
}
__device__ __forceinline__ f16x2 nib_hi_biased(uint32_t w, const NibConsts& k) {
  return as_h2(and_or(w, k.hi_mask, k.magic));
}
__device__ __forceinline__ f16x2 nib_lo_to_h2(uint32_t w) {
  const uint32_t v = (w & 0x000f000fu) | 0x64006400u;
  return as_h2(v) - (f16x2){(f16)1032.0f, (f16)1032.0f};
}
__device__ __forceinline__ f16x2 nib_hi_to_h2(uint32_t w) {
  const uint32_t v = (w & 0x00f000f0u) | 0x64006400u;
  return as_h2(v) * (f16x2){(f16)0.0625f, (f16)0.0625f} + (f16x2){(f16)-72.0f, (f16)-72.0f};
}

// Sum over the 4 lanes of a quad (xor 1, xor 2) with DPP.
__device__ __forceinline__ float quad_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xb1, 0xf, 0xf, false));  // [1,0,3,2]
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4e, 0xf, 0xf, false));  // [2,3,0,1]
  return v;
}

// Full-wave sum; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
  v = quad_sum(v);
  v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x101f));  // xor 4
  v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x201f));  // xor 8
  v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401f));  // xor 16
  const int lane = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  return v + __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, __builtin_bit_cast(int, v)));
}

// Cross-workgroup hand-off without cache-wide fences.
//
// A device-scope release/acquire fence costs an L2 write-back / invalidate on
// every XCD (buffer_wbl2 / buffer_inv).  Those exist for ordinary accesses;
// here every word that crosses workgroups is itself a device-scope atomic
// access: relaxed agent-scope atomic stores and loads, which gfx950 performs
// as stores/loads with the device-coherence bit (sc1) at full store/load
// bandwidth.  A workgroup publishes its partials with such stores, waits until
// they are acknowledged (vmcnt counts stores on gfx9), and only then counts
// its arrival with an atomic add (a read-modify-write, always performed at
// device scope); the workgroup that observes the final count reads the
// partials with device-scope atomic loads and resets the counter with an
// atomic swap whose return it also waits for, so the next launch starts from
// zero.
__device__ __forceinline__ void publish(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void publish(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void publish(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float collect(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t collect(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Raw buffer resource (gfx9 V#: stride 0, 32-bit data format); loads at or
// past num_records return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// The same device-coherent (sc1) stores and loads, sixteen bytes at a time
// through a buffer resource (cache-policy operand 16 = sc1 on gfx950), for
// hand-offs of whole accumulator registers.
constexpr int kSc1 = 16;
// Cache-policy operand 2 = nt on gfx950: data read once (weights, scales).
constexpr int kNonTemporal = 2;
__device__ __forceinline__ void publish16(__amdgpu_buffer_rsrc_t r, uint32_t off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, kSc1);
}
__device__ __forceinline__ f32x4 collect16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kSc1));
}

// Workgroup barrier for LDS data only: waits for this wave's LDS operations,
// not for its outstanding global loads (__syncthreads' fence would also wait
// for every in-flight vector-memory load, e.g. a prefetch ring).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Waits until every vector-memory operation this thread issued (loads,
// stores, atomics) has been acknowledged; the memory clobber keeps the
// compiler from moving memory accesses across it.
__device__ __forceinline__ void wait_published() { asm volatile("s_waitcnt vmcnt(0)" : : : "memory"); }

// Counts this workgroup's arrival on `counter`; returns the count before it.
__device__ __forceinline__ int arrive(int* counter) {
  return __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Entry of a collect path, right after the branch on an arrival count: no
// memory access of the collect may be moved above it (the partials are read
// only once the count shows every split published; the hardware issues them
// after the branch that needs the count).
__device__ __forceinline__ void after_last_arrival() { asm volatile("" ::: "memory"); }

// Zeroes a counter and waits for the swap to be performed.
__device__ __forceinline__ void reset_counter(int* counter) {
  const int old = __hip_atomic_exchange(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("s_waitcnt vmcnt(0)" : : "v"(old) : "memory");
}

}  // namespace lb

// Host-side helpers shared by the C-ABI translation units.
namespace lbh {

inline int launch_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? LB_OK : LB_ERR_HIP;
}

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// Compute units of the current device (cached per device; 256 on a full MI355X,
// fewer in a compute-partitioned mode).
inline int device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = __atomic_load_n(&cache[dev], __ATOMIC_RELAXED);
  if (v <= 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    __atomic_store_n(&cache[dev], v, __ATOMIC_RELAXED);
  }
  return v;
}

}  // namespace lbh
