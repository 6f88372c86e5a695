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

// Device-scope (all XCDs) release of this workgroup's global writes followed by
// an arrival count on `counter`; returns the count before this arrival.
// Call from one thread after a __syncthreads() that follows the writes.
__device__ __forceinline__ int arrive_release(int* counter) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  return __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Device-scope acquire: later loads observe writes released by other workgroups.
__device__ __forceinline__ void acquire_device() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent"); }

}  // namespace lb

// Host-side helpers shared by the C-ABI translation units.
namespace lbh {

inline int launch_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? LB_OK : LB_ERR_HIP;
}

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace lbh
