// Streaming-read probe: the bandwidth a launch that does nothing but read a
// buffer reaches on this device, the ceiling the bandwidth-bound decode and
// rowwise kernels are measured against.  Not part of the reference's
// interface; bench.py's --stream-probe mode times it.
//
// Workgroup w reads bytes [w * B / G, (w + 1) * B / G) (16-byte aligned
// ranges) with 16-byte loads, `depth` loads in flight per lane, and folds the
// data into one word so the loads cannot be dropped; lane 0 stores the word.

#include "lb_common.hpp"

namespace lb {
namespace probe {

constexpr int kThreads = 256;
constexpr int kDepth = 8;

__global__ __launch_bounds__(kThreads) void stream_read_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                               uint32_t* __restrict__ sink) {
  const int64_t g = gridDim.x;
  const int64_t b0 = n16 * blockIdx.x / g, b1 = n16 * (blockIdx.x + 1) / g;
  uint32_t acc = 0;
  int64_t i = b0 + threadIdx.x;
  for (; i + (kDepth - 1) * kThreads < b1; i += kDepth * kThreads) {
    u32x4 v[kDepth];
#pragma unroll
    for (int d = 0; d < kDepth; ++d) v[d] = src[i + d * kThreads];
#pragma unroll
    for (int d = 0; d < kDepth; ++d) acc ^= v[d][0] ^ v[d][1] ^ v[d][2] ^ v[d][3];
  }
  for (; i < b1; i += kThreads) {
    const u32x4 v = src[i];
    acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  acc = (uint32_t)__builtin_bit_cast(int, wave_sum(__builtin_bit_cast(float, acc & 0x7fffffu)));
  if ((threadIdx.x & 63) == 0) sink[blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6)] = acc;
}

}  // namespace probe
}  // namespace lb

extern "C" int lb_probe_stream_read(const void* src, size_t bytes, uint32_t* sink, int32_t workgroups,
                                    lb_stream_t stream) {
  if (!src || !sink || workgroups <= 0 || bytes % 16 != 0) return LB_ERR_ARG;
  if (!lbh::aligned(src, 16)) return LB_ERR_ALIGN;
  if (bytes == 0) return LB_OK;
  hipLaunchKernelGGL(lb::probe::stream_read_kernel, dim3((unsigned)workgroups), dim3(lb::probe::kThreads), 0,
                     (hipStream_t)stream, reinterpret_cast<const lb::u32x4*>(src), (int64_t)(bytes / 16), sink);
  return lbh::launch_status();
}
