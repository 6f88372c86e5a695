// Streaming-read probe: the bandwidth a launch that does nothing but read a
// buffer reaches on this device, the ceiling the bandwidth-bound decode and
// rowwise kernels are measured against.  Not part of the reference's
// interface; bench.py's --stream-probe mode times it.
//
// Workgroup w reads bytes [w * B / G, (w + 1) * B / G) (16-byte aligned
// ranges) with 16-byte non-temporal loads, a ring of `kDepth` loads in flight
// per lane refilled one at a time, and folds the data into one word so the
// loads cannot be dropped; the word is stored only if it matches a value no
// input produces in practice.  Measured on MI355X against other forms of the
// same read (46 MB, 12 rotating buffers, graph replay): plain loads in
// unrolled batches of 8 reach 62 % of 8 TB/s, this ring 73 % (1024
// workgroups); torch.sum over the same bytes 10 %.

#include "lb_common.hpp"

namespace lb {
namespace probe {

constexpr int kThreads = 256;
constexpr int kDepth = 8;

__global__ __launch_bounds__(kThreads) void stream_read_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                               uint32_t* __restrict__ sink) {
  const int64_t g = gridDim.x;
  const int64_t b0 = n16 * blockIdx.x / g, b1 = n16 * (blockIdx.x + 1) / g;
  const int64_t rounds = (b1 - b0) / kThreads;  // whole rounds of the workgroup's 16-byte items
  const u32x4* s = src + b0 + threadIdx.x;
  uint32_t acc = 0;
  u32x4 v[kDepth];
  if (rounds > 0) {
#pragma unroll
  for (int d = 0; d < kDepth; ++d) v[d] = __builtin_nontemporal_load(s + min((int64_t)d, rounds - 1) * kThreads);
  int64_t r = 0;
  for (; r + 2 * kDepth <= rounds; r += kDepth) {
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
      acc ^= v[d][0] ^ v[d][1] ^ v[d][2] ^ v[d][3];
      v[d] = __builtin_nontemporal_load(s + (r + d + kDepth) * kThreads);
    }
  }
#pragma unroll
  for (int d = 0; d < kDepth; ++d) {
    if (r + d < rounds) {
      acc ^= v[d][0] ^ v[d][1] ^ v[d][2] ^ v[d][3];
      if (r + d + kDepth < rounds) v[d] = __builtin_nontemporal_load(s + (r + d + kDepth) * kThreads);
    }
  }
#pragma unroll
  for (int d = 0; d < kDepth; ++d)
    if (r + kDepth + d < rounds) acc ^= v[d][0] ^ v[d][1] ^ v[d][2] ^ v[d][3];
  }
  // the partial last round
  const int64_t tail = b0 + rounds * kThreads + threadIdx.x;
  if (tail < b1) {
    const u32x4 t = __builtin_nontemporal_load(src + tail);
    acc ^= t[0] ^ t[1] ^ t[2] ^ t[3];
  }
  if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;
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
