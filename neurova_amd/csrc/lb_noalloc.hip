// lb_marlin_gemm_noalloc: lb_marlin_gemm for callers that cannot allocate
// (code under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc).  The split-K partials live in `scratch`, a file-scope device
// array of kNoAllocScratchBytes that every GPU the library runs on holds from
// the library's load until the process ends.  Each call on a GPU shares that
// GPU's copy, which keeps the last call's contents; the kernels write every
// partial before they read it, so nothing in it has to start at zero (the
// split counters are in the caller's workspace, zero on entry as for
// lb_marlin_gemm).  Calls that overlap on one GPU (different streams) race on
// the array and must be serialised by the caller.
//
// In host code `scratch` names a host-side stand-in, not device memory: its
// device address comes from hipGetSymbolAddress, once per device with that
// device current, and only that address is passed to kernels.

#include <mutex>

#include "lb_common.hpp"
#include "marlin_run.hpp"

namespace {

// 64 MiB per GPU: the split-K partials of every decode shape of BASELINE.json
// configs[4] and of the reference's published projections (lm_head 5120 ->
// 248320 included) up to M = 64 (tests/test_plan_cpu.py checks it).
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The device that `stream` launches on (the current device for the null stream).
int stream_device(hipStream_t stream, int* dev) {
  if (stream == nullptr) return hipGetDevice(dev) == hipSuccess ? LB_OK : LB_ERR_HIP;
  return hipStreamGetDevice(stream, dev) == hipSuccess ? LB_OK : LB_ERR_HIP;
}

// Device address of `scratch` on `dev`, looked up once per device with that
// device current (the array is per device: each GPU holds its own copy).
int scratch_on(int dev, void** out) {
  if (dev < 0 || dev >= kMaxDevices) return LB_ERR_ARG;
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess) return LB_ERR_HIP;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return LB_ERR_HIP;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev && hipSetDevice(cur) != hipSuccess) return LB_ERR_HIP;
    if (e != hipSuccess || p == nullptr) return LB_ERR_HIP;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return LB_OK;
}

}  // namespace

extern "C" size_t lb_marlin_noalloc_scratch_limit(void) { return kNoAllocScratchBytes; }

extern "C" int lb_marlin_gemm_noalloc(const uint16_t* A, const int32_t* B, uint16_t* C, const uint16_t* s,
                                      int64_t prob_m, int64_t prob_n, int64_t prob_k, int32_t* workspace,
                                      int64_t workspace_len, int64_t groupsize, lb_stream_t stream) {
  hipStream_t st = (hipStream_t)stream;
  int dev = 0;
  int e = stream_device(st, &dev);
  if (e != LB_OK) return e;
  void* p = nullptr;
  e = scratch_on(dev, &p);
  if (e != LB_OK) return e;
  e = lb::marlin::run(lb::marlin::V_PLAIN, A, B, C, s, prob_m, prob_n, prob_k, workspace, workspace_len, groupsize,
                      nullptr, nullptr, p, kNoAllocScratchBytes, st);
  // run() checks the plan's partials against the bytes it is given before it
  // launches anything: a problem that needs more than the array is refused
  return e == LB_ERR_SCRATCH ? LB_ERR_NOALLOC_LIMIT : e;
}
