// Python module `langburst_cuda` for the MI355X build: the hot-path ops of the
// reference's extension (langburst/csrc/langburst_ext.cpp:259-344) with the
// same names, argument order, keyword names, defaults, dtypes, shapes and
// error messages, implemented as thin wrappers over the C ABI in
// include/langburst_lowbit.h.  Tensors are launched on the caller's current
// HIP stream; nothing here synchronises.
//
// Only the low-bit projection ops are provided; the reference module's other
// ops (RMSNorm, GDN, attention, sampling) are outside this library.

#include <torch/extension.h>
#include <c10/hip/HIPStream.h>
#include <c10/core/DeviceGuard.h>

#include <hip/hip_runtime_api.h>

#include <cstdlib>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "../../include/langburst_lowbit.h"

namespace py = pybind11;

#define LB_CHECK_DEV(x) TORCH_CHECK((x).is_cuda(), #x " must be CUDA")
#define LB_CHECK_CONTIG(x) TORCH_CHECK((x).is_contiguous(), #x " must be contiguous")
#define LB_CHECK_HALF(x) TORCH_CHECK((x).scalar_type() == at::kHalf, #x " must be fp16")
#define LB_CHECK_FLOAT(x) TORCH_CHECK((x).scalar_type() == at::kFloat, #x " must be fp32")
#define LB_CHECK_U8(x) TORCH_CHECK((x).scalar_type() == at::kByte, #x " must be uint8")
#define LB_CHECK_I64(x) TORCH_CHECK((x).scalar_type() == at::kLong, #x " must be int64")

namespace {

inline lb_stream_t stream_of(const torch::Tensor& t) {
  return reinterpret_cast<lb_stream_t>(c10::hip::getCurrentHIPStream(t.get_device()).stream());
}

inline const uint16_t* h16(const torch::Tensor& t) { return reinterpret_cast<const uint16_t*>(t.data_ptr()); }
inline uint16_t* h16m(const torch::Tensor& t) { return reinterpret_cast<uint16_t*>(t.data_ptr()); }

inline void lb_ok(int status, const char* what) {
  TORCH_CHECK(status == LB_OK, what, " failed with code ", status, " (", lb_status_string(status), ")");
}

// ---------------------------------------------------------------- rowwise ---

void check_lowbit_args(const torch::Tensor& qweight, const torch::Tensor& scales, int64_t cols, int64_t group_size,
                       int64_t bits) {
  LB_CHECK_DEV(qweight); LB_CHECK_DEV(scales);
  LB_CHECK_CONTIG(qweight); LB_CHECK_CONTIG(scales);
  LB_CHECK_U8(qweight); LB_CHECK_HALF(scales);
  TORCH_CHECK(qweight.dim() == 2, "qweight must be [rows, packed_cols]");
  TORCH_CHECK(scales.dim() == 2, "scales must be [rows, n_groups]");
  TORCH_CHECK(cols > 0 && group_size > 0, "cols and group_size must be positive");
  TORCH_CHECK(bits >= 2 && bits <= 8, "bits must be in [2, 8]");
  const int64_t n_groups = (cols + group_size - 1) / group_size;
  const int64_t packed_need = (cols * bits + 7) / 8;
  TORCH_CHECK(scales.size(0) == qweight.size(0), "scales rows mismatch");
  TORCH_CHECK(scales.size(1) >= n_groups, "scales group count too small");
  TORCH_CHECK(qweight.size(1) >= packed_need, "qweight packed_cols too small");
}

void check_rows_per_cta(int64_t rows_per_cta) {
  TORCH_CHECK(rows_per_cta == 4 || rows_per_cta == 8 || rows_per_cta == 16, "rows_per_cta must be one of 4, 8, 16");
}

torch::Tensor lowbit_gemv(torch::Tensor qweight, torch::Tensor scales, torch::Tensor x, int64_t cols,
                          int64_t group_size, int64_t bits, int64_t rows_per_cta) {
  check_lowbit_args(qweight, scales, cols, group_size, bits);
  check_rows_per_cta(rows_per_cta);
  LB_CHECK_DEV(x); LB_CHECK_CONTIG(x); LB_CHECK_HALF(x);
  TORCH_CHECK(x.dim() == 1, "x must be [cols]");
  TORCH_CHECK(x.size(0) >= cols, "x cols mismatch");
  const c10::DeviceGuard guard(x.device());
  auto y = torch::empty({qweight.size(0)}, x.options());
  lb_ok(lb_lowbit_gemv(qweight.data_ptr<uint8_t>(), qweight.size(0), qweight.size(1), h16(scales), scales.size(1),
                       h16(x), h16m(y), cols, group_size, bits, rows_per_cta, stream_of(x)),
        "lowbit_gemv");
  return y;
}

std::vector<torch::Tensor> lowbit_gemv_pair(torch::Tensor qweight_a, torch::Tensor scales_a, torch::Tensor qweight_b,
                                            torch::Tensor scales_b, torch::Tensor x, int64_t cols, int64_t group_size,
                                            int64_t bits, int64_t rows_per_cta) {
  check_lowbit_args(qweight_a, scales_a, cols, group_size, bits);
  check_lowbit_args(qweight_b, scales_b, cols, group_size, bits);
  check_rows_per_cta(rows_per_cta);
  LB_CHECK_DEV(x); LB_CHECK_CONTIG(x); LB_CHECK_HALF(x);
  TORCH_CHECK(qweight_a.sizes() == qweight_b.sizes(), "pair qweight shapes must match");
  TORCH_CHECK(scales_a.sizes() == scales_b.sizes(), "pair scale shapes must match");
  TORCH_CHECK(x.dim() == 1, "x must be [cols]");
  TORCH_CHECK(x.size(0) >= cols, "x cols mismatch");
  const c10::DeviceGuard guard(x.device());
  auto ya = torch::empty({qweight_a.size(0)}, x.options());
  auto yb = torch::empty({qweight_a.size(0)}, x.options());
  lb_ok(lb_lowbit_gemv_pair(qweight_a.data_ptr<uint8_t>(), h16(scales_a), qweight_b.data_ptr<uint8_t>(), h16(scales_b),
                            qweight_a.size(0), qweight_a.size(1), scales_a.size(1), h16(x), h16m(ya), h16m(yb), cols,
                            group_size, bits, rows_per_cta, stream_of(x)),
        "lowbit_gemv_pair");
  return {ya, yb};
}

torch::Tensor lowbit_gemm(torch::Tensor qweight, torch::Tensor scales, torch::Tensor x, int64_t cols,
                          int64_t group_size, int64_t bits, int64_t rows_per_cta) {
  check_lowbit_args(qweight, scales, cols, group_size, bits);
  check_rows_per_cta(rows_per_cta);
  LB_CHECK_DEV(x); LB_CHECK_CONTIG(x); LB_CHECK_HALF(x);
  TORCH_CHECK(x.dim() == 2, "x must be [batch, cols]");
  TORCH_CHECK(x.size(1) >= cols, "x cols mismatch");
  const c10::DeviceGuard guard(x.device());
  auto y = torch::empty({x.size(0), qweight.size(0)}, x.options());
  lb_ok(lb_lowbit_gemm(qweight.data_ptr<uint8_t>(), qweight.size(0), qweight.size(1), h16(scales), scales.size(1),
                       h16(x), x.size(0), x.size(1), h16m(y), cols, group_size, bits, rows_per_cta, stream_of(x)),
        "lowbit_gemm");
  return y;
}

torch::Tensor lowbit_row_dequant(torch::Tensor qweight, torch::Tensor scales, torch::Tensor row, int64_t cols,
                                 int64_t group_size, int64_t bits) {
  check_lowbit_args(qweight, scales, cols, group_size, bits);
  LB_CHECK_DEV(row); LB_CHECK_CONTIG(row); LB_CHECK_I64(row);
  TORCH_CHECK(row.numel() == 1, "row must be scalar int64 tensor");
  const c10::DeviceGuard guard(scales.device());
  auto out = torch::empty({cols}, scales.options());
  lb_ok(lb_lowbit_row_dequant(qweight.data_ptr<uint8_t>(), qweight.size(0), qweight.size(1), h16(scales),
                              scales.size(1), row.data_ptr<int64_t>(), h16m(out), cols, group_size, bits,
                              stream_of(scales)),
        "lowbit_row_dequant");
  return out;
}

// ----------------------------------------------------------------- marlin ---

int marlin_max_par() {
  int max_par = 16;
  if (const char* env = std::getenv("LANGBURST_MARLIN_MAX_PAR")) max_par = std::atoi(env);
  TORCH_CHECK(max_par >= 1 && max_par <= 16, "LANGBURST_MARLIN_MAX_PAR must be in [1, 16]");
  return max_par;
}

// Shared shape checks of the Marlin ops; returns (M, N, normalised group).
struct MarlinShape {
  int64_t m, n, k, group;
};

MarlinShape check_marlin_common(const torch::Tensor& qweight, const torch::Tensor& scales, const torch::Tensor& out,
                                const torch::Tensor& workspace, int64_t prob_m, int64_t cols, int64_t group_size,
                                const char* out_name) {
  TORCH_CHECK(cols % 128 == 0, "Marlin requires K divisible by 128");
  const int64_t prob_k = cols;
  TORCH_CHECK(qweight.dim() == 2 && qweight.size(0) == prob_k / 16, "marlin qweight must be [K/16, N*2]");
  TORCH_CHECK(qweight.size(1) % 2 == 0, "marlin qweight second dim must be N*2");
  const int64_t prob_n = qweight.size(1) / 2;
  TORCH_CHECK(prob_n % 256 == 0, "Marlin requires N divisible by 256");
  TORCH_CHECK(scales.dim() == 2 && scales.size(1) == prob_n, "marlin scales must be [K/group, N]");
  TORCH_CHECK(out.dim() == 2 && out.size(0) == prob_m && out.size(1) == prob_n, out_name);
  int64_t groupsize = group_size;
  if (groupsize <= 0 || groupsize == prob_k) groupsize = -1;
  TORCH_CHECK(groupsize == -1 || (groupsize == 128 && scales.size(0) == prob_k / groupsize),
              "Marlin supports group_size -1 or 128");
  const int max_par = marlin_max_par();
  TORCH_CHECK(workspace.numel() >= prob_n / 128 * max_par, "marlin workspace too small");
  return {prob_m, prob_n, prob_k, groupsize};
}

// Device scratch (split-K partials, argmax keys, the MLP's activations) for
// the ops below.  The reference's _out ops take every buffer from the caller
// and allocate nothing; here each (device, stream) keeps one buffer, grown on
// demand (the caching allocator's stream ordering makes the swap safe for
// launches already queued on that stream), so that repeated calls allocate
// nothing.  Calls on one stream run in order and may share it.  A call under
// HIP graph capture takes a buffer of its own from the capture's pool instead
// (baked into the graph, so replays allocate nothing either), which keeps
// graphs independent of the eager buffer and of each other.
struct OpScratch {
  torch::Tensor hold;  // keeps a capture-time buffer alive until the launch is queued
  void* ptr = nullptr;
  size_t bytes = 0;
};

OpScratch op_scratch(size_t bytes, const torch::Tensor& like) {
  OpScratch r;
  if (bytes == 0) return r;
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream_of(like));
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cap) != hipSuccess) cap = hipStreamCaptureStatusNone;
  if (cap != hipStreamCaptureStatusNone) {
    r.hold = torch::empty({(int64_t)bytes}, like.options().dtype(torch::kUInt8));
    r.ptr = r.hold.data_ptr();
    r.bytes = bytes;
    return r;
  }
  static std::mutex mu;
  static std::map<std::pair<int, hipStream_t>, torch::Tensor> cache;
  std::lock_guard<std::mutex> lock(mu);
  torch::Tensor& t = cache[{like.get_device(), st}];
  if (!t.defined() || (size_t)t.numel() < bytes) {
    t = torch::Tensor();
    const size_t grown = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);  // whole MiB
    t = torch::empty({(int64_t)grown}, like.options().dtype(torch::kUInt8));
  }
  r.ptr = t.data_ptr();
  r.bytes = (size_t)t.numel();
  return r;
}

OpScratch scratch_for(int64_t m, int64_t n, int64_t k, int64_t g, const torch::Tensor& like) {
  return op_scratch(lb_marlin_scratch_bytes(m, n, k, g), like);
}

void run_lowbit_marlin_gemm(torch::Tensor qweight, torch::Tensor scales, torch::Tensor x, torch::Tensor out,
                            torch::Tensor workspace, int64_t cols, int64_t group_size) {
  LB_CHECK_DEV(qweight); LB_CHECK_DEV(scales); LB_CHECK_DEV(x); LB_CHECK_DEV(out); LB_CHECK_DEV(workspace);
  LB_CHECK_CONTIG(qweight); LB_CHECK_CONTIG(scales); LB_CHECK_CONTIG(x); LB_CHECK_CONTIG(out); LB_CHECK_CONTIG(workspace);
  TORCH_CHECK(qweight.scalar_type() == at::kInt, "marlin qweight must be int32");
  LB_CHECK_HALF(scales); LB_CHECK_HALF(x); LB_CHECK_HALF(out);
  TORCH_CHECK(workspace.scalar_type() == at::kInt, "marlin workspace must be int32");
  TORCH_CHECK(x.dim() == 2, "x must be [batch, cols]");
  TORCH_CHECK(x.size(1) == cols, "x cols mismatch");
  const MarlinShape sh = check_marlin_common(qweight, scales, out, workspace, x.size(0), cols, group_size,
                                             "marlin out shape mismatch");
  const c10::DeviceGuard guard(x.device());
  auto scratch = scratch_for(sh.m, sh.n, sh.k, sh.group, x);
  const int err = lb_marlin_gemm(h16(x), qweight.data_ptr<int32_t>(), h16m(out), h16(scales), sh.m, sh.n, sh.k,
                                 workspace.data_ptr<int32_t>(), workspace.numel(), sh.group, scratch.ptr,
                                 scratch.bytes, stream_of(x));
  TORCH_CHECK(err == 0, "Marlin kernel failed with code ", err);
}

torch::Tensor lowbit_marlin_gemm(torch::Tensor qweight, torch::Tensor scales, torch::Tensor x, int64_t cols,
                                 int64_t group_size) {
  TORCH_CHECK(x.dim() == 2, "x must be [batch, cols]");
  TORCH_CHECK(qweight.dim() == 2 && qweight.size(1) % 2 == 0, "marlin qweight must be [K/16, N*2]");
  const int64_t prob_n = qweight.size(1) / 2;
  const c10::DeviceGuard guard(x.device());
  auto y = torch::empty({x.size(0), prob_n}, x.options());
  auto workspace = torch::zeros({prob_n / 128 * 16}, torch::TensorOptions().dtype(torch::kInt32).device(x.device()));
  run_lowbit_marlin_gemm(qweight, scales, x, y, workspace, cols, group_size);
  return y;
}

void lowbit_marlin_gemm_out(torch::Tensor qweight, torch::Tensor scales, torch::Tensor x, torch::Tensor out,
                            torch::Tensor workspace, int64_t cols, int64_t group_size) {
  run_lowbit_marlin_gemm(qweight, scales, x, out, workspace, cols, group_size);
}

void lowbit_marlin_gemm_silu_packed_out(torch::Tensor qweight, torch::Tensor scales, torch::Tensor mixed,
                                        torch::Tensor out, torch::Tensor workspace, int64_t cols, int64_t group_size) {
  LB_CHECK_DEV(qweight); LB_CHECK_DEV(scales); LB_CHECK_DEV(mixed); LB_CHECK_DEV(out); LB_CHECK_DEV(workspace);
  LB_CHECK_CONTIG(qweight); LB_CHECK_CONTIG(scales); LB_CHECK_CONTIG(mixed); LB_CHECK_CONTIG(out); LB_CHECK_CONTIG(workspace);
  TORCH_CHECK(qweight.scalar_type() == at::kInt, "marlin qweight must be int32");
  LB_CHECK_HALF(scales); LB_CHECK_HALF(mixed); LB_CHECK_HALF(out);
  TORCH_CHECK(workspace.scalar_type() == at::kInt, "marlin workspace must be int32");
  TORCH_CHECK(mixed.dim() == 2, "mixed must be [batch, 2*cols]");
  TORCH_CHECK(mixed.size(1) == 2 * cols, "mixed width must be 2*cols");
  const MarlinShape sh = check_marlin_common(qweight, scales, out, workspace, mixed.size(0), cols, group_size,
                                             "marlin out shape mismatch");
  const c10::DeviceGuard guard(mixed.device());
  auto scratch = scratch_for(sh.m, sh.n, sh.k, sh.group, mixed);
  const int err = lb_marlin_gemm_silu_packed(h16(mixed), qweight.data_ptr<int32_t>(), h16m(out), h16(scales), sh.m,
                                             sh.n, sh.k, workspace.data_ptr<int32_t>(), workspace.numel(), sh.group,
                                             scratch.ptr, scratch.bytes, stream_of(mixed));
  TORCH_CHECK(err == 0, "Marlin silu-packed kernel failed with code ", err);
}

void lowbit_marlin_gemm_argmax_out(torch::Tensor qweight, torch::Tensor scales, torch::Tensor x,
                                   torch::Tensor scratch_out, torch::Tensor workspace, torch::Tensor argmax_state,
                                   torch::Tensor argmax_out, torch::Tensor argmax_sync, int64_t argmax_epoch,
                                   int64_t cols, int64_t group_size) {
  LB_CHECK_DEV(qweight); LB_CHECK_DEV(scales); LB_CHECK_DEV(x);
  LB_CHECK_DEV(scratch_out); LB_CHECK_DEV(workspace); LB_CHECK_DEV(argmax_state); LB_CHECK_DEV(argmax_out);
  LB_CHECK_DEV(argmax_sync);
  LB_CHECK_CONTIG(qweight); LB_CHECK_CONTIG(scales); LB_CHECK_CONTIG(x);
  LB_CHECK_CONTIG(scratch_out); LB_CHECK_CONTIG(workspace); LB_CHECK_CONTIG(argmax_state); LB_CHECK_CONTIG(argmax_out);
  LB_CHECK_CONTIG(argmax_sync);
  TORCH_CHECK(qweight.scalar_type() == at::kInt, "marlin qweight must be int32");
  LB_CHECK_HALF(scales); LB_CHECK_HALF(x); LB_CHECK_HALF(scratch_out);
  TORCH_CHECK(workspace.scalar_type() == at::kInt, "marlin workspace must be int32");
  LB_CHECK_I64(argmax_state); LB_CHECK_I64(argmax_out);
  TORCH_CHECK(argmax_sync.scalar_type() == at::kInt, "argmax_sync must be int32");
  TORCH_CHECK(x.dim() == 2, "x must be [batch, cols]");
  TORCH_CHECK(x.size(1) == cols, "x cols mismatch");
  const int64_t prob_m = x.size(0);
  const MarlinShape sh = check_marlin_common(qweight, scales, scratch_out, workspace, prob_m, cols, group_size,
                                             "marlin scratch_out shape mismatch");
  TORCH_CHECK(argmax_state.dim() == 1 && argmax_state.numel() >= prob_m, "argmax_state must be [batch]");
  TORCH_CHECK(argmax_out.dim() == 1 && argmax_out.numel() >= prob_m, "argmax_out must be [batch]");
  TORCH_CHECK(argmax_sync.dim() == 1 && argmax_sync.numel() >= 2, "argmax_sync must be [2]");
  TORCH_CHECK(argmax_epoch > 0, "argmax_epoch must be positive");
  const c10::DeviceGuard guard(x.device());
  auto scratch = scratch_for(sh.m, sh.n, sh.k, sh.group, x);
  const int err = lb_marlin_gemm_argmax(h16(x), qweight.data_ptr<int32_t>(), h16(scales), sh.m, sh.n, sh.k,
                                        workspace.data_ptr<int32_t>(), workspace.numel(), sh.group,
                                        argmax_state.data_ptr<int64_t>(), argmax_out.data_ptr<int64_t>(),
                                        argmax_sync.data_ptr<int32_t>(), (int32_t)argmax_epoch, scratch.ptr,
                                        scratch.bytes, stream_of(x));
  TORCH_CHECK(err == 0, "Marlin argmax kernel failed with code ", err);
}

void lowbit_marlin_mlp_streaming_out(torch::Tensor gate_up_qweight, torch::Tensor gate_up_scales,
                                     torch::Tensor down_qweight, torch::Tensor down_scales, torch::Tensor x,
                                     torch::Tensor out, torch::Tensor accum, torch::Tensor sync, int64_t epoch,
                                     int64_t hidden_i, int64_t intermediate_i, int64_t gate_group_size_i,
                                     int64_t down_group_size_i) {
  LB_CHECK_DEV(gate_up_qweight); LB_CHECK_DEV(gate_up_scales); LB_CHECK_DEV(down_qweight); LB_CHECK_DEV(down_scales);
  LB_CHECK_DEV(x); LB_CHECK_DEV(out); LB_CHECK_DEV(accum); LB_CHECK_DEV(sync);
  LB_CHECK_CONTIG(gate_up_qweight); LB_CHECK_CONTIG(gate_up_scales); LB_CHECK_CONTIG(down_qweight);
  LB_CHECK_CONTIG(down_scales); LB_CHECK_CONTIG(x); LB_CHECK_CONTIG(out); LB_CHECK_CONTIG(accum); LB_CHECK_CONTIG(sync);
  TORCH_CHECK(gate_up_qweight.scalar_type() == at::kInt && down_qweight.scalar_type() == at::kInt,
              "Marlin qweight must be int32");
  LB_CHECK_HALF(gate_up_scales); LB_CHECK_HALF(down_scales); LB_CHECK_HALF(x); LB_CHECK_HALF(out);
  LB_CHECK_FLOAT(accum);
  TORCH_CHECK(sync.scalar_type() == at::kInt, "sync must be int32");
  TORCH_CHECK(x.dim() == 2, "x must be [batch, hidden]");
  const int64_t batch = x.size(0);
  const int64_t hidden = hidden_i, intermediate = intermediate_i;
  TORCH_CHECK(hidden > 0 && intermediate > 0, "hidden/intermediate must be positive");
  TORCH_CHECK(hidden % 16 == 0 && intermediate % 16 == 0, "hidden/intermediate must be divisible by 16");
  TORCH_CHECK(x.size(1) == hidden, "x hidden mismatch");
  TORCH_CHECK(out.dim() == 2 && out.size(0) == batch && out.size(1) == hidden, "out must be [batch, hidden]");
  TORCH_CHECK(accum.dim() == 2 && accum.size(0) == batch && accum.size(1) == hidden, "accum must be [batch, hidden]");
  TORCH_CHECK(sync.dim() == 1 && sync.numel() >= 2 * batch, "sync must have at least 2*batch int32 elements");
  TORCH_CHECK(gate_up_qweight.dim() == 2 && gate_up_qweight.size(0) == hidden / 16 &&
                  gate_up_qweight.size(1) == 4 * intermediate,
              "gate_up qweight must be [hidden/16, (2*intermediate)*2]");
  TORCH_CHECK(down_qweight.dim() == 2 && down_qweight.size(0) == intermediate / 16 &&
                  down_qweight.size(1) == 2 * hidden,
              "down qweight must be [intermediate/16, hidden*2]");
  int64_t gate_group = gate_group_size_i, down_group = down_group_size_i;
  if (gate_group <= 0 || gate_group == hidden) gate_group = -1;
  if (down_group <= 0 || down_group == intermediate) down_group = -1;
  TORCH_CHECK(gate_group == -1 || gate_group == 128, "gate_up Marlin group_size must be -1 or 128");
  TORCH_CHECK(down_group == -1 || down_group == 128, "down Marlin group_size must be -1 or 128");
  const int64_t gate_groups = gate_group == -1 ? 1 : hidden / gate_group;
  const int64_t down_groups = down_group == -1 ? 1 : intermediate / down_group;
  TORCH_CHECK(gate_up_scales.dim() == 2 && gate_up_scales.size(0) == gate_groups &&
                  gate_up_scales.size(1) == 2 * intermediate,
              "gate_up scales shape mismatch");
  TORCH_CHECK(down_scales.dim() == 2 && down_scales.size(0) == down_groups && down_scales.size(1) == hidden,
              "down scales shape mismatch");
  TORCH_CHECK(epoch > 0, "epoch must be positive");
  const c10::DeviceGuard guard(x.device());
  auto scratch = op_scratch(lb_marlin_mlp_scratch_bytes(batch, hidden, intermediate), x);
  const int err = lb_marlin_mlp_streaming(gate_up_qweight.data_ptr<int32_t>(), h16(gate_up_scales),
                                          down_qweight.data_ptr<int32_t>(), h16(down_scales), h16(x), h16m(out),
                                          accum.data_ptr<float>(), sync.data_ptr<int32_t>(), batch, hidden,
                                          intermediate, gate_group, down_group, scratch.ptr, scratch.bytes,
                                          stream_of(x));
  TORCH_CHECK(err == 0, "Marlin streaming MLP failed with code ", err, " (", lb_status_string(err), ")");
}

// The decode MLP the reference's _fused_marlin_down runs as two ops
// (langburst/adapters/qwen36_impl/model.py:1460-1470: gate/up GEMM, then the
// SiLU-packed down GEMM), as one call, bit-identical to the two ops (two
// launches, the gate_up one storing fp16(silu(g) * u) where its tiles pair the
// gate and up chunks).  `workspace` is int32, zero on entry and left zero.
void lowbit_marlin_mlp_fused_out(torch::Tensor gate_up_qweight, torch::Tensor gate_up_scales,
                                 torch::Tensor down_qweight, torch::Tensor down_scales, torch::Tensor x,
                                 torch::Tensor out, torch::Tensor workspace, int64_t hidden, int64_t intermediate,
                                 int64_t gate_group_size, int64_t down_group_size) {
  LB_CHECK_DEV(gate_up_qweight); LB_CHECK_DEV(gate_up_scales); LB_CHECK_DEV(down_qweight); LB_CHECK_DEV(down_scales);
  LB_CHECK_DEV(x); LB_CHECK_DEV(out); LB_CHECK_DEV(workspace);
  LB_CHECK_CONTIG(gate_up_qweight); LB_CHECK_CONTIG(gate_up_scales); LB_CHECK_CONTIG(down_qweight);
  LB_CHECK_CONTIG(down_scales); LB_CHECK_CONTIG(x); LB_CHECK_CONTIG(out); LB_CHECK_CONTIG(workspace);
  TORCH_CHECK(gate_up_qweight.scalar_type() == at::kInt && down_qweight.scalar_type() == at::kInt,
              "Marlin qweight must be int32");
  LB_CHECK_HALF(gate_up_scales); LB_CHECK_HALF(down_scales); LB_CHECK_HALF(x); LB_CHECK_HALF(out);
  TORCH_CHECK(workspace.scalar_type() == at::kInt, "workspace must be int32");
  TORCH_CHECK(x.dim() == 2, "x must be [batch, hidden]");
  const int64_t batch = x.size(0);
  TORCH_CHECK(x.size(1) == hidden, "x hidden mismatch");
  TORCH_CHECK(out.dim() == 2 && out.size(0) == batch && out.size(1) == hidden, "out must be [batch, hidden]");
  TORCH_CHECK(gate_up_qweight.dim() == 2 && gate_up_qweight.size(0) == hidden / 16 &&
                  gate_up_qweight.size(1) == 4 * intermediate,
              "gate_up qweight must be [hidden/16, (2*intermediate)*2]");
  TORCH_CHECK(down_qweight.dim() == 2 && down_qweight.size(0) == intermediate / 16 &&
                  down_qweight.size(1) == 2 * hidden,
              "down qweight must be [intermediate/16, hidden*2]");
  int64_t gate_group = gate_group_size, down_group = down_group_size;
  if (gate_group <= 0 || gate_group == hidden) gate_group = -1;
  if (down_group <= 0 || down_group == intermediate) down_group = -1;
  const int64_t gate_groups = gate_group == 128 ? hidden / 128 : 1;
  const int64_t down_groups = down_group == 128 ? intermediate / 128 : 1;
  TORCH_CHECK(gate_up_scales.dim() == 2 && gate_up_scales.size(0) == gate_groups &&
                  gate_up_scales.size(1) == 2 * intermediate,
              "gate_up scales shape mismatch");
  TORCH_CHECK(down_scales.dim() == 2 && down_scales.size(0) == down_groups && down_scales.size(1) == hidden,
              "down scales shape mismatch");
  const int64_t ws_need = lb_marlin_mlp_fused_workspace_len(batch, hidden, intermediate);
  TORCH_CHECK(workspace.numel() >= ws_need, "workspace must hold at least ", ws_need, " int32 elements");
  const c10::DeviceGuard guard(x.device());
  auto scratch = op_scratch(lb_marlin_mlp_fused_scratch_bytes(batch, hidden, intermediate), x);
  lb_ok(lb_marlin_mlp_fused(h16(x), gate_up_qweight.data_ptr<int32_t>(), h16(gate_up_scales),
                            down_qweight.data_ptr<int32_t>(), h16(down_scales), h16m(out), batch, hidden,
                            intermediate, gate_group, down_group, workspace.data_ptr<int32_t>(), workspace.numel(),
                            scratch.ptr, scratch.bytes, stream_of(x)),
        "lowbit_marlin_mlp_fused_out");
}

// Dense fp16 W[N, K] of a Marlin tensor (no reference op; the reference's
// inverse reader is csrc/marlin_mlp_stream.cu:109-133).
torch::Tensor lowbit_marlin_dequant(torch::Tensor qweight, torch::Tensor scales, int64_t cols, int64_t group_size) {
  LB_CHECK_DEV(qweight); LB_CHECK_DEV(scales);
  LB_CHECK_CONTIG(qweight); LB_CHECK_CONTIG(scales);
  TORCH_CHECK(qweight.scalar_type() == at::kInt, "marlin qweight must be int32");
  LB_CHECK_HALF(scales);
  TORCH_CHECK(cols % 128 == 0, "Marlin requires K divisible by 128");
  TORCH_CHECK(qweight.dim() == 2 && qweight.size(0) == cols / 16 && qweight.size(1) % 2 == 0,
              "marlin qweight must be [K/16, N*2]");
  const int64_t prob_n = qweight.size(1) / 2;
  TORCH_CHECK(prob_n % 256 == 0, "Marlin requires N divisible by 256");
  int64_t g = group_size;
  if (g <= 0 || g == cols) g = -1;
  TORCH_CHECK(g == -1 || (g == 128 && scales.size(0) == cols / 128), "Marlin supports group_size -1 or 128");
  TORCH_CHECK(scales.dim() == 2 && scales.size(1) == prob_n, "marlin scales must be [K/group, N]");
  const c10::DeviceGuard guard(qweight.device());
  auto w = torch::empty({prob_n, cols}, scales.options());
  lb_ok(lb_marlin_dequant(qweight.data_ptr<int32_t>(), h16(scales), h16m(w), prob_n, cols, g, stream_of(qweight)),
        "lowbit_marlin_dequant");
  return w;
}

}  // namespace

PYBIND11_MODULE(langburst_cuda, m) {
  m.doc() = "LangBurst low-bit projection kernels for MI355X (gfx950)";
  m.def("lowbit_gemv", &lowbit_gemv, "Groupwise symmetric low-bit GEMV: y = dequant(qweight, scales, bits) @ x",
        py::arg("qweight"), py::arg("scales"), py::arg("x"), py::arg("cols"), py::arg("group_size"), py::arg("bits"),
        py::arg("rows_per_cta") = 8);
  m.def("lowbit_row_dequant", &lowbit_row_dequant, "Dequantize one low-bit row, used for embeddings");
  m.def("lowbit_gemv_pair", &lowbit_gemv_pair, "Two groupwise symmetric low-bit GEMVs sharing the same input vector",
        py::arg("qweight_a"), py::arg("scales_a"), py::arg("qweight_b"), py::arg("scales_b"), py::arg("x"),
        py::arg("cols"), py::arg("group_size"), py::arg("bits"), py::arg("rows_per_cta") = 8);
  m.def("lowbit_gemm", &lowbit_gemm, "Groupwise symmetric low-bit GEMM: y = x @ dequant(qweight, scales, bits).T",
        py::arg("qweight"), py::arg("scales"), py::arg("x"), py::arg("cols"), py::arg("group_size"), py::arg("bits"),
        py::arg("rows_per_cta") = 8);
  m.def("lowbit_marlin_gemm", &lowbit_marlin_gemm, "Marlin W4A16 GEMM: y = x @ dequant(qweight, scales).T",
        py::arg("qweight"), py::arg("scales"), py::arg("x"), py::arg("cols"), py::arg("group_size"));
  m.def("lowbit_marlin_gemm_out", &lowbit_marlin_gemm_out, "Marlin W4A16 GEMM into preallocated output/workspace",
        py::arg("qweight"), py::arg("scales"), py::arg("x"), py::arg("out"), py::arg("workspace"), py::arg("cols"),
        py::arg("group_size"));
  m.def("lowbit_marlin_mlp_streaming_out", &lowbit_marlin_mlp_streaming_out,
        "Marlin-layout MLP: gate/up projection, SiLU gate and down projection with float32 intermediates",
        py::arg("gate_up_qweight"), py::arg("gate_up_scales"), py::arg("down_qweight"), py::arg("down_scales"),
        py::arg("x"), py::arg("out"), py::arg("accum"), py::arg("sync"), py::arg("epoch"), py::arg("hidden"),
        py::arg("intermediate"), py::arg("gate_group_size"), py::arg("down_group_size"));
  m.def("lowbit_marlin_gemm_silu_packed_out", &lowbit_marlin_gemm_silu_packed_out,
        "Marlin W4A16 GEMM whose A operand is SiLU(mixed[:K]) * mixed[K:] computed inside the kernel",
        py::arg("qweight"), py::arg("scales"), py::arg("mixed"), py::arg("out"), py::arg("workspace"),
        py::arg("cols"), py::arg("group_size"));
  m.def("lowbit_marlin_gemm_argmax_out", &lowbit_marlin_gemm_argmax_out,
        "Marlin W4A16 GEMM with fused row argmax into argmax_out (scratch_out is not written)",
        py::arg("qweight"), py::arg("scales"), py::arg("x"), py::arg("scratch_out"), py::arg("workspace"),
        py::arg("argmax_state"), py::arg("argmax_out"), py::arg("argmax_sync"), py::arg("argmax_epoch"),
        py::arg("cols"), py::arg("group_size"));
  m.def("lowbit_marlin_dequant", &lowbit_marlin_dequant, "Dense fp16 W[N, K] of a Marlin tensor",
        py::arg("qweight"), py::arg("scales"), py::arg("cols"), py::arg("group_size"));
  m.def("lowbit_marlin_mlp_fused_out", &lowbit_marlin_mlp_fused_out,
        "Marlin W4A16 decode MLP: down(SiLU(gate) * up) of x, bit-identical to the gate_up GEMM then the "
        "SiLU-packed down GEMM",
        py::arg("gate_up_qweight"), py::arg("gate_up_scales"), py::arg("down_qweight"), py::arg("down_scales"),
        py::arg("x"), py::arg("out"), py::arg("workspace"), py::arg("hidden"), py::arg("intermediate"),
        py::arg("gate_group_size"), py::arg("down_group_size"));
  m.def("lowbit_marlin_mlp_fused_workspace_len",
        [](int64_t batch, int64_t hidden, int64_t intermediate) {
          return lb_marlin_mlp_fused_workspace_len(batch, hidden, intermediate);
        },
        "int32 elements of the workspace lowbit_marlin_mlp_fused_out needs", py::arg("batch"), py::arg("hidden"),
        py::arg("intermediate"));
  m.def("abi_version", []() { return lb_abi_version(); });
  m.attr("__provides__") = py::make_tuple("lowbit_gemv", "lowbit_row_dequant", "lowbit_gemv_pair", "lowbit_gemm",
                                          "lowbit_marlin_gemm", "lowbit_marlin_gemm_out",
                                          "lowbit_marlin_mlp_streaming_out", "lowbit_marlin_gemm_silu_packed_out",
                                          "lowbit_marlin_gemm_argmax_out");
}
