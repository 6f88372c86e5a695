/*
 * langburst_lowbit.h -- C ABI of the MI355X (gfx950) low-bit weight-only
 * projection library (liblangburst_lowbit.so).
 *
 * Plain pointers and sizes only.  Every entry point:
 *   - validates its arguments before touching the GPU and returns a status
 *     code (LB_OK == 0) instead of raising;
 *   - enqueues its kernels on `stream` (a hipStream_t; NULL = default stream)
 *     and never synchronises;
 *   - reads/writes caller-owned device memory only (plus `scratch` when the
 *     entry point takes one).
 * fp16 tensors are passed as uint16_t* holding IEEE binary16 bits.
 * Shapes use the reference's names: K = input (reduction) columns ("cols"),
 * N = output rows, M = batch rows.
 *
 * Reference paths below are relative to GizAI/neurova's langburst/.
 */
#ifndef LANGBURST_LOWBIT_H
#define LANGBURST_LOWBIT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  1 and 2 keep the meaning of marlin_cuda's ERR_PROB_SHAPE /
 * ERR_KERN_SHAPE (csrc/marlin_cuda_kernel.cu:914-915). */
enum lb_status {
  LB_OK = 0,
  LB_ERR_PROB_SHAPE = 1, /* problem shape not supported (N % 256, K % 128, ...) */
  LB_ERR_KERN_SHAPE = 2, /* no kernel configuration for this shape */
  LB_ERR_ARG = 3,        /* invalid argument: null pointer, bits, rows_per_cta, sizes */
  LB_ERR_ALIGN = 4,      /* a pointer is not aligned as the kernels require */
  LB_ERR_WORKSPACE = 5,  /* workspace shorter than required */
  LB_ERR_SCRATCH = 6,    /* scratch buffer shorter than lb_marlin_scratch_bytes() */
  LB_ERR_HIP = 7,        /* the HIP runtime reported an error at launch */
  /* 8 is not used */
  LB_ERR_NOALLOC_LIMIT = 9 /* lb_marlin_gemm_noalloc: the problem needs more than its static scratch */
};

typedef void* lb_stream_t; /* hipStream_t */

/* Human-readable text for a status code (static storage). */
const char* lb_status_string(int status);
/* Version of this ABI; bumped on any signature change. */
int lb_abi_version(void);

/* ---------------- Rowwise symmetric 2..8-bit groupwise layout ----------------
 * qweight: uint8 [rows, packed_cols], each row an LSB-first bitstream of
 *          `cols` codes of `bits` bits (packed_cols >= ceil(cols*bits/8));
 * scales:  fp16  [rows, scale_cols] (scale_cols >= ceil(cols/group_size));
 * dequant: (code - 2^(bits-1)) * scale[row, c / group_size]; fp32 accumulate.
 * rows_per_cta must be 4, 8 or 16 (the reference's tuning knob; accepted and
 * validated, the gfx950 kernels choose their own tiling).
 */

/* y[rows] = dequant(W) @ x[cols].
 * Replaces lowbit_gemv (csrc/lowbit_gemv.cu:303-316, launcher :270-291). */
int lb_lowbit_gemv(const uint8_t* qweight, int64_t rows, int64_t packed_cols,
                   const uint16_t* scales, int64_t scale_cols,
                   const uint16_t* x, uint16_t* y,
                   int64_t cols, int64_t group_size, int64_t bits, int64_t rows_per_cta,
                   lb_stream_t stream);

/* Two GEMVs with identical shapes sharing x.
 * Replaces lowbit_gemv_pair (csrc/lowbit_gemv.cu:375-397, launcher :318-356). */
int lb_lowbit_gemv_pair(const uint8_t* qweight_a, const uint16_t* scales_a,
                        const uint8_t* qweight_b, const uint16_t* scales_b,
                        int64_t rows, int64_t packed_cols, int64_t scale_cols,
                        const uint16_t* x, uint16_t* y_a, uint16_t* y_b,
                        int64_t cols, int64_t group_size, int64_t bits, int64_t rows_per_cta,
                        lb_stream_t stream);

/* Y[batch, rows] = X[batch, :cols] @ dequant(W)^T; X rows are x_stride apart.
 * Replaces lowbit_gemm (csrc/lowbit_gemv.cu:433-445, launcher :399-421). */
int lb_lowbit_gemm(const uint8_t* qweight, int64_t rows, int64_t packed_cols,
                   const uint16_t* scales, int64_t scale_cols,
                   const uint16_t* x, int64_t batch, int64_t x_stride, uint16_t* y,
                   int64_t cols, int64_t group_size, int64_t bits, int64_t rows_per_cta,
                   lb_stream_t stream);

/* out[cols] = dequant(W[*row_index]) as fp16; the row index is read on the
 * device; an out-of-range index yields zeros.
 * Replaces lowbit_row_dequant (csrc/lowbit_gemv.cu:468-480, kernel :226-248). */
int lb_lowbit_row_dequant(const uint8_t* qweight, int64_t rows, int64_t packed_cols,
                          const uint16_t* scales, int64_t scale_cols,
                          const int64_t* row_index, uint16_t* out,
                          int64_t cols, int64_t group_size, int64_t bits,
                          lb_stream_t stream);

/* ---------------- Marlin W4A16 layout ("marlin_v1") ----------------
 * B (qweight): int32 [K/16, 2N], 16x16-tile transposed, 1024-entry permuted
 *              4-bit codes, zero point 8;
 * s (scales):  fp16 [K/groupsize, N] in the 64-entry permuted order, or
 *              [1, N] in the 32-entry per-column order when groupsize == -1;
 * groupsize:   128, or -1 / <= 0 / == K for one scale per column;
 * workspace:   int32, zero on entry, at least N/128 elements (the reference
 *              sizes it N/128*16); left zero on return;
 * scratch:     device memory of at least lb_marlin_scratch_bytes() bytes
 *              (may be NULL when that is 0); contents need no initialisation.
 * Requires N % 256 == 0 and K % 128 == 0; any M >= 0.
 */

/* Bytes of scratch the Marlin entry points need for this problem. */
size_t lb_marlin_scratch_bytes(int64_t prob_m, int64_t prob_n, int64_t prob_k, int64_t groupsize);

/* The plan a Marlin entry point makes for this problem (no counterpart in the
 * reference; for tests and tools, no device work).  variant: 0 lb_marlin_gemm,
 * 1 lb_marlin_gemm_silu_packed, 2 lb_marlin_gemm_argmax; workspace_len as the
 * call would pass it.  Fills out[10]:
 *   [0] form: 0 decode tiles with the A slice staged whole, 1 decode tiles
 *       with A fragments loaded per step, 2 decode tiles with A through an
 *       LDS ring, 3 prefill GEMM tiles with the split-tail schedule, 4 prefill
 *       GEMM tiles with the stream-K schedule (every resident workgroup runs
 *       an equal range of the tiles' scale-group stages);
 *   [1] decode: 64-column chunks per workgroup; prefill: 16-row blocks;
 *   [2] decode: k splits of every column tile; split-tail: k splits of the
 *       tail tiles; stream-K: 1;
 *   [3] decode: 16-row MFMA blocks; split-tail: whole tiles; stream-K: 0;
 *   [4] workgroups; [5] dynamic LDS bytes per workgroup; [6] scratch bytes;
 *   [7] workspace entries used; [8] kernel launches; [9] compute units planned for.
 * Returns LB_OK, or the status the entry point would return for the shape. */
int lb_marlin_describe_plan(int64_t prob_m, int64_t prob_n, int64_t prob_k, int64_t groupsize, int32_t variant,
                            int64_t workspace_len, int64_t* out);

/* C[M, N] = A[M, K] @ dequant(B), fp32 accumulate, fp16 C.  Grouped scales:
 * the fp16 weights fp16(fp16(q - 8) * s) are accumulated, as the reference
 * does; per-column scales: fp16(sum of x * (q - 8)) * s, as the reference.
 * Results differ from the reference's only by fp32 summation order.
 * Replaces marlin_cuda (csrc/marlin_cuda_kernel.cu:917-1005) as called by
 * run_lowbit_marlin_gemm (csrc/langburst_ext.cpp:67-114). */
int lb_marlin_gemm(const uint16_t* A, const int32_t* B, uint16_t* C, const uint16_t* s,
                   int64_t prob_m, int64_t prob_n, int64_t prob_k,
                   int32_t* workspace, int64_t workspace_len, int64_t groupsize,
                   void* scratch, size_t scratch_bytes, lb_stream_t stream);

/* Same product with A = fp16(silu(mixed[:, :K]) * mixed[:, K:2K]) formed in
 * the kernel; mixed is fp16 [M, 2K].
 * Replaces marlin_cuda_silu_packed (csrc/marlin_cuda_kernel.cu:1102-1184) as
 * called by lowbit_marlin_gemm_silu_packed_out (csrc/langburst_ext.cpp:131-185). */
int lb_marlin_gemm_silu_packed(const uint16_t* mixed, const int32_t* B, uint16_t* C, const uint16_t* s,
                               int64_t prob_m, int64_t prob_n, int64_t prob_k,
                               int32_t* workspace, int64_t workspace_len, int64_t groupsize,
                               void* scratch, size_t scratch_bytes, lb_stream_t stream);

/* argmax_out[m] = argmax_n C[m, n] (first index among equal maxima; +0 > -0),
 * without writing C.  argmax_state[m] receives the winning packed key
 * (order-preserving value bits << 32 | 0xffffffff - index).  argmax_sync and
 * epoch are accepted for interface parity and not otherwise needed.
 * Replaces marlin_cuda_argmax (csrc/marlin_cuda_kernel.cu:1007-1100) as called
 * by lowbit_marlin_gemm_argmax_out (csrc/langburst_ext.cpp:187-257). */
int lb_marlin_gemm_argmax(const uint16_t* A, const int32_t* B, const uint16_t* s,
                          int64_t prob_m, int64_t prob_n, int64_t prob_k,
                          int32_t* workspace, int64_t workspace_len, int64_t groupsize,
                          int64_t* argmax_state, int64_t* argmax_out,
                          int32_t* argmax_sync, int32_t epoch,
                          void* scratch, size_t scratch_bytes, lb_stream_t stream);

/* Bytes of scratch lb_marlin_mlp_streaming needs. */
size_t lb_marlin_mlp_scratch_bytes(int64_t batch, int64_t hidden, int64_t intermediate);

/* out[batch, hidden] = down( silu(gate(x)) * up(x) ) with the streaming
 * kernel's numerics: float32 weights (q-8)*s, float32 activations, one fp16
 * rounding at the end.  gate_up is a Marlin tensor [hidden -> 2*intermediate]
 * (gate = first half), down is [intermediate -> hidden].  accum (fp32
 * [batch, hidden]) and sync (int32 [>= 2*batch]) are accepted for interface
 * parity.
 * Replaces lowbit_marlin_mlp_streaming_out (csrc/marlin_mlp_stream.cu:219-287). */
int lb_marlin_mlp_streaming(const int32_t* gate_up_qweight, const uint16_t* gate_up_scales,
                            const int32_t* down_qweight, const uint16_t* down_scales,
                            const uint16_t* x, uint16_t* out, float* accum, int32_t* sync,
                            int64_t batch, int64_t hidden, int64_t intermediate,
                            int64_t gate_group_size, int64_t down_group_size,
                            void* scratch, size_t scratch_bytes, lb_stream_t stream);

/* Decode MLP: out[batch, hidden] = down(fp16(silu(g) * u)) with
 * [g | u] = fp16(gate_up(x)); gate_up is a Marlin tensor [hidden -> 2*intermediate]
 * (gate = first half), down is [intermediate -> hidden].  The numerics of the
 * reference's production MLP, which runs the gate_up projection and then
 * down.gemm_silu_packed as two launches (adapters/qwen36_impl/model.py:1460-1470
 * _fused_marlin_down, loader.py:337-368): bit-identical to lb_marlin_gemm followed
 * by lb_marlin_gemm_silu_packed.  Two launches as well; where the gate_up
 * projection plans decode tiles of 2 or 4 chunks, its launch pairs the gate and
 * up chunks of the same neurons and stores fp16(silu(g) * u) instead of [g | u].
 * No reference op: replaces that pair of calls.
 * workspace: int32 [lb_marlin_mlp_fused_workspace_len()], zero on entry, left zero.
 * scratch:   lb_marlin_mlp_fused_scratch_bytes() bytes, 256-byte aligned.
 * Calls that share a workspace or scratch must not overlap. */
size_t lb_marlin_mlp_fused_scratch_bytes(int64_t batch, int64_t hidden, int64_t intermediate);
int64_t lb_marlin_mlp_fused_workspace_len(int64_t batch, int64_t hidden, int64_t intermediate);
int lb_marlin_mlp_fused(const uint16_t* x, const int32_t* gate_up_qweight, const uint16_t* gate_up_scales,
                        const int32_t* down_qweight, const uint16_t* down_scales, uint16_t* out,
                        int64_t batch, int64_t hidden, int64_t intermediate,
                        int64_t gate_group_size, int64_t down_group_size,
                        int32_t* workspace, int64_t workspace_len,
                        void* scratch, size_t scratch_bytes, lb_stream_t stream);

/* lb_marlin_gemm without caller scratch and without any allocation: no
 * counterpart in the reference; for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The split-K partials go to a static device array of
 * lb_marlin_noalloc_scratch_limit() bytes (64 MiB) that each GPU holds until
 * the process ends; problems whose plan needs more return
 * LB_ERR_NOALLOC_LIMIT before anything is launched (every decode shape up to
 * M = 64 of the BASELINE.json projections and of the reference's published
 * ones, lm_head 5120 -> 248320 included, fits; M = 2048 prefill does not).  All
 * calls on one GPU share that array: calls that overlap (other streams) race
 * and must be serialised by the caller.  Same arguments, workspace contract
 * and results as lb_marlin_gemm. */
size_t lb_marlin_noalloc_scratch_limit(void);
int lb_marlin_gemm_noalloc(const uint16_t* A, const int32_t* B, uint16_t* C, const uint16_t* s,
                           int64_t prob_m, int64_t prob_n, int64_t prob_k,
                           int32_t* workspace, int64_t workspace_len, int64_t groupsize, lb_stream_t stream);

/* Dense fp16 W[N, K] = fp16((q - 8) * s) (or q - 8 for per-column scales),
 * bit-exact with the reference's in-kernel dequant (csrc/marlin_cuda_kernel.cu:131-159).
 * No reference counterpart as an op: the inverse of the layout is the
 * reference's scalar reader csrc/marlin_mlp_stream.cu:109-133. */
int lb_marlin_dequant(const int32_t* B, const uint16_t* s, uint16_t* w_nk,
                      int64_t prob_n, int64_t prob_k, int64_t groupsize, lb_stream_t stream);

/* ---------------- Measurement probe (no reference counterpart) ----------------
 * Reads `bytes` (a multiple of 16) of device memory at `src` with 16-byte
 * non-temporal loads over `workgroups` workgroups of 256 threads, each a
 * contiguous range (a ring of 8 loads in flight per lane), and folds the data
 * into one word per workgroup, stored to sink[workgroup] only when it equals a
 * fixed value (sink holds `workgroups` words): the streaming-read ceiling that
 * the bandwidth-bound kernels are compared with. */
int lb_probe_stream_read(const void* src, size_t bytes, uint32_t* sink, int32_t workgroups, lb_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* LANGBURST_LOWBIT_H */
