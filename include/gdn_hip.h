/*
 * C ABI of the MI355X (gfx950) gated-delta-rule library, libgdn_hip.so.
 *
 * Plain pointers and sizes only; every pointer is device memory unless stated.
 * All entry points are asynchronous on `stream`, allocate nothing, validate
 * their arguments on the host before any launch, and return
 * hipErrorInvalidValue for an unsupported configuration (the reference's
 * cudaErrorInvalidValue contract, kernels/chunk_delta_cuda.cu:706-708,727),
 * otherwise the first launch error.  They are reentrant: no global state.
 *
 * Tensor layouts (contiguous, row-major) follow kernels/chunk_delta_cuda.h:12-20:
 *   q, k : bf16 [B, T, HQK, DK]   v-head h reads qk-head h / (HV / HQK)
 *   v    : bf16 [B, T, HV, DV]
 *   g    : fp32 [B, T, HV]        log-decay (<= 0), cumulated inside chunks
 *   beta : fp32 [B, T, HV]
 *   o    : bf16 [B, T, HV, DV]    (out)
 *   state: fp32 [B, HV, DK, DV]
 * q and k are expected L2-normalised by the caller, as in the reference
 * (kernels/chunk_delta_cuda.h:23-25).  Only DK = DV = 128 and chunk_size = 64
 * are supported (the reference validates the same single configuration).
 */
#ifndef GDN_HIP_H_
#define GDN_HIP_H_

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GDN_DTYPE_BF16 0
#define GDN_DTYPE_FP16 1
#define GDN_DTYPE_FP32 2

/* Workspace bytes for one deltanet_chunk_prefill call (0 for an unsupported
 * configuration).  Replaces deltanet_prefill_workspace_size,
 * kernels/chunk_delta_cuda.h:39.  Includes the debug tail, so the same size
 * serves dump_debug = 0 and 1. */
size_t deltanet_prefill_workspace_size(int B, int T, int HV, int DK, int DV, int chunk_size);

/* Allocation-free deltanet_chunk_prefill (dump_debug = 0): the workspace is
 * a 48 MiB device array the library holds per GPU until the process ends,
 * so the call allocates nothing (no hipMalloc, no allocating library call).
 * No counterpart in the reference: it is for callers that cannot allocate --
 * code under HIP graph capture, tight serving loops.  Every call on one GPU
 * shares that array, so calls that overlap on one GPU (two streams, say)
 * race; calls in one stream do not.  A call whose live workspace exceeds the
 * array (more than 712 chunk-heads, e.g. T > 1408 at HV = 32) returns
 * hipErrorInvalidValue before any launch. */
hipError_t deltanet_chunk_prefill_noalloc(const void* q, const void* k, const void* v,
                                          const float* g, const float* beta, void* o,
                                          const float* initial_state, float* final_state, int B,
                                          int T, int HV, int HQK, int DK, int DV, int chunk_size,
                                          hipStream_t stream);

/* deltanet_prefill_status for the array deltanet_chunk_prefill_noalloc uses
 * on the current device: synchronises `stream`, then returns hipSuccess, or
 * hipErrorLaunchTimeOut when a bounded wait of the last allocation-free call
 * on this device gave up.  Allocates nothing.  No counterpart in the
 * reference (for the same callers as deltanet_chunk_prefill_noalloc). */
hipError_t deltanet_prefill_noalloc_status(hipStream_t stream);

/* Workspace bytes for dump_debug = 0 only (no counterpart in the reference,
 * whose size always includes its debug regions): a 256-byte header with the
 * status word, then 69 KB per (chunk, v-head). */
size_t deltanet_prefill_live_workspace_size(int B, int T, int HV, int DK, int DV,
                                            int chunk_size);

/* Chunked gated-delta-rule prefill.  Replaces deltanet_chunk_prefill,
 * kernels/chunk_delta_cuda.h:47-55 (same argument order and meaning; HIP
 * stream and error types).  initial_state may be NULL (zeros); initial_state
 * and final_state may be the same buffer.  workspace_bytes must be at least
 * the live size (dump_debug = 0) or the full size (dump_debug != 0).
 * dump_debug != 0 additionally writes, past the live workspace, per
 * chunk-head (index (b * NC + chunk) * HV + h) fp32 T = (I - A)^-1, A, T right
 * after the diagonal 16x16 blocks are inverted (A below them; the reference's
 * post-leaf view), M = s (Q K^T o Gamma) (each [64][64]), the in-chunk cumsum
 * of g ([64]) and the state at the chunk's start ([DK][DV]).
 * The scan's waits are bounded: should one run out (another process holding
 * the device, say) the call still completes, leaves o and final_state
 * incomplete and sets the workspace's status word; deltanet_prefill_status
 * reports it. */
hipError_t deltanet_chunk_prefill(const void* q, const void* k, const void* v, const float* g,
                                  const float* beta, void* o, const float* initial_state,
                                  float* final_state, int B, int T, int HV, int HQK, int DK,
                                  int DV, int chunk_size, void* workspace, size_t workspace_bytes,
                                  hipStream_t stream, int dump_debug);

/* Outcome of the last prefill call (any deltanet_chunk_prefill* entry) that
 * used this workspace: synchronises `stream`, then returns hipSuccess, or
 * hipErrorLaunchTimeOut when one of that call's bounded waits gave up (its o
 * and final state are incomplete).  No counterpart in the reference, whose
 * kernels do not wait on one another. */
hipError_t deltanet_prefill_status(const void* workspace, size_t workspace_bytes,
                                   hipStream_t stream);

/* Names of the reference's bf16-wmma o-pass twin (kernels/chunk_delta_cuda_tco.h:39,47);
 * same implementation and workspace as the two entries above. */
size_t deltanet_tcop_prefill_workspace_size(int B, int T, int HV, int DK, int DV, int chunk_size);
hipError_t deltanet_tcop_chunk_prefill(const void* q, const void* k, const void* v,
                                       const float* g, const float* beta, void* o,
                                       const float* initial_state, float* final_state, int B,
                                       int T, int HV, int HQK, int DK, int DV, int chunk_size,
                                       void* workspace, size_t workspace_bytes,
                                       hipStream_t stream, int dump_debug);

/* Fused prefill on raw inputs.  Replaces the reference's TensorRT adapter
 * runGdnChunkPrefillSm87 (export/patches/orin_text_engine/files/cpp/kernels/
 * gdnKernels/gdnChunkPrefillSm87.cu:189-316), which runs separate kernels for
 * the q/k L2 norm, the fp16 -> bf16 conversions, the gate math, the prefill,
 * the bf16 -> fp16 conversion of o and a copy of the final state; here the
 * prefill's two kernels do all of it while loading and storing.
 *   q, k    : [B, T, HQK, 128] raw (not normalised); each row is scaled by
 *             rsqrt(sum x^2 + 1e-6) in fp32 and rounded to bf16
 *   v       : [B, T, HV, 128] (rounded to bf16)
 *   a, b    : [B, T, HV]; A_log: fp32 [HV]; dt_bias: [HV]
 *             g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b), fp32
 *   o       : [B, T, HV, 128] (out; the bf16-rounded value)
 *   state   : fp32 [B, HV, 128, 128], the initial state on entry and the
 *             final state on return (the adapter's h0_source)
 * q, k, v, a, b, dt_bias and o share io_dtype (GDN_DTYPE_FP16 as in the
 * plugin, or GDN_DTYPE_BF16).  The workspace is at least
 * deltanet_prefill_live_workspace_size bytes for the same B, T, HV. */
hipError_t deltanet_chunk_prefill_fused(const void* q, const void* k, const void* v,
                                        const void* a, const void* b, const float* A_log,
                                        const void* dt_bias, void* o, float* state, int B, int T,
                                        int HV, int HQK, int io_dtype, void* workspace,
                                        size_t workspace_bytes, hipStream_t stream);

/* Prefill followed by the gated RMSNorm (the reference runs that post-op as a
 * separate TensorRT plugin, kernel::gatedRmsNormForward,
 * export/patches/orin_text_engine/files/cpp/kernels/gatedRmsNorm/gatedRmsNormKernel.h:17-18,
 * after the prefill).  Same arguments as deltanet_chunk_prefill (dump_debug = 0)
 * plus z (bf16 [B, T, HV, 128]), norm_weight (bf16 [128]) and eps; y (bf16
 * [B, T, HV, 128]) receives gated_rmsnorm(o, z) = bf16(bf16(w * bf16(o *
 * rsqrt(mean(o^2) + eps))) * silu(z)), o being the bf16 output of
 * deltanet_chunk_prefill: the prefill writes o into y and the gated RMSNorm
 * kernel rewrites it in place.  Workspace as for deltanet_chunk_prefill. */
hipError_t deltanet_chunk_prefill_norm(const void* q, const void* k, const void* v,
                                       const float* g, const float* beta, const void* z,
                                       const void* norm_weight, float eps, void* y,
                                       const float* initial_state, float* final_state, int B,
                                       int T, int HV, int HQK, int DK, int DV, int chunk_size,
                                       void* workspace, size_t workspace_bytes,
                                       hipStream_t stream);

/* deltanet_chunk_prefill_norm with the gated RMSNorm inside the scan (no
 * counterpart in the reference): each of the 8 work-groups that share a row's
 * 128 columns writes its o columns of a chunk and counts itself in with a
 * device-scope atomic; the group that completes the count normalises that
 * chunk of the head in place, with the standalone kernel's arithmetic.  No
 * group waits on another.  Where the plain prefill would take the paired
 * 32-column scan (more slice groups than CUs) this runs
 * deltanet_chunk_prefill_norm's two kernels.  Same arguments and the same
 * bits as deltanet_chunk_prefill_norm; slower than it (opt-in). */
hipError_t deltanet_chunk_prefill_norm_fused(const void* q, const void* k, const void* v,
                                             const float* g, const float* beta, const void* z,
                                             const void* norm_weight, float eps, void* y,
                                             const float* initial_state, float* final_state,
                                             int B, int T, int HV, int HQK, int DK, int DV,
                                             int chunk_size, void* workspace,
                                             size_t workspace_bytes, hipStream_t stream);

/* Variable-length prefill (no counterpart in the reference kernel: its torch
 * fallback drops cu_seqlens, transformers modeling_qwen3_5.py:259).
 * q, k, v, g, beta, o are packed [1, total_tokens, H, D]; cu_seqlens is a
 * device int32 [num_seqs + 1], normally cu_seqlens[0] = 0, non-decreasing,
 * cu_seqlens[num_seqs] = total_tokens; initial_state (or NULL) and
 * final_state are [num_seqs, HV, DK, DV].  Chunks never straddle sequences.
 * cu_seqlens is not read on the host; the kernels clamp every value into
 * [0, total_tokens] and each sequence's end to no earlier than its start, and
 * never form a chunk past the workspace's bound, so a malformed cu_seqlens
 * gives wrong results but no access out of bounds. */
size_t deltanet_prefill_varlen_workspace_size(int total_tokens, int num_seqs, int HV, int DK,
                                              int DV, int chunk_size);
size_t deltanet_prefill_varlen_live_workspace_size(int total_tokens, int num_seqs, int HV,
                                                   int DK, int DV, int chunk_size);
hipError_t deltanet_chunk_prefill_varlen(const void* q, const void* k, const void* v,
                                         const float* g, const float* beta, void* o,
                                         const float* initial_state, float* final_state,
                                         const int32_t* cu_seqlens, int num_seqs,
                                         int total_tokens, int HV, int HQK, int DK, int DV,
                                         int chunk_size, void* workspace,
                                         size_t workspace_bytes, hipStream_t stream,
                                         int dump_debug);

/* deltanet_chunk_prefill (cu_seqlens NULL: B sequences of T tokens) or
 * deltanet_chunk_prefill_varlen (cu_seqlens set, B = 1, T = total tokens)
 * with raw bf16 q and k rows, L2-normalised inside the kernels as
 * x rsqrt(sum x^2 + 1e-6) in fp32 and rounded to bf16 -- transformers'
 * use_qk_l2norm_in_kernel=True (models/qwen3_5/modeling_qwen3_5.py:242-245,
 * 270-271).  No counterpart in the reference kernel, whose callers normalise
 * first (kernels/chunk_delta_cuda.h:23-25).  Workspace as for the entry it
 * mirrors. */
hipError_t deltanet_chunk_prefill_l2norm(const void* q, const void* k, const void* v,
                                         const float* g, const float* beta, void* o,
                                         const float* initial_state, float* final_state,
                                         const int32_t* cu_seqlens, int num_seqs, int B, int T,
                                         int HV, int HQK, void* workspace,
                                         size_t workspace_bytes, hipStream_t stream);

/* Recurrent step (decode; T >= 1 tokens per sequence), state updated in
 * place.  Fused native form of the torch token recurrence the reference runs
 * for decode (transformers modeling_qwen3_5.py:331-380,
 * torch_recurrent_gated_delta_rule); the reference ships no native decode. */
hipError_t deltanet_recurrent_step(const void* q, const void* k, const void* v, const float* g,
                                   const float* beta, void* o, float* state, int B, int T, int HV,
                                   int HQK, int DK, int DV, hipStream_t stream);

/* deltanet_recurrent_step with raw bf16 q and k rows, L2-normalised in the
 * kernel as in deltanet_chunk_prefill_l2norm (transformers'
 * use_qk_l2norm_in_kernel=True for decode, modeling_qwen3_5.py:343-345). */
hipError_t deltanet_recurrent_step_l2norm(const void* q, const void* k, const void* v,
                                          const float* g, const float* beta, void* o,
                                          float* state, int B, int T, int HV, int HQK, int DK,
                                          int DV, hipStream_t stream);

/* Gated RMSNorm y = rmsnorm(x) * w * silu(z) over rows of dv elements.
 * Replaces kernel::gatedRmsNormForward (export/patches/orin_text_engine/files/
 * cpp/kernels/gatedRmsNorm/gatedRmsNormKernel.h:17-18), which was fp16-only.
 * io_dtype (x, z, y): GDN_DTYPE_BF16 or GDN_DTYPE_FP16; w_dtype: io_dtype or
 * GDN_DTYPE_FP32 (selects transformers' rounding of w * n).
 * dv in {64, 128, 256, 512}. */
hipError_t gdn_gated_rmsnorm_forward(const void* x, const void* z, const void* w, void* y,
                                     int64_t rows, int dv, float eps, int io_dtype, int w_dtype,
                                     hipStream_t stream);

/* Causal depthwise conv1d over time with optional SiLU (no counterpart in the
 * reference's kernels: the step upstream of q/k/v that transformers runs as
 * causal_conv1d_fn, models/qwen3_5/modeling_qwen3_5.py:219-240,470-476).
 * x, y: [B][T][D] of io_dtype (GDN_DTYPE_BF16 or GDN_DTYPE_FP16) with
 * channels contiguous and the given batch / token strides (elements,
 * multiples of 8; 16-byte aligned bases); w: [D][K] and bias: [D] (or NULL)
 * of w_dtype (io_dtype or GDN_DTYPE_FP32).  D a multiple of 8, K in 2..4,
 * silu 0 or 1.  Tokens before the first are zero.
 * y = io(act(w_dtype(sum_j w[j] x[t-K+1+j] + bias))), the sum in fp32 with
 * the taps oldest first and the bias last. */
hipError_t gdn_causal_conv1d_fwd(const void* x, const void* w, const void* bias, void* y, int B,
                                 int T, int D, int K, int64_t x_bstride, int64_t x_tstride,
                                 int64_t y_bstride, int64_t y_tstride, int io_dtype, int w_dtype,
                                 int silu, hipStream_t stream);

/* Decode-time update of the same conv (causal_conv1d_update,
 * modeling_qwen3_5.py:199-216,457-463): the window is conv_state's state_len
 * tokens followed by the T new ones; y gets the last T outputs and conv_state
 * (updated in place) the window's last state_len tokens.  x, y: [B][D][T]
 * and conv_state: [B][D][state_len], all io_dtype, with the given strides
 * (elements; the state's token stride is 1); state_len in K-1..8; dtypes,
 * K and silu as in gdn_causal_conv1d_fwd. */
hipError_t gdn_causal_conv1d_update(const void* x, void* conv_state, const void* w,
                                    const void* bias, void* y, int B, int T, int D, int K,
                                    int state_len, int64_t x_bstride, int64_t x_tstride,
                                    int64_t x_dstride, int64_t s_bstride, int64_t s_dstride,
                                    int64_t y_bstride, int64_t y_tstride, int64_t y_dstride,
                                    int io_dtype, int w_dtype, int silu, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* GDN_HIP_H_ */
