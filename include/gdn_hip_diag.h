/*
 * Diagnostic entry points of libgdn_hip.so: per-kernel timing, a bounded-wait
 * test hook, the host mirror of the varlen chunk bookkeeping and an HBM
 * streaming probe.  None is part of the drop-in boundary (include/gdn_hip.h)
 * and none has a counterpart in the reference; benchmarks and tests use them.
 * Conventions as in gdn_hip.h.
 */
#ifndef GDN_HIP_DIAG_H_
#define GDN_HIP_DIAG_H_

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Per-kernel timing of deltanet_chunk_prefill (for benchmarks that attribute
 * time to each kernel).  deltanet_prefill_kernel_count() kernels are launched;
 * events[i] is recorded on `stream` before kernel i and events[count] after
 * the last, so hipEventElapsedTime(events[i], events[i + 1]) is kernel i's
 * duration.  n_events must equal count + 1; the other arguments are as in
 * deltanet_chunk_prefill (dump_debug = 0). */
int deltanet_prefill_kernel_count(void);
const char* deltanet_prefill_kernel_name(int i);
hipError_t deltanet_chunk_prefill_timed(const void* q, const void* k, const void* v,
                                        const float* g, const float* beta, void* o,
                                        const float* initial_state, float* final_state, int B,
                                        int T, int HV, int HQK, int DK, int DV, int chunk_size,
                                        void* workspace, size_t workspace_bytes,
                                        hipStream_t stream, hipEvent_t* events, int n_events);

/* One kernel of deltanet_chunk_prefill on its own (for benchmarks that time
 * back-to-back launches of a single kernel).  kernel 0 (prep) fills the
 * workspace from the inputs; kernel 1 (scan) reads a workspace that kernel 0
 * filled for the same arguments and writes o and final_state.  Arguments as
 * in deltanet_chunk_prefill (dump_debug = 0); kernel outside
 * [0, deltanet_prefill_kernel_count()) returns hipErrorInvalidValue. */
hipError_t deltanet_chunk_prefill_kernel(const void* q, const void* k, const void* v,
                                         const float* g, const float* beta, void* o,
                                         const float* initial_state, float* final_state, int B,
                                         int T, int HV, int HQK, int DK, int DV, int chunk_size,
                                         void* workspace, size_t workspace_bytes,
                                         hipStream_t stream, int kernel);

/* deltanet_chunk_prefill (DK = DV = 128, chunk 64, dump_debug = 0) with the
 * scan's bounded waits limited to spin_limit polls each (the library's own
 * limit is 2^20).  With a small limit the waits give up, every kernel still
 * returns normally, and deltanet_prefill_status then reports
 * hipErrorLaunchTimeOut: the test of that error path. */
hipError_t deltanet_chunk_prefill_spin(const void* q, const void* k, const void* v,
                                       const float* g, const float* beta, void* o,
                                       const float* initial_state, float* final_state, int B,
                                       int T, int HV, int HQK, void* workspace,
                                       size_t workspace_bytes, hipStream_t stream,
                                       unsigned spin_limit);

/* deltanet_chunk_prefill / _varlen (DK = DV = 128, chunk 64, dump_debug = 0)
 * with the scan instance chosen by the caller: slice_cols 16 runs one scan
 * work-group per 16 value columns of a (sequence, head), 32 the paired
 * instance with one per 32 columns, 0 the library's own choice (16 while the
 * 16-column groups fit on the device's CUs at once, 32 beyond).  Both give
 * bitwise the same o and final state.  cu_seqlens NULL: num_seqs sequences of
 * T tokens; otherwise a device array [num_seqs + 1] and T the total token
 * count.  spin_limit 0 keeps the library's bounded-wait limit, otherwise as in
 * deltanet_chunk_prefill_spin.  Other slice_cols: hipErrorInvalidValue. */
hipError_t deltanet_chunk_prefill_cols(const void* q, const void* k, const void* v,
                                       const float* g, const float* beta, void* o,
                                       const float* initial_state, float* final_state,
                                       const int32_t* cu_seqlens, int num_seqs, int T, int HV,
                                       int HQK, void* workspace, size_t workspace_bytes,
                                       hipStream_t stream, int slice_cols, unsigned spin_limit);

/* Host mirror of the kernels' sequence bookkeeping for a packed batch
 * (host memory, no GPU involved): for each sequence s its first chunk id,
 * the chunks the scan processes (never past the workspace's chunk bound),
 * its first token and its token count after clamping cu_seqlens into
 * [0, total_tokens].  Returns the workspace's chunk bound per head, or -1 for
 * invalid arguments.  Runs the same code as the kernels (gdn_seq.h). */
int deltanet_varlen_chunk_map(const int32_t* cu_seqlens, int num_seqs, int total_tokens,
                              int32_t* seq_first_chunk, int32_t* seq_chunk_count,
                              int32_t* seq_first_token, int32_t* seq_token_count);

/* Host twins of the kernels' block-cooperative lookups over a packed batch
 * (host memory, no GPU involved), run phase by phase for `nt` simulated
 * threads with the kernels' shared arithmetic (gdn_seq.h):
 *   deltanet_varlen_chunks_before  the scan's chunk count of sequences
 *       [0, upto) (saturating at 2^30), nt a multiple of 64 up to 1024;
 *   deltanet_varlen_locate_chunk   the prep's global chunk id -> sequence,
 *       first token and row count, written to seq_tok_rows[0..2]; returns 1
 *       when found, 0 when the chunk does not exist, nt a power of two up to
 *       1024 (the prep runs 256).
 * Both return -1 for invalid arguments. */
int deltanet_varlen_chunks_before(const int32_t* cu_seqlens, int num_seqs, int total_tokens,
                                  int upto, int nt);
int deltanet_varlen_locate_chunk(const int32_t* cu_seqlens, int num_seqs, int total_tokens,
                                 int cid, int nt, int32_t* seq_tok_rows);

/* Two-level chunk-group scan (prototype for measurement; same results as
 * deltanet_chunk_prefill / _varlen to rounding).  Each sequence's chunks are
 * cut into `segments` chunk-aligned segments; pass 1 scans every segment
 * from a zero state (end state B_j) and from the identity with v = 0 (the
 * segment's transition Phi_j), a combine kernel forms the entry states
 * E_j = Phi_{j-1} E_{j-1} + B_{j-1} in fp32, and a replay scans every segment
 * from E_j.  cu_seqlens_host is HOST memory [num_seqs + 1] (well-formed,
 * starting at 0), or NULL for num_seqs sequences of T tokens; T is the total
 * token count when it is given.  The call synchronises `stream` once to copy
 * its segment table.  events: NULL, or 6 events recorded at the start and
 * after the prep, pass 1 (B), pass 1 (Phi), the combine and the replay.  No
 * counterpart in the reference (its carry kernel is the plain serial scan,
 * kernels/chunk_delta_cuda.cu:348-417). */
size_t deltanet_prefill_twolevel_workspace_size(const int32_t* cu_seqlens_host, int num_seqs,
                                                int T, int HV, int segments);
hipError_t deltanet_chunk_prefill_twolevel(const void* q, const void* k, const void* v,
                                           const float* g, const float* beta, void* o,
                                           const float* initial_state, float* final_state,
                                           const int32_t* cu_seqlens_host, int num_seqs, int T,
                                           int HV, int HQK, int segments, void* workspace,
                                           size_t workspace_bytes, hipStream_t stream,
                                           hipEvent_t* events, int n_events);

/* HBM streaming probe (benchmarks only): kind 0 reads a and b and writes
 * c = a ^ b, `bytes` each (three streams, the gated RMSNorm's pattern);
 * kind 1 reads and rewrites c in place (the decode state's pattern).
 * nontemporal != 0 uses non-temporal loads and stores.  For kinds 0 and 1
 * `blocks` work-groups of 256 threads stride over the 16-byte vectors.  Kind
 * 2 is kind 0 in the gated RMSNorm's own launch shape, one pass with no loop:
 * each of the 256 threads of ceil(bytes / (4096 P)) work-groups moves
 * P = `blocks` (1..4) vectors, 256 vectors apart.  bytes must be a nonzero
 * multiple of 16, otherwise hipErrorInvalidValue. */
hipError_t gdn_stream_probe(int kind, int nontemporal, const void* a, const void* b, void* c,
                            size_t bytes, int blocks, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* GDN_HIP_DIAG_H_ */
