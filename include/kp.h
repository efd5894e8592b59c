/*
 * kp.h -- C ABI of the MI355X (gfx950) fused graph-fragment kernels.
 *
 * The reference (SherlockNoMad/KernelProblems) is a corpus of torch graph
 * fragments; each fragment's drop-in contract is a Python
 * `kernel_function(*inputs) -> outputs` whose results must match the
 * fragment's `Model.forward` (e.g. v8/7884328a5557/optimized_kernel.py:37-55
 * against v8/7884328a5557/problem.py:9-33).  The aten operators those
 * fragments are built from are what this library replaces; the Python layer in
 * kernelproblems_amd/ binds these entry points with ctypes and rebuilds each
 * fragment's exact signature on top of them.
 *
 * Conventions shared by every entry point:
 *  - All pointers are device pointers (HIP global memory) except the small
 *    host arrays `*_terms` / `*_strides`, which are read before return.
 *  - bf16 tensors are passed as raw 16-bit storage (`void*`); strides are in
 *    elements, never bytes.  The innermost dimension is always unit-stride.
 *  - `stream` is a hipStream_t (NULL = the legacy default stream).  Every call
 *    only enqueues work: no host synchronisation, no allocation; scratch memory
 *    comes from the caller through (workspace, workspace_bytes).
 *  - Calls on distinct streams with distinct workspaces are independent;
 *    calls that share a workspace must be ordered by the caller.
 *  - Return value: KP_OK or one of the KP_E* codes below; on KP_EHIP,
 *    kp_last_hip_error() returns the hipError_t of the failed launch.
 */
#ifndef KP_H_
#define KP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KP_OK 0
#define KP_EINVAL 1        /* rejected argument: null pointer, shape, stride, alignment, dtype code */
#define KP_EUNSUPPORTED 2  /* valid call outside what this build implements (message via kp_last_error_message) */
#define KP_EHIP 3          /* a HIP runtime call or launch failed */
#define KP_EWORKSPACE 4    /* workspace_bytes smaller than the matching *_workspace_size() */
#define KP_EBUSY 5         /* kp_rmsnorm_bwd_bf16_noalloc: an unfinished call on another stream holds the scratch */

#define KP_DTYPE_F32 0
#define KP_DTYPE_BF16 1

#define KP_ROPE_HALF 0        /* rotate-half pairing: (i, i + D/2) */
#define KP_ROPE_INTERLEAVED 1 /* complex pairing: (2i, 2i + 1) */

/* Library identification and error reporting (per calling thread). */
const char* kp_version(void);
int kp_last_hip_error(void);
const char* kp_last_error_message(void);

/* Benchmark timing hook (no counterpart in the reference, whose timing lives
 * in an external harness).  While set, every entry point launches its
 * dominant kernel with hipExtLaunchKernel, which stamps start_event and
 * stop_event (hipEvent_t, timing enabled) at that kernel's own start and
 * completion: the row kernel of the RMSNorm entry points (and of
 * kp_embedding_rmsnorm_fwd_bf16), the gather kernel
 * of kp_embedding_fwd_bf16, the whole four-launch pipeline of kp_embedding_bwd_bf16
 * (start event at its first kernel's start, stop event at its last kernel's end),
 * the kernel of kp_rope_bf16 (and of kp_rope_c64), the copy kernel of kp_unshard_bf16, the
 * kernels of kp_swiglu_fwd_bf16 / kp_swiglu_bwd_bf16 / kp_silu_bf16 / kp_swiglu_fwd_bwd_bf16, the row kernel of
 * kp_cross_entropy_fwd_bf16, the kernel of kp_cross_entropy_bwd_bf16, the row
 * kernel of kp_cross_entropy_fwd_bwd_bf16 and
 * the kernel of kp_stream_probe.
 * Pass NULL, NULL to clear.  Per calling thread. */
void kp_profile_dominant_kernel(void* start_event, void* stop_event);

/* Block timeline hook (measurement only; no counterpart in the reference).
 * While set, the vectorized RMSNorm backward row kernel (the dominant kernel
 * of kp_rmsnorm_bwd_bf16, its allocation-free form and kp_rmsnorm_fwd_bwd_bf16
 * on 16-byte rows of N a multiple of 512) writes, for each row block b below
 * bytes / 32, four 64-bit words starting at word 4 b of buf: the device's
 * constant 100 MHz clock (s_memrealtime) when the block
 * starts, when its last row's stores have completed, and when its
 * weight-gradient partial row has been stored, then the XCC id the block ran
 * on.  buf is device memory; pass NULL (or bytes < 32) to clear.  Per calling
 * thread, like kp_profile_dominant_kernel. */
void kp_debug_block_trace(void* buf, size_t bytes);

/* ------------------------------------------------------------------------
 * RMSNorm forward, optionally fused with the residual add in front of it.
 *
 * Replaces torch.ops.aten._fused_rms_norm.default as called at
 *   v7/59f786beb25f/problem.py:16      (returns y and rstd)
 *   v8/4b90e2d83144/problem.py:16      (y only, returned as views)
 *   v7/215dd2e6a519/problem.py:16-25   (weight = strided [8,512] view of an FSDP flat buffer)
 * and the add.Tensor -> _fused_rms_norm region of
 *   v8/7884328a5557/problem.py:20-33   (h = add_61 + mm_220, y = rms(h)).
 *
 * x_terms[0..n_x), 1 <= n_x <= 3: bf16 [M, N] tensors with row strides
 *   x_strides[]; the normalised row is h = bf16(bf16(x0 + x1) + x2), each add
 *   computed in fp32 and rounded to bf16 (eager bf16 add.Tensor), or x0.
 * h_out (bf16 [M, N], row stride h_stride): receives h when n_x > 1; may be NULL.
 * weight: bf16; element i is weight[(i / w_seg_len) * w_seg_stride + i % w_seg_len]
 *   (a contiguous weight has w_seg_len = N); NULL means no weight.
 * y (bf16 [M, N], row stride y_stride) = bf16(fp32(h) * rstd * fp32(w)).
 * rstd (fp32 [M], may be NULL) = 1 / sqrt(sum(h^2) / N + eps).
 */
int kp_rmsnorm_fwd_bf16(const void* const* x_terms, const int64_t* x_strides, int n_x,
                        const void* weight, int64_t w_seg_len, int64_t w_seg_stride,
                        void* h_out, int64_t h_stride,
                        void* y, int64_t y_stride,
                        float* rstd,
                        int64_t M, int64_t N, float eps, void* stream);

/* ------------------------------------------------------------------------
 * RMSNorm backward with its neighbouring elementwise ops fused in.
 *
 * Replaces torch.ops.aten._fused_rms_norm_backward.default (+ _to_copy of the
 * weight gradient) as called at
 *   v7/45990c83cfd6/problem.py:17-28   (rstd recomputed by a forward; dx, dw bf16)
 *   v8/d8f596b3df34/problem.py:26-45   (dy = mm_664 + mm_666; out = add_218 + dx; dw -> f32)
 *   v7/ed20955ec34b/problem.py          (dy = (view_1794 + mm_672) + mm_674)
 *   v8/3c6c589cdf81/problem.py:22-53   (x = (add_61 + mm_220) + mm_223 recomputed, rstd recomputed)
 * following the decomposition torch/_decomp/decompositions.py:1815-1887.
 *
 * dy = bf16 running sum of dy_terms[0..n_dy), x = bf16 running sum of
 * x_terms[0..n_x) (both 1..3 terms, rounding as in kp_rmsnorm_fwd_bf16).
 * rstd: fp32 [M] as produced by the forward; NULL = recompute from x with eps.
 * dx = bf16((g - xhat * sum(xhat * g) / N) * rstd), g = dy * w, xhat = x * rstd;
 *   if dx_residual != NULL the stored value is bf16(dx_residual + bf16(dx)).
 * dw[j] = sum over rows of dy * xhat, accumulated in fp32 with a fixed
 *   two-stage order (run-to-run bitwise deterministic).  Written to dw_f32
 *   (fp32 [N]; rounded to bf16 first when dw_f32_round_bf16 != 0, the
 *   reference's bf16 -> _to_copy(f32)) and/or dw_bf16 (bf16 [N]).  Both may be
 *   NULL; weight must be non-NULL whenever either is requested.
 * dx may be one of the bf16 inputs itself (a dy term or dx_residual, same
 *   base and row stride: the residual gradient accumulated in place); each
 *   row is read by the waves that write it.  Partial overlap is undefined.
 * workspace: at least kp_rmsnorm_bwd_workspace_size(M, N) bytes, 16-byte aligned.
 */
size_t kp_rmsnorm_bwd_workspace_size(int64_t M, int64_t N);
int kp_rmsnorm_bwd_bf16(const void* const* dy_terms, const int64_t* dy_strides, int n_dy,
                        const void* const* x_terms, const int64_t* x_strides, int n_x,
                        const float* rstd,
                        const void* weight, int64_t w_seg_len, int64_t w_seg_stride,
                        const void* dx_residual, int64_t dxr_stride,
                        void* dx, int64_t dx_stride,
                        float* dw_f32, void* dw_bf16, int dw_f32_round_bf16,
                        int64_t M, int64_t N, float eps,
                        void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * RMSNorm backward that allocates nothing and takes no workspace.
 *
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): the same computation and arguments as
 * kp_rmsnorm_bwd_bf16, with the weight-gradient partial rows kept in a static
 * device array of kp_rmsnorm_bwd_noalloc_max_bytes() bytes (8 MiB) that each
 * GPU holds until the process ends.  The partial rows take one fp32 row of N
 * per row block, and the row-block count is the device's CU count times the
 * blocks per CU (1 by default; the KP_RMS_BWD_BPC tuning knob raises it): on
 * a 256-CU MI355X at the default that is room for N <= 8192, every
 * configuration here.  A shape whose partial rows do not fit returns
 * KP_EUNSUPPORTED before launching anything.  Every call on one GPU shares
 * that GPU's array: calls ordered on one stream are safe; a call on a
 * different stream while the previous call on that GPU has not finished
 * returns KP_EBUSY and launches nothing (the library records an event after
 * each call's launches and queries it; the first call on a device creates
 * that event and looks up the array's address).  A stream under graph
 * capture is not guarded: the caller orders captured calls.  No hipMalloc,
 * hipFree or hipMemset is made.
 */
size_t kp_rmsnorm_bwd_noalloc_max_bytes(void);
int kp_rmsnorm_bwd_bf16_noalloc(const void* const* dy_terms, const int64_t* dy_strides, int n_dy,
                                const void* const* x_terms, const int64_t* x_strides, int n_x,
                                const float* rstd,
                                const void* weight, int64_t w_seg_len, int64_t w_seg_stride,
                                const void* dx_residual, int64_t dxr_stride,
                                void* dx, int64_t dx_stride,
                                float* dw_f32, void* dw_bf16, int dw_f32_round_bf16,
                                int64_t M, int64_t N, float eps, void* stream);

/* ------------------------------------------------------------------------
 * RMSNorm forward and backward of the same rows in one row pass.
 *
 * Replaces the _fused_rms_norm -> _fused_rms_norm_backward region (plus the
 * gradient adds in front of the backward and the residual add after it) of
 *   v6/0b493aad68f0/problem.py:16-47   (y returned as 3 views; dy = (mm_670 + mm_672) + mm_674;
 *                                       out = add_220 + dx feeds embedding_dense_backward)
 *   v5/118d525f44e0/problem.py:16-50   (the same chain over a flat-buffer weight view)
 *   v6/822931829090/problem.py:10-66   (y as 3 views, 3-term dy, residual)
 *   v6/408ac0979ac5/problem.py:10-63   (x = embedding + mm_3 recomputed, 2-term dy, residual)
 *   v6/e9198b707240/problem.py          (2-term dy, residual)
 * where the forward's rstd is used only by the backward.  Every argument has
 * its kp_rmsnorm_bwd_bf16 meaning (there is no rstd input: it is recomputed
 * from x with eps); in addition the same pass writes
 *   y (bf16 [M, N], row stride y_stride) = bf16(fp32(x) * rstd * fp32(w)),
 *   h_out (bf16 [M, N], may be NULL) = the summed x terms when n_x > 1,
 *   rstd_out (fp32 [M], may be NULL) = the rstd both halves used,
 * reading x once where the two-operator sequence reads it twice.
 * workspace: at least kp_rmsnorm_fwd_bwd_workspace_size(M, N) bytes, 16-byte aligned.
 */
size_t kp_rmsnorm_fwd_bwd_workspace_size(int64_t M, int64_t N);
int kp_rmsnorm_fwd_bwd_bf16(const void* const* dy_terms, const int64_t* dy_strides, int n_dy,
                            const void* const* x_terms, const int64_t* x_strides, int n_x,
                            const void* weight, int64_t w_seg_len, int64_t w_seg_stride,
                            void* h_out, int64_t h_stride,
                            void* y, int64_t y_stride,
                            float* rstd_out,
                            const void* dx_residual, int64_t dxr_stride,
                            void* dx, int64_t dx_stride,
                            float* dw_f32, void* dw_bf16, int dw_f32_round_bf16,
                            int64_t M, int64_t N, float eps,
                            void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Token embedding fused into the RMSNorm forward that consumes it:
 *   h[t, :] = table[indices[t], :]   (bit copy; written only when h_out != NULL)
 *   y[t, :] = bf16(fp32(h) * rstd_t * fp32(w)),  rstd_t = 1 / sqrt(sum(h^2) / N + eps)
 * in one launch: the gathered rows go straight from the table into the norm's
 * registers instead of through an HBM intermediate.
 *
 * Replaces embedding.default -> _fused_rms_norm.default at
 * v8/12545c1e9b06/problem.py:24-42 (table = [128256, 4096] view of an FSDP
 * flat buffer, ids i64 [1, 8192], the norm weight read in place from the
 * layer buffer).  table: bf16 [V, N] rows (row stride table_row_stride);
 * indices: T integers of index_bytes (4 or 8); weight as in
 * kp_rmsnorm_fwd_bf16; y / h_out: bf16 [T, N] with the given row strides;
 * rstd: fp32 [T] or NULL.  An index outside [0, V) contributes nothing (row 0
 * is read in its place and discarded): its h and y rows are zero and, when
 * error_flag != NULL, *error_flag is set to 1.
 * Rows, strides and pointers must be 16-byte granular with N a fast-path row
 * length; otherwise KP_EUNSUPPORTED (compose kp_embedding_fwd_bf16 and
 * kp_rmsnorm_fwd_bf16 instead).
 */
int kp_embedding_rmsnorm_fwd_bf16(const void* table, int64_t V, int64_t table_row_stride, const void* indices,
                                  int index_bytes, int64_t T, const void* weight, int64_t w_seg_len,
                                  int64_t w_seg_stride, void* h_out, int64_t h_stride, void* y, int64_t y_stride,
                                  float* rstd, int64_t N, float eps, int32_t* error_flag, void* stream);

/* ------------------------------------------------------------------------
 * Streaming-ceiling probe (a measurement aid; no counterpart in the
 * reference).  Reads n_in (0..4) arrays of in_bytes each and writes n_out
 * (1..2; or 3 with n_in = 3) arrays of out_bytes each (sizes multiples of 16
 * below 4 GiB, arrays 16-byte aligned) with the fragment kernels' access
 * form: 16-byte non-temporal loads, 1 KiB per wave instruction, one-shot grid
 * of 256-thread blocks holding chunks_per_thread (1, 2, 4 or 8) chunks per
 * thread per array, stores non-temporal (KP_STORE_NONTEMPORAL) or
 * device-scope write-through (KP_STORE_WRITE_THROUGH).  Inputs shorter than
 * the outputs read as zeros past their end.  bench.py times it on each
 * workload's byte mix under every tile size and store policy and reports the
 * fastest as the bandwidth plain streaming of those bytes reaches on this GPU.
 */
#define KP_STORE_NONTEMPORAL 0
#define KP_STORE_WRITE_THROUGH 1
int kp_stream_probe(const void* const* in, int n_in, int64_t in_bytes, void* const* out, int n_out,
                    int64_t out_bytes, int chunks_per_thread, int store_policy, void* stream);

/* ------------------------------------------------------------------------
 * Embedding forward: out[t, :] = table[indices[t], :] (bit copy).
 *
 * Replaces torch.ops.aten.embedding.default at v7/1e49beb8a123/problem.py:23
 * (table = [128256, 4096] view of an FSDP flat buffer, ids i64 [1, 8192]).
 * indices: T integers of index_bytes (4 or 8) each, contiguous.
 * An index outside [0, V) gives a zero-filled output row (the 16-byte path
 * reads table row 0 in its place and masks it away) and, when
 * error_flag != NULL, sets *error_flag to 1 (never cleared here).
 * One wave per token: T above 4 * (2^31 - 1) tokens on the 16-byte path
 * returns KP_EUNSUPPORTED.
 */
int kp_embedding_fwd_bf16(const void* table, int64_t V, int64_t D, int64_t table_row_stride,
                          const void* indices, int index_bytes, int64_t T,
                          void* out, int64_t out_row_stride,
                          int32_t* error_flag, void* stream);

/* ------------------------------------------------------------------------
 * Embedding backward, dense: G[v, :] = sum over {t : indices[t] == v,
 * v != padding_idx} of grad[t, :] (divided by the id's count when
 * scale_grad_by_freq), accumulated in fp32; every row of G is written (rows
 * without contributions as zeros; rows of the zero shares filled by the first
 * two launches are written as zeros first, then their sums when touched).
 *
 * Replaces torch.ops.aten.embedding_dense_backward.default (+ _to_copy f32)
 * at v7/a12a160cb11b/problem.py:16-20, following the decomposition
 * torch/_decomp/decompositions.py:1245-1275.
 *
 * Deterministic sort-and-segment: (id, t) keys are sorted; the sorted order
 * is cut into windows of 32 keys, each id's contributions inside a window are
 * summed in fp32 in ascending t, and an id whose keys span several windows
 * adds its window partial sums in window order.  No float atomics; the result
 * is bitwise reproducible run to run.
 * grad: bf16 [T, D] with row stride grad_row_stride.  indices as above.
 * grad_table: [V, D] contiguous, out_dtype KP_DTYPE_F32 or KP_DTYPE_BF16; with
 *   KP_DTYPE_F32 and out_round_bf16 != 0 every value is first rounded to bf16.
 * padding_idx < 0 means none.  Out-of-range ids are skipped and flagged.
 * Limits of this build: T < 2^31 (KP_EUNSUPPORTED otherwise); any V -- the
 *   sort keys hold ids below 2^21 - 1, so a larger vocabulary runs the
 *   pipeline once per slab of that many rows, each pass writing its slab.
 */
size_t kp_embedding_bwd_workspace_size(int64_t T, int64_t V, int64_t D);
int kp_embedding_bwd_bf16(const void* grad, int64_t grad_row_stride,
                          const void* indices, int index_bytes, int64_t T,
                          int64_t V, int64_t D, int64_t padding_idx, int scale_grad_by_freq,
                          void* grad_table, int out_dtype, int out_round_bf16,
                          void* workspace, size_t workspace_bytes,
                          int32_t* error_flag, void* stream);

/* ------------------------------------------------------------------------
 * RMSNorm backward (optionally with its forward) whose residual-epilogue
 * output feeds the dense embedding backward of the same tokens, without that
 * output ever reaching HBM.
 *
 * Replaces the _fused_rms_norm(_backward) -> add.Tensor(add_220, dx) ->
 * embedding_dense_backward -> _to_copy chains of
 *   v6/0b493aad68f0/problem.py:16-71   (forward + backward; y returned as 3 views)
 *   v5/118d525f44e0/problem.py:16-80   (the same over a flat-buffer weight view)
 *   v8/f6251e84e3fa/problem.py:10-57   (backward from the saved rstd)
 * where add_tensor_2 = add_220 + dx is an intermediate, not an output.
 *
 * Norm: every argument has its kp_rmsnorm_bwd_bf16 meaning with one x term
 *   (x, x_stride) and dx_residual required: g = bf16(dx_residual + bf16(dx)).
 *   rstd: fp32 [M], or NULL to recompute it from x with eps; with rstd ==
 *   NULL the same pass may also write the forward's y (bf16 [M, N], row
 *   stride y_stride, may be NULL) and rstd_out (fp32 [M], may be NULL).
 * Embedding: row t of g is token t with id indices[t] (index_bytes 4 or 8);
 *   grad_table [V, N] (out_dtype KP_DTYPE_F32 or _BF16, out_round_bf16 as in
 *   kp_embedding_bwd_bf16) = for each id the fp32 sum of its tokens' g rows
 *   in ascending token order (rows of ids no token has are zero), the same
 *   bits as kp_embedding_bwd_bf16 of a stored g; ids equal to padding_idx or
 *   outside [0, V) contribute nothing (out-of-range ids set *error_flag).
 *   There is no scale_grad_by_freq (the chains pass False).
 * One row pass walks each run of equal ids in sorted order and sums g into
 * registers; rows of skipped ids still count for y and the weight gradient.
 * The weight gradient is deterministic (a fixed grouping of rows into partial
 * rows, then a fixed-order sum) but groups rows differently from
 * kp_rmsnorm_bwd_bf16, so its last bits may differ from that entry's.
 * Supported: N = 2048, 4096 or 8192, 1..3 dy terms, rows 16-byte aligned with
 * strides a multiple of 8, a 16-byte aligned weight with segment length and
 * stride multiples of 8, a 16-byte aligned grad_table, V < 2^21, M < 2^31;
 * anything else returns KP_EUNSUPPORTED (run the norm entry point and then
 * kp_embedding_bwd_bf16).
 * workspace: at least kp_rmsnorm_embedding_bwd_workspace_size(M, N, V) bytes,
 * 16-byte aligned.
 */
size_t kp_rmsnorm_embedding_bwd_workspace_size(int64_t M, int64_t N, int64_t V);
int kp_rmsnorm_embedding_bwd_bf16(const void* const* dy_terms, const int64_t* dy_strides, int n_dy,
                                  const void* x, int64_t x_stride,
                                  const float* rstd,
                                  const void* weight, int64_t w_seg_len, int64_t w_seg_stride,
                                  const void* dx_residual, int64_t dxr_stride,
                                  void* y, int64_t y_stride, float* rstd_out,
                                  float* dw_f32, void* dw_bf16, int dw_f32_round_bf16,
                                  int64_t M, int64_t N, float eps,
                                  const void* indices, int index_bytes, int64_t V, int64_t padding_idx,
                                  void* grad_table, int out_dtype, int out_round_bf16,
                                  void* workspace, size_t workspace_bytes,
                                  int32_t* error_flag, void* stream);

/* ------------------------------------------------------------------------
 * Rotary position embedding on up to two tensors (q and k) in one launch.
 *
 * Replaces the _to_copy f32 -> view_as_complex -> mul -> view_as_real ->
 * _to_copy bf16 chain of
 *   v7/e29b92927600/problem.py:16-37   (k, freqs_cis given per position)
 *   v8/c8c60d8f7015/problem.py:18-71   (q and k, freqs_cis gathered by position ids)
 *   v7/5c65f62b0422/problem.py:16-40   (backward: grad given as a transposed view)
 * and the rotate-half form of the north-star configuration.
 *
 * Tensor i (i = 0, 1; tensor 1 optional, x1 == NULL): x_i and out_i are bf16
 *   [B, S, H_i, D] with element strides {b, s, h} in x_strides_i[3] /
 *   out_strides_i[3] and unit stride on D (D even).
 * positions: NULL (position of (b, s) is s) or B*S integers of pos_bytes
 *   (4 or 8) at positions[b * pos_stride_b + s * pos_stride_s].
 * Angles: when freqs_cis == NULL, inv_freq[i] = fp32(theta^(-2i/D)) and the
 *   rotation of pair i at position p is (cos a, sin a), a = fp32(fp32(p) *
 *   inv_freq[i]), evaluated in fp32 in-kernel.  Otherwise freqs_cis is a
 *   complex64 table (interleaved float pairs) [freq_rows, D/2] with row
 *   stride freq_row_stride (complex elements) and pair i of position p uses
 *   freqs_cis[p, i] (p must lie in [0, freq_rows)).
 * pairing KP_ROPE_HALF pairs (i, i + D/2); KP_ROPE_INTERLEAVED pairs (2i, 2i+1).
 * out = (x_a * c - x_b * s, x_b * c + x_a * s) computed in fp32 and stored as
 *   bf16, or as fp32 for tensor i when bit i of out_f32_mask is set (the
 *   fragment v7/0f38bc55457c/problem.py returns its q rotation in fp32);
 *   conj != 0 uses (c, -s) (the backward of the forward rotation).
 * With a table, a position outside [0, freq_rows) contributes nothing: its
 *   output is zero and *error_flag (if non-NULL) is set to 1.
 */
int kp_rope_bf16(const void* x0, void* out0, int64_t H0, const int64_t* x0_strides, const int64_t* out0_strides,
                 const void* x1, void* out1, int64_t H1, const int64_t* x1_strides, const int64_t* out1_strides,
                 int64_t B, int64_t S, int64_t D,
                 const void* positions, int pos_bytes, int64_t pos_stride_b, int64_t pos_stride_s,
                 int pairing, double theta,
                 const float* freqs_cis, int64_t freq_rows, int64_t freq_row_stride,
                 int conj, int out_f32_mask, int32_t* error_flag, void* stream);

/* kp_rope_bf16 with every output written twice: out0_copy (and out1_copy,
 * required when x1 != NULL) receive the same values as out0 / out1, laid out
 * with the same strides, from one pass over the inputs.  Replaces the
 * fragment that rotates q and k twice and returns both pairs as separate
 * tensors:
 *   v5/ca76bd89ec38/problem.py:10-132 (and its repeat v4/6b92d6e665ab)
 * A copy may not be its own output (KP_EINVAL).
 */
int kp_rope_bf16_twice(const void* x0, void* out0, int64_t H0, const int64_t* x0_strides,
                       const int64_t* out0_strides, const void* x1, void* out1, int64_t H1,
                       const int64_t* x1_strides, const int64_t* out1_strides, int64_t B, int64_t S, int64_t D,
                       const void* positions, int pos_bytes, int64_t pos_stride_b, int64_t pos_stride_s,
                       int pairing, double theta, const float* freqs_cis, int64_t freq_rows,
                       int64_t freq_row_stride, int conj, int out_f32_mask, void* out0_copy, void* out1_copy,
                       int32_t* error_flag, void* stream);

/* ------------------------------------------------------------------------
 * Rotary position embedding on complex64 data: q and k already viewed as
 * complex (fp32 (re, im) pairs), multiplied by a complex64 table row per
 * position, complex64 out:
 *   out[b, s, h, i] = x[b, s, h, i] * t[p, i]   (* conj(t[p, i]) when conj != 0)
 *   (a + bi)(c + di) = (ac - bd) + (ad + bc)i in fp32.
 *
 * Replaces the index -> mul (-> mul) regions at
 *   v1/075cb40f3d5d/problem.py:8-27   (q and k, table gathered by position ids)
 *   v1/9cd8f72e74ce/problem.py:8-17   (q, table row s for position s, a conjugated table)
 *   v1/d7efc428b2f5/problem.py:8-406  (33 q / k pairs, one gathered table)
 * Tensor i (i = 0, 1; tensor 1 optional, x1 == NULL): x_i, out_i complex64
 *   [B, S, H_i, P] with strides {b, s, h} in complex elements and unit stride
 *   on P.  positions as in kp_rope_bf16 (NULL: position of (b, s) is s).
 *   freqs_cis: complex64 [freq_rows, >= P], row stride in complex elements.
 * A position outside [0, freq_rows) contributes nothing: its output is zero
 * and *error_flag (if non-NULL) is set to 1.
 */
int kp_rope_c64(const void* x0, void* out0, int64_t H0, const int64_t* x0_strides, const int64_t* out0_strides,
                const void* x1, void* out1, int64_t H1, const int64_t* x1_strides, const int64_t* out1_strides,
                int64_t B, int64_t S, int64_t P,
                const void* positions, int pos_bytes, int64_t pos_stride_b, int64_t pos_stride_s,
                const float* freqs_cis, int64_t freq_rows, int64_t freq_row_stride, int conj,
                int32_t* error_flag, void* stream);

/* ------------------------------------------------------------------------
 * FSDP parameter unshard: n_seg (<= 16) column ranges of a row-strided bf16
 * view src[shards, *] (row stride shard_stride) copied to contiguous outputs.
 * Segment s covers columns [col_off[s], col_off[s] + col_len[s]) of every
 * shard row and lands in dst[s] as a contiguous [shards, col_len[s]] block.
 *
 * Replaces the view -> split_with_sizes -> clone(contiguous_format) chains of
 * the per-layer parameters in v8/94985bdb7630/problem.py (and
 * v8/7815074de963, v8/12545c1e9b06, v8/8e33a91b7364), in one launch.
 */
int kp_unshard_bf16(const void* src, int64_t shards, int64_t shard_stride,
                    const int64_t* col_off, const int64_t* col_len, void* const* dst, int n_seg, void* stream);

/* ------------------------------------------------------------------------
 * SwiGLU gate forward: out = bf16(bf16(silu(a)) * b), silu(x) = x / (1 + exp(-x))
 * in fp32 (eager bf16 silu rounds its result to bf16 before the multiply).
 *
 * Replaces the silu.default -> mul.Tensor region at
 * v8/c68dae22972b/problem.py:15-28 (a = w1 output mm_4, b = w3 output mm_5,
 * bf16 [8192, 14336]).
 * a, b, out: bf16 [M, N] with unit inner stride and the given row strides
 * (elements; ignored when M == 1).  out may be one of the inputs (in place);
 * partial overlap is undefined.
 */
int kp_swiglu_fwd_bf16(const void* a, int64_t a_stride, const void* b, int64_t b_stride,
                       void* out, int64_t out_stride, int64_t M, int64_t N, void* stream);

/* ------------------------------------------------------------------------
 * SwiGLU gate backward:
 *   db = bf16(g * s)
 *   da = bf16(t * sig * (1 + a * (1 - sig))),  t = bf16(g * b),  sig = 1 / (1 + exp(-a))
 * all in fp32 from bf16 operands (aten mul.Tensor, then silu_backward).
 *
 * Replaces the mul.Tensor, mul.Tensor -> silu_backward.default region at
 * v8/385e1beb9bb9/problem.py:17-33: g = mm_662 (gradient of the gate
 * product), s = silu_recomputed, b = _unsafe_view_5_recomputed (w3 output),
 * a = _unsafe_view_4_recomputed (w1 output); db is the first output (the w3
 * branch gradient), da the second (the w1 branch gradient).
 * All arrays bf16 [M, N], unit inner stride, row strides in elements.
 */
int kp_swiglu_bwd_bf16(const void* g, int64_t g_stride, const void* s, int64_t s_stride,
                       const void* b, int64_t b_stride, const void* a, int64_t a_stride,
                       void* db, int64_t db_stride, void* da, int64_t da_stride,
                       int64_t M, int64_t N, void* stream);

/* ------------------------------------------------------------------------
 * SiLU alone: out = bf16(silu(a)), silu(x) = x / (1 + exp(-x)) in fp32.
 *
 * Replaces silu.default at v7/58e7a4d6cde3/problem.py:10-19 (a = w1 output
 * mm_221, bf16 [8192, 14336]).  a, out: bf16 [M, N], unit inner stride, row
 * strides in elements.  Same bits as torch's eager bf16 silu.
 */
int kp_silu_bf16(const void* a, int64_t a_stride, void* out, int64_t out_stride, int64_t M, int64_t N, void* stream);

/* ------------------------------------------------------------------------
 * SwiGLU gate forward recomputed together with its backward, s = bf16(silu(a))
 * kept in registers:
 *   h  = bf16(s * b)
 *   db = bf16(g * s)
 *   da = bf16(t * sig * (1 + a * (1 - sig))),  t = bf16(g * b),  sig = 1 / (1 + exp(-a))
 *
 * Replaces the silu -> mul -> mul -> mul -> silu_backward region at
 * v6/182d2dcd0652/problem.py:10-46 (also v5/441b7bf23822/problem.py:10-48 and
 * v4/c72358b8111e/problem.py:10-48): a = mm_4 (w1 output), b = mm_5 (w3
 * output), g = mm_662 (gradient of the gate product); h, db, da are the
 * fragment's three outputs in order.  3 reads and 3 writes per element where
 * kp_swiglu_fwd_bf16 + kp_swiglu_bwd_bf16 with a stored s take 3 + 6.
 * All arrays bf16 [M, N], unit inner stride, row strides in elements.
 */
int kp_swiglu_fwd_bwd_bf16(const void* a, int64_t a_stride, const void* b, int64_t b_stride,
                           const void* g, int64_t g_stride, void* h, int64_t h_stride,
                           void* db, int64_t db_stride, void* da, int64_t da_stride,
                           int64_t M, int64_t N, void* stream);

/* ------------------------------------------------------------------------
 * Cross-entropy forward over a vocabulary, sum reduction:
 *   lse_i = log(sum_j exp(x_ij)),  x = fp32 of the bf16 logits
 *   *loss = scale * sum over {i : targets[i] != ignore_index} of (lse_i - x_{i, targets[i]})
 *   *total_weight = number of such rows (fp32)
 *
 * Replaces the _to_copy(f32) -> _log_softmax -> nll_loss_forward(weight None,
 * reduction sum, ignore_index) -> div(8192) region at
 * v8/71f1d2c9f38b/problem.py:15-40 (logits mm_224 bf16 [8192, 128256],
 * targets i64 [8192]; scale = 1/8192), without materialising the fp32
 * log-softmax.  logits: bf16 [M, V], unit inner stride, row stride
 * row_stride.  targets: M integers of target_bytes (4 or 8).  loss,
 * total_weight: one fp32 each (device).  row_lse: optional fp32 [M] (lse_i).
 * A target outside [0, V) that is not ignore_index counts as ignored and,
 * when error_flag != NULL, sets *error_flag = 1.  workspace: at least
 * kp_cross_entropy_fwd_workspace_size(M) bytes, 8-byte aligned.  The sum over
 * rows is taken in fp64 in a fixed order (bitwise reproducible).
 */
size_t kp_cross_entropy_fwd_workspace_size(int64_t M);
int kp_cross_entropy_fwd_bf16(const void* logits, int64_t row_stride, int64_t M, int64_t V,
                              const void* targets, int target_bytes, int64_t ignore_index, float scale,
                              float* loss, float* total_weight, float* row_lse, int32_t* error_flag,
                              void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Cross-entropy backward from the saved log-softmax, to bf16:
 *   out_ij = bf16(grad_ij - exp(L_ij) * s_i),  grad_ij = -grad_loss if j == targets[i] else 0,
 *   s_i = sum_j grad_ij (-grad_loss, or 0 for an ignored row)
 * in fp32 (expf), as nll_loss_backward(reduction sum) then
 * _log_softmax_backward_data then _to_copy(bf16) evaluate it.
 *
 * Replaces v8/622c35f5d1c6/problem.py:16-33 (L = _log_softmax fp32
 * [8192, 128256], targets i64 [8192], grad_loss = ones_like(div) / 8192;
 * the total_weight input is unused by the sum reduction).
 * log_softmax: fp32 [M, V], row stride lsm_row_stride; grad_logits: bf16
 * [M, V], row stride out_row_stride.  Targets and error_flag as in the
 * forward (an out-of-range target's row gets s_i = 0).
 */
int kp_cross_entropy_bwd_bf16(const float* log_softmax, int64_t lsm_row_stride, const void* targets,
                              int target_bytes, int64_t ignore_index, float grad_loss, void* grad_logits,
                              int64_t out_row_stride, int64_t M, int64_t V, int32_t* error_flag, void* stream);

/* ------------------------------------------------------------------------
 * Cross-entropy forward and backward straight from the logits, the
 * log-softmax never stored:
 *   out_ij = bf16( grad_ij - exp(x_ij - lse_i) * s_i ),
 *   grad_ij = -grad_loss at (i, t_i) of counted rows, else 0;  s_i = sum_j grad_ij
 * and, when loss / total_weight are given, the forward's
 *   *loss = scale * sum over counted rows of (lse_i - x_{i, t_i}),  *total_weight = #counted rows.
 *
 * Replaces the _to_copy(f32) -> _log_softmax -> nll_loss_forward(sum) -> div
 * -> ones_like -> div -> nll_loss_backward -> _log_softmax_backward_data ->
 * _to_copy(bf16) region at v5/fb5b36393cbd/problem.py:16-59 (also
 * v4/80ad8e737b06/problem.py:16-59): logits mm_224 bf16 [8192, 128256],
 * targets i64 [8192], grad_loss = 1/8192.  fp32 arithmetic; the lse is the
 * forward's (kp_cross_entropy_fwd_bf16).  logits / grad_logits: bf16 [M, V],
 * unit inner stride, row strides in elements; grad_logits may be logits
 * itself (in place).  Rows with an ignored or out-of-range target get zero
 * gradient (out-of-range ones also set *error_flag).  loss and total_weight
 * are both NULL (no forward outputs, no workspace) or both given; then the
 * workspace is kp_cross_entropy_fwd_workspace_size(M) bytes, 8-byte aligned.
 * One launch holds each row in registers when V % 8 == 0, V <= 131072 and
 * rows are 16-byte aligned (4 bytes of HBM traffic per element); other
 * shapes take two passes over the row.
 */
int kp_cross_entropy_fwd_bwd_bf16(const void* logits, int64_t row_stride, int64_t M, int64_t V,
                                  const void* targets, int target_bytes, int64_t ignore_index,
                                  float grad_loss, void* grad_logits, int64_t out_row_stride,
                                  float scale, float* loss, float* total_weight, int32_t* error_flag,
                                  void* workspace, size_t workspace_bytes, void* stream);

/* Self-test of the SwiGLU arithmetic (no counterpart in the reference): for
 * every bf16 bit pattern i (65536 of each, uint32 device arrays) writes the
 * fp32 bits of the fast sigmoid used by the backward kernels and of the IEEE
 * quotient 1 / (1 + expf(-x)) it stands for, and of the fast bf16 silu used by
 * the forward kernels and of bf16(x / (1 + expf(-x))).  tests/ compare them. */
int kp_swiglu_math_selftest(uint32_t* sig_fast, uint32_t* sig_ieee, uint32_t* silu_fast, uint32_t* silu_ref,
                            void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KP_H_ */
