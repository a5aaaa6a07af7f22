/*
 * kda_mi355x.h -- C ABI of the MI355X (gfx950) KDA hot path.
 *
 * Drop-in boundary for the chunked Kimi-Delta-Attention forward (WY/UT form),
 * the single-token recurrent decode step and varlen (cu_seqlens) scheduling.
 *
 * Conventions (all entry points):
 *   - every tensor pointer is device memory; work is enqueued on `stream` and
 *     is stream-ordered; nothing is allocated by the library (the chunked
 *     forward takes a caller-provided workspace);
 *   - tensors are row-major, token-major: q, k, g are [B, T, H, dk], v and o
 *     are [B, T, H, dv], beta is [B, T, H]; states are [N, H, dk, dv] fp32;
 *   - g is the per-channel log-decay (g = log alpha <= 0), beta in (0, 1);
 *     no 1/sqrt(d) scale is applied unless `scale` says so (1.0 reproduces
 *     the reference, which applies none: net/kda.py:293, :693-696);
 *   - the kernels move several elements per lane access, so pointers are
 *     aligned to that access: 16 bytes for the chunked forward's (kda_chunk_fwd,
 *     its no-allocation form, cc_scan, the layer forward) q, k, v, g, o,
 *     workspace and cc_scan's beta32, the chunked backward's and cc_scan
 *     backward's inputs, gradients, states and workspace, and the decode
 *     steps' state; 4 elements for the decode step's v and o and the epilogues'
 *     tensors; 2 elements for the prologues' projections and outputs.
 *     Other pointers need only element alignment.  Torch and XLA
 *     allocations satisfy this; a misaligned pointer is rejected with
 *     KDA_ERR_INVALID_ARGUMENT before anything is enqueued;
 *   - return value 0 on success, a negative kda_status_t otherwise; the
 *     message of the last failure on the calling thread is kda_last_error().
 *     Invalid arguments are rejected before anything is enqueued; there is
 *     no fallback path of any kind.
 *
 * Reference = romannekrasovaillm/axiom.  Each entry point names the reference
 * interface it replaces.
 */
#ifndef KDA_MI355X_H_
#define KDA_MI355X_H_

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#if defined(__GNUC__)
#define KDA_API __attribute__((visibility("default")))
#else
#define KDA_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

typedef enum kda_status_t {
  KDA_OK = 0,
  KDA_ERR_INVALID_ARGUMENT = -1, /* bad pointer, shape or value            */
  KDA_ERR_UNSUPPORTED = -2,      /* valid request this build does not run  */
  KDA_ERR_WORKSPACE = -3,        /* workspace missing or too small         */
  KDA_ERR_HIP = -4               /* HIP runtime / launch failure           */
} kda_status_t;

typedef enum kda_dtype_t {
  KDA_DTYPE_F32 = 0,             /* all inputs fp32: exact (fp32 MFMA) mode */
  KDA_DTYPE_BF16 = 1,            /* q, k, v, g, beta bf16                   */
  KDA_DTYPE_F16 = 2,             /* q, k, v, g, beta fp16                   */
  KDA_DTYPE_BF16_F32GATES = 3    /* q, k, v bf16; g, beta fp32              */
} kda_dtype_t;

/*
 * Chunked KDA forward.
 *
 * Replaces the reference's whole-sequence KDA scan seam
 *   net/kernels/kda_cc_fused_persist.py:920  cc_scan(q, k, v, alpha, beta32, S, tile, chunk)
 * and the jax scan it stands in for, net/kda.py:856-926 (apply_chunked_cc,
 * body cc_chunk_step net/kda.py:634-705), called from net/kda.py:844 with the
 * batch axis vmapped at net/model.py:341.  Generalised to the FLA-style
 * signature (q, k, v, g, beta, h0, cu_seqlens) -> (o, ht):
 *   - g replaces alpha (g = log alpha), beta is [B,T,H] (not replicated),
 *   - the batch is explicit instead of vmapped,
 *   - h0 (nullable, zeros if null; the reference passes zeros at
 *     net/kda.py:850) and ht (nullable) are [N, H, dk, dv] fp32 with N = B,
 *     or N = n_seqs when cu_seqlens is given,
 *   - cu_seqlens (nullable, int32 [n_seqs+1], requires B == 1) packs n_seqs
 *     independent sequences into one stream (absent in the reference; defined
 *     by "packed run == independent per-sequence runs"),
 *   - T need not be a multiple of `chunk`: a ragged tail is handled in place
 *     and ht is the state after the last real token.
 * o is written in out_dtype (KDA_DTYPE_F32 or KDA_DTYPE_BF16); the reference
 * seam emits fp32 (net/kernels/kda_cc_fused_persist.py:660).
 * Supported: dk == dv in {64, 128}, chunk == 64, in_dtype any kda_dtype_t.
 * cu_seqlens values are clamped on the device into a non-decreasing sequence
 * inside [0, T] so no access can leave the tensors; kda_varlen_status reports
 * whether a repair was needed.
 * Operand range of 16-bit inputs (BF16, F16, BF16_F32GATES): the matrix-core
 * operands are fp16 (range +-65504).  Supported: q and k rows of unit L2
 * norm as the reference's layer produces them (net/kda.py:200-201), |q scale|
 * and |k| below 2^15 per element, and |v|, U = (I + L)^-1 (beta v), the
 * state (h0 and its evolution) and v~ = U - W S below 2^15 in magnitude.
 * Outside this range a result is not finite; the state kernels detect it and
 * kda_chunk_fwd_status reports KDA_STATUS_NONFINITE.  fp32 inputs (exact
 * mode) have fp32 range.
 */
KDA_API int kda_chunk_fwd(hipStream_t stream,
                  const void* q, const void* k, const void* v,
                  const void* g, const void* beta,
                  const float* h0,
                  const int32_t* cu_seqlens, int32_t n_seqs,
                  void* o, float* ht,
                  int B, int T, int H, int dk, int dv, int chunk, float scale,
                  int in_dtype, int out_dtype,
                  void* workspace, size_t workspace_bytes);

/*
 * kda_chunk_fwd without a workspace argument: the workspace is a file-scope
 * device array of the library (256 MiB = 268435456 bytes, one per device,
 * held from the library's load until the process ends), so the call allocates nothing (no hipMalloc, no allocating library
 * routine) and only launches kernels.  No counterpart in the reference: it is
 * for callers that cannot allocate -- code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation.  Arguments, results and
 * errors as kda_chunk_fwd run with the scratch as its workspace (a varlen
 * call whose fastest schedule needs more runs in the segments that fit);
 * a call whose least workspace (kda_chunk_fwd_workspace_min) exceeds the
 * scratch returns KDA_ERR_WORKSPACE.  All calls on one device
 * share its scratch: calls that overlap on one device (two streams or
 * threads) race and must be ordered by the caller.
 */
KDA_API int kda_chunk_fwd_noalloc(hipStream_t stream,
                  const void* q, const void* k, const void* v,
                  const void* g, const void* beta,
                  const float* h0,
                  const int32_t* cu_seqlens, int32_t n_seqs,
                  void* o, float* ht,
                  int B, int T, int H, int dk, int dv, int chunk, float scale,
                  int in_dtype, int out_dtype);

/* Workspace bytes of kda_chunk_fwd's fastest schedule for these arguments
 * (0 on bad input).  n_seqs <= 0 means dense (no cu_seqlens).  Host-only; no
 * HIP call. */
KDA_API size_t kda_chunk_fwd_workspace(int B, int T, int H, int dk, int dv, int chunk,
                               int32_t n_seqs, int in_dtype);

/* The least workspace kda_chunk_fwd accepts for these arguments (0 on bad
 * input).  Equal to kda_chunk_fwd_workspace except for varlen calls (at most
 * 2048 sequences) whose intra-chunk results exceed 160 MiB: given less than
 * kda_chunk_fwd_workspace (and at least this), such a call runs in segments
 * of a position-major unit numbering, the largest that fit its workspace,
 * with the same results bit for bit and more time (config 3: 3.9 ms with
 * the 5.8 GB workspace, 4.7 ms with the ~0.23 GB minimum).  No counterpart in
 * the reference (varlen is absent there).  Host-only; no HIP call. */
KDA_API size_t kda_chunk_fwd_workspace_min(int B, int T, int H, int dk, int dv, int chunk,
                                   int32_t n_seqs, int in_dtype);

/*
 * Status of the last kda_chunk_fwd (or kda_chunk_fwd_noalloc: pass
 * workspace = NULL) on `stream` with these arguments, copied to *flags_out
 * (synchronising the stream).  Bits: 1, 2, 4, 8 as kda_varlen_status (varlen
 * calls); 65536 (KDA_STATUS_NONFINITE) an o or final state value of a 16-bit
 * input call is not finite: an fp16 operand left its range (see the
 * precondition of kda_chunk_fwd) or the inputs were not finite.  No
 * counterpart in the reference, whose bf16 operands have fp32 range.
 */
#define KDA_STATUS_NONFINITE 65536
KDA_API int kda_chunk_fwd_status(hipStream_t stream, const void* workspace, size_t workspace_bytes,
                         int B, int T, int H, int dk, int dv, int chunk, int32_t n_seqs,
                         int in_dtype, int32_t* flags_out);

/*
 * After a varlen kda_chunk_fwd on `stream`, copy the device-side validation
 * word of its workspace to *flags_out (synchronising the stream).  Bits:
 * 1 cu[0] != 0, 2 cu[n] != T, 4 decreasing entry, 8 entry outside [0, T].
 */
KDA_API int kda_varlen_status(hipStream_t stream, const void* workspace, size_t workspace_bytes,
                      int B, int T, int H, int dk, int dv, int chunk, int32_t n_seqs,
                      int in_dtype, int32_t* flags_out);

/*
 * One recurrent decode step for B*H chains, state updated in place.
 *
 * Replaces net/kda.py:298-310 (_delta_step) followed by the read-out
 * net/kda.py:293 (o = S^T q) inside recurrent_step (net/kda.py:277-295):
 *   S <- (I - beta k k^T) diag(alpha) S + beta k v^T,  o = S^T (scale q).
 * q, k, g: [B, H, dk]; v: [B, H, dv]; beta: [B, H]; state: [B, H, dk, dv] fp32
 * (in place); o: [B, H, dv] in out_dtype.  in_dtype: F32, BF16 or F16.
 */
KDA_API int kda_recurrent_step(hipStream_t stream,
                       const void* q, const void* k, const void* v,
                       const void* g, const void* beta,
                       float* state, void* o,
                       int B, int H, int dk, int dv, float scale,
                       int in_dtype, int out_dtype);

/*
 * The reference seam verbatim:
 *   net/kernels/kda_cc_fused_persist.py:920  cc_scan(q, k, v, alpha, beta32, S, tile=16, chunk=32)
 * q, k: (T, H*dk) bf16; v: (T, H*dv) bf16; alpha: (T, H*dk) fp32 in (0, 1];
 * beta32: (T, H*32) fp32 (beta replicated over 32 columns, recovered as the
 * mean, :435); S_in: (H, dk, dv) fp32.  Outputs o: (T, H*dv) fp32 and S_out:
 * (H, dk, dv) fp32 (functional: S_in is not modified unless S_out == S_in).
 * Errors as the reference (net/kernels/kda_cc_fused_persist.py:737-749):
 * T % chunk != 0 -> KDA_ERR_INVALID_ARGUMENT; tile outside [1, 16] ->
 * KDA_ERR_INVALID_ARGUMENT.  The result does not depend on chunk or tile in
 * exact arithmetic; the kernels always run with C = 64 and 16-row tiles.
 */
KDA_API int kda_cc_scan(hipStream_t stream,
                const void* q, const void* k, const void* v,
                const float* alpha, const float* beta32, const float* S_in,
                float* o, float* S_out,
                int T, int H, int dk, int dv, int tile, int chunk,
                void* workspace, size_t workspace_bytes);

/* Workspace bytes kda_cc_scan needs (0 on bad input).  Host-only. */
KDA_API size_t kda_cc_scan_workspace(int T, int H, int dk, int dv, int chunk);

/*
 * The seam's backward rule: kernel_bwd, net/kernels/kda_cc_fused_persist.py
 * :1710-1763 (the custom_vjp backward of cc_scan, :895-911; the adjoint of
 * net/kernels/kda_cc_fused_bwd.py:117-239 scanned in reverse, :794-842).
 * Inputs as kda_cc_scan plus the cotangents d_o (T, H*dv) fp32 of o and dS
 * (H, dk, dv) fp32 of S_out.  Outputs in the primal dtypes: dq, dk (T, H*dk)
 * and dv (T, H*dv) bf16; dalpha (T, H*dk) fp32 (= d(log alpha) / alpha);
 * dbeta32 (T, H*32) fp32 (the beta cotangent / 32 on each column); dS_in
 * (H, dk, dv) fp32.  Errors as kda_cc_scan.  Caller workspace of
 * kda_cc_scan_bwd_workspace bytes.
 */
KDA_API int kda_cc_scan_bwd(hipStream_t stream,
                const void* q, const void* k, const void* v,
                const float* alpha, const float* beta32, const float* S_in,
                const float* d_o, const float* dS,
                void* dq, void* dk, void* dv, float* dalpha, float* dbeta32, float* dS_in,
                int T, int H, int dk_dim, int dv_dim, int tile, int chunk,
                void* workspace, size_t workspace_bytes);

/* Workspace bytes kda_cc_scan_bwd needs (0 on bad input).  Host-only. */
KDA_API size_t kda_cc_scan_bwd_workspace(int T, int H, int dk, int dv, int chunk);

/*
 * The seam for its vmapped caller: net/model.py:341-347 maps cc_scan over the
 * batch (jax.vmap), so the custom call sees a leading batch axis.  These take
 * the seam's operands with that axis -- q, k, alpha (B, T, H*dk), v (B, T,
 * H*dv), beta32 (B, T, H*32), S_in (B, H, dk, dv) -- and run the B elements
 * in one launch each (the batch folded into the kernels' grids), with the
 * results, errors and cotangents of B separate kda_cc_scan /
 * kda_cc_scan_bwd calls.  An XLA FFI handler registered with
 * vmap_method="expand_dims" binds them directly (B = 1 is kda_cc_scan).
 */
KDA_API int kda_cc_scan_batched(hipStream_t stream,
                const void* q, const void* k, const void* v,
                const float* alpha, const float* beta32, const float* S_in,
                float* o, float* S_out,
                int B, int T, int H, int dk, int dv, int tile, int chunk,
                void* workspace, size_t workspace_bytes);
KDA_API size_t kda_cc_scan_batched_workspace(int B, int T, int H, int dk, int dv, int chunk);
KDA_API int kda_cc_scan_bwd_batched(hipStream_t stream,
                const void* q, const void* k, const void* v,
                const float* alpha, const float* beta32, const float* S_in,
                const float* d_o, const float* dS,
                void* dq, void* dk, void* dv, float* dalpha, float* dbeta32, float* dS_in,
                int B, int T, int H, int dk_dim, int dv_dim, int tile, int chunk,
                void* workspace, size_t workspace_bytes);
KDA_API size_t kda_cc_scan_bwd_batched_workspace(int B, int T, int H, int dk, int dv, int chunk);

/*
 * Chunked backward: gradients of (o, final state) = kda_chunk_fwd(q, k, v, g,
 * beta, h0) for dense [B,T,H,d] inputs (no cu_seqlens).  Replaces the
 * reference's backward rule of the cc_scan custom_vjp,
 *   net/kernels/kda_cc_fused_persist.py:1707  kernel_bwd(q, k, v, alpha, beta32, S, do, dS)
 *   (the reverse scan of the per-chunk adjoint, :794-842 and
 *   net/kernels/kda_cc_fused_bwd.py:117-228),
 * in the FLA-style layout of kda_chunk_fwd.  dout [B,T,H,dv] is the cotangent
 * of o (dout_dtype KDA_DTYPE_F32 or KDA_DTYPE_BF16), dht [B,H,dk,dv] fp32 the
 * cotangent of the final state (null = 0), h0 as in the forward (null = 0).
 * Outputs, all fp32: dq, dk, dg [B,T,H,dk], dv [B,T,H,dv], dbeta [B,T,H] and,
 * when dh0 is not null, dh0 [B,H,dk,dv].  dg is the cotangent of the log
 * decay g (the reference's alpha form has dalpha = dg / alpha).  q, k, v, g,
 * beta, in_dtype, scale and chunk as in kda_chunk_fwd; the workspace is
 * caller-owned, kda_chunk_bwd_workspace bytes.  Precision: fp32 inputs keep
 * an fp32 workspace (gradients within 1e-4 relative of an fp64 reference);
 * 16-bit inputs store the forward-side intermediates (gamma q, lambda k, Aqk,
 * T, W and each chunk's incoming state) in fp16, the width the forward gives
 * them, with the cotangents, U and v~ kept fp32 (within 1e-3 relative of an
 * fp64 reference, 1e-4 of an emulation of those roundings).
 */
KDA_API int kda_chunk_bwd(hipStream_t stream,
                const void* q, const void* k, const void* v, const void* g, const void* beta,
                const float* h0, const void* dout, const float* dht,
                float* dq, float* dk, float* dv, float* dg, float* dbeta, float* dh0,
                int B, int T, int H, int dk_dim, int dv_dim, int chunk, float scale,
                int in_dtype, int dout_dtype, void* workspace, size_t workspace_bytes);

/* Workspace bytes kda_chunk_bwd needs (0 on bad input).  Host-only. */
KDA_API size_t kda_chunk_bwd_workspace(int B, int T, int H, int dk_dim, int dv_dim, int chunk);

/*
 * Standalone batched unit-triangular solve, per head h:
 *   transpose == 0:  X = (I + L)^-1 B      net/kernels/kda_ut_solve.py:525  kernel(a, b)
 *   transpose != 0:  X = (I + L)^-T B      net/kernels/kda_ut_solve.py:536  kernel_t(a, b)
 * with L = the strictly lower part of a [H][C][C] (a's diagonal and upper
 * part are not read: a is unit lower triangular in the reference's
 * contract), b and x [H][C][N], all row-major, of one dtype KDA_DTYPE_F32 or
 * KDA_DTYPE_BF16 (fp32 arithmetic).  1 <= C <= 64, N >= 1.
 */
KDA_API int kda_ut_solve(hipStream_t stream, const void* a, const void* b, void* x,
                int H, int C, int N, int dtype, int transpose);

/*
 * Backward rule of the differentiable solve (the custom_vjp of
 * net/kernels/kda_ut_solve.py:601-636, adjoint :563-588): given a, the
 * forward solution x and its cotangent dx, writes db = the sibling solve of
 * dx (transposed for the forward solve, plain for the transposed one) and
 * da = strict_lower(-db x^T) (forward solve) or strict_lower(-x db^T)
 * (transposed solve); da's diagonal and upper part are written as zero.
 * Shapes, dtype and `transpose` (of the forward solve) as kda_ut_solve.
 */
KDA_API int kda_ut_solve_bwd(hipStream_t stream, const void* a, const void* x, const void* dx,
                void* da, void* db, int H, int C, int N, int dtype, int transpose);

/*
 * Prologue of the KDA layer around kda_chunk_fwd: per channel the causal
 * depthwise short convolution of the projections (net/shortconv.py:14-33,
 * continued across calls by buffers as net/kda.py:383-389), swish
 * (net/norm.py:15-17), and for q and k the per-head L2 normalisation
 * x / (||x|| + 1e-12) (net/norm.py:53-66) -- net/kda.py:194-202.  qp, kp, vp
 * [B,T,H*d] in in_dtype (KDA_DTYPE_F32 or KDA_DTYPE_BF16); conv taps wq, wk, wv
 * [K, H*d] fp32 (w[i] weights the input i steps back, 1 <= K <= 8); buffers
 * b*_in [B, K-1, H*d] fp32 (the previous K-1 inputs, oldest first; null =
 * zeros) and b*_out (the last K-1 inputs after this call; null = not kept; may
 * equal b*_in); outputs q, k, v [B,T,H,d] in out_dtype (KDA_DTYPE_F32 or
 * KDA_DTYPE_BF16).  d = dk = dv in {64, 128}.
 */
KDA_API int kda_prologue(hipStream_t stream,
                const void* qp, const void* kp, const void* vp,
                const float* wq, const float* wk, const float* wv,
                const float* bq_in, const float* bk_in, const float* bv_in,
                float* bq_out, float* bk_out, float* bv_out,
                void* q, void* k, void* v,
                int B, int T, int H, int d, int K, int in_dtype, int out_dtype);

/*
 * Epilogue of the KDA layer before the output projection (net/kda.py:205-214
 * without W_o): y = sigmoid(gate) * o / sqrt(mean over the head's dv
 * channels of o^2 + eps) (net/norm.py:69-73, eps = 1e-6 there).  o
 * [B,T,H,dv] and gate logits [B,T,H*dv] in their dtypes (F32 or BF16), y
 * [B,T,H*dv] in out_dtype.  dv in {64, 128}.
 */
KDA_API int kda_epilogue(hipStream_t stream, const void* o, const void* gate, void* y,
                int B, int T, int H, int dv, float eps, int o_dtype, int gate_dtype, int out_dtype);

/*
 * Backward of kda_prologue: the adjoint of net/kda.py:194-202 after the convs
 * of :383-389 (autodiff through net/shortconv.py:14-33 and net/norm.py:15-17,
 * 53-66 in the reference), written out: L2-norm adjoint (zero on a row whose
 * norm is zero, the tangent convention net/tests/test_22_l2norm_padding_
 * gradient.py pins), swish adjoint, conv transpose.  Inputs as kda_prologue
 * (qp, kp, vp [B,T,H*d] in in_dtype, F32 or BF16; taps [K,H*d] fp32; incoming
 * buffers [B,K-1,H*d] fp32 or NULL for zeros) plus dq, dk, dv [B,T,H,d] fp32.
 * Outputs fp32: dqp, dkp, dvp [B,T,H*d]; dwq, dwk, dwv [K,H*d] (sums over the
 * batch, overwritten); dbq, dbk, dbv [B,K-1,H*d], the incoming buffers'
 * gradients (NULL to skip; unused when K == 1).  The forward is recomputed.
 * Caller workspace of kda_prologue_bwd_workspace bytes.  d in {64, 128},
 * 1 <= K <= 8.
 */
KDA_API int kda_prologue_bwd(hipStream_t stream, const void* qp, const void* kp, const void* vp,
                const float* wq, const float* wk, const float* wv,
                const float* bq_in, const float* bk_in, const float* bv_in,
                const float* dq, const float* dk, const float* dv,
                float* dqp, float* dkp, float* dvp, float* dwq, float* dwk, float* dwv,
                float* dbq, float* dbk, float* dbv,
                int B, int T, int H, int d, int K, int in_dtype, void* workspace, size_t workspace_bytes);

/* Workspace bytes kda_prologue_bwd needs (0 on bad input).  Host-only. */
KDA_API size_t kda_prologue_bwd_workspace(int B, int T, int H, int d, int K);

/*
 * Backward of kda_epilogue (net/kda.py:205-214 without W_o, and
 * net/norm.py:69-73, differentiated by autodiff in the reference): given
 * o [B,T,H,dv], gate logits [B,T,H*dv] and dy [B,T,H*dv], writes
 * dout [B,T,H,dv] fp32 and dgate [B,T,H*dv] in dgate_dtype.  All input
 * dtypes F32 or BF16.  One launch.  dv in {64, 128}.
 */
KDA_API int kda_epilogue_bwd(hipStream_t stream, const void* o, const void* gate, const void* dy,
                float* dout, void* dgate, int B, int T, int H, int dv, float eps,
                int o_dtype, int gate_dtype, int dy_dtype, int dgate_dtype);

/*
 * One decode token of the whole KDA layer between its projections and W_o,
 * with the short-conv buffers and the state carried in place: the streaming
 * recurrent_step of net/kda.py:277-295 (conv steps net/shortconv.py:36-62,
 * postprocess :194-202, delta rule :298-310, o = S^T q :293, output gate
 * :205-214 without W_o).  qp, kp, vp [B, H*d], g [B,H,d] (log decay), beta
 * [B,H], gate logits [B, H*d] in in_dtype (KDA_DTYPE_F32 or KDA_DTYPE_BF16);
 * conv taps [K, H*d] fp32; buffers [B, K-1, H*d] fp32 and state [B,H,d,d]
 * fp32 updated in place; y [B, H*d] in out_dtype (F32 or BF16).  One fused
 * launch (a workgroup per (b, h): conv, swish, L2 norm, the state step, the
 * gated RMSNorm); the caller workspace of kda_decode_layer_workspace bytes is
 * still required and validated (the ABI is unchanged) but not written.
 * d in {64, 128}, 1 <= K <= 8.
 */
KDA_API int kda_decode_layer_step(hipStream_t stream,
                const void* qp, const void* kp, const void* vp,
                const void* g, const void* beta, const void* gate,
                const float* wq, const float* wk, const float* wv,
                float* bq, float* bk, float* bv, float* state, void* y,
                int B, int H, int d, int K, float scale, float eps, int in_dtype, int out_dtype,
                void* workspace, size_t workspace_bytes);

/* Workspace bytes kda_decode_layer_step needs (0 on bad input).  Host-only. */
KDA_API size_t kda_decode_layer_workspace(int B, int H, int d, int in_dtype);

/*
 * The chunked (prefill / training-forward) KDA layer between its projections
 * and W_o: replaces the body of net/kda.py:790-853 (_apply_chunked_cc_persistent:
 * short_conv -> _postprocess -> cc_scan -> _output_gate, :839-853), with the
 * conv history carried across calls as chunk_step does (net/kda.py:356-358,
 * :383-389) and an optional initial state.  qp, kp, vp [B,T,H*d]; g [B,T,H,d]
 * log decay; beta [B,T,H] -- in in_dtype (KDA_DTYPE_BF16, KDA_DTYPE_BF16_F32GATES
 * or KDA_DTYPE_F32, as for kda_chunk_fwd); gate logits [B,T,H*d] in gate_dtype;
 * conv taps, buffers as kda_prologue (1 <= K <= 8); h0 / ht as kda_chunk_fwd;
 * y [B,T,H*d] = sigmoid(gate) * RMSNorm_head(o) in out_dtype (F32 or BF16).
 * With bf16 projections and K <= 4 the prologue runs inside the intra kernel
 * (no q, k, v round trip through memory; results equal kda_prologue followed
 * by kda_chunk_fwd and kda_epilogue bit for bit); otherwise it is its own pass.
 * o_out: NULL, or [B,T,H,d] fp32 that receives the scan's output o (the
 * epilogue's input; a training caller keeps it for kda_epilogue_bwd instead
 * of recomputing it).  Caller workspace of kda_layer_fwd_workspace bytes.
 * d in {64, 128}.
 */
KDA_API int kda_layer_fwd(hipStream_t stream,
                const void* qp, const void* kp, const void* vp,
                const void* g, const void* beta, const void* gate,
                const float* wq, const float* wk, const float* wv,
                const float* bq_in, const float* bk_in, const float* bv_in,
                float* bq_out, float* bk_out, float* bv_out,
                const float* h0, float* ht, void* y, float* o_out,
                int B, int T, int H, int d, int K, float scale, float eps,
                int in_dtype, int gate_dtype, int out_dtype, void* workspace, size_t workspace_bytes);

/* Workspace bytes kda_layer_fwd needs (0 on bad input).  Host-only. */
KDA_API size_t kda_layer_fwd_workspace(int B, int T, int H, int d, int K, int in_dtype);

/* Message of the last failure on the calling thread ("" if none). */
KDA_API const char* kda_last_error(void);

/* ABI version of this library (major * 100 + minor). */
KDA_API int kda_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* KDA_MI355X_H_ */
