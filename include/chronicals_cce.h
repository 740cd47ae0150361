/*
 * chronicals_cce.h — C ABI of the MI355X (gfx950) fused linear cross-entropy
 * ("Cut Cross-Entropy") library, libchronicals_cce.so.
 *
 * The reference (Ajwebdevs/Chronicals v0.1.4) exposes this path as Python:
 *   chronicals/kernels/cut_cross_entropy.py:1023  cut_cross_entropy(...)
 *   chronicals/kernels/cut_cross_entropy.py:815   CutCrossEntropyFunction (autograd)
 *   chronicals/kernels/cut_cross_entropy.py:567   CutCrossEntropyForward.forward
 *   chronicals/kernels/cut_cross_entropy.py:703   CutCrossEntropyBackward.backward
 * and has no native library of its own; the entry points below are what a
 * ctypes/torch-extension binding of those two static methods needs: plain
 * device pointers, sizes and a HIP stream, no torch types.
 *
 * Conventions
 *   - hidden  [N][d] and weight [V][d] are row-major bf16 (raw 16-bit words),
 *     16-byte aligned, d a multiple of 8.  All arithmetic accumulates in fp32.
 *   - Limits: N <= 2^21 tokens per call, V <= 2^30, d <= 2^20; larger
 *     problems return CCE_ERR_INVALID_ARG.  chunk_size above 2^20 is clamped.
 *   - labels [N] are int64 (labels_int64 = 1) or int32 (labels_int64 = 0).
 *     A row whose label equals ignore_index contributes nothing; a label
 *     outside [0, V) that is not ignore_index has no target logit (loss = lse),
 *     as in the reference (cut_cross_entropy.py:663-668).
 *   - bias is an optional fp32 [V] vector (NULL for none).
 *   - Every call enqueues work on `stream` (a hipStream_t; NULL = default
 *     stream) and returns without synchronising.  Results are deterministic:
 *     no floating-point atomics are used.
 *   - Scratch memory is supplied by the caller (`workspace`), sized by the
 *     *_workspace_bytes queries; the library makes no device allocation at
 *     run time.  Loading it reserves one static device array of
 *     CCE_NOALLOC_SCRATCH_BYTES (64 MiB) on each device it runs on, the
 *     scratch of cce_forward_noalloc, whether or not that entry point is
 *     called.
 *   - Return value 0 = success; otherwise a CCE_ERR_* code, with a message
 *     from cce_last_error() (thread-local).
 */
#ifndef CHRONICALS_CCE_H
#define CHRONICALS_CCE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CCE_ABI_VERSION 7

#define CCE_OK 0
#define CCE_ERR_INVALID_ARG 1
#define CCE_ERR_WORKSPACE 2
#define CCE_ERR_HIP 3

/* reduction: 'none' / 'mean' / 'sum' (triton_kernels.py:2481-2491) */
#define CCE_REDUCTION_NONE 0
#define CCE_REDUCTION_MEAN 1
#define CCE_REDUCTION_SUM 2

/* element types (gradient outputs; logits of the logits-in entry points) */
#define CCE_DTYPE_BF16 0
#define CCE_DTYPE_F32 1
#define CCE_DTYPE_F16 2

/* label-smoothing forms of the logits-in entry points */
#define CCE_SMOOTH_LOGV 0    /* eps*log(V) (cut_cross_entropy.py:1237-1239)                   */
#define CCE_SMOOTH_UNIFORM 1 /* eps*(lse - mean_v x), the uniform-target CE
                                (triton_kernels.py:189-193, :2915, :2952-2956)               */

/* rows of cce_forward's lse_out / target_out: every row, as
   CutCrossEntropyForward.forward returns (cut_cross_entropy.py:671, :692), or
   only the rows with a label (ignored rows read 0), which lets the forward
   skip the ignored rows' share of the logits GEMM.  The loss, n_valid and
   everything cce_backward reads are the same either way. */
#define CCE_LSE_ALL_ROWS 0
#define CCE_LSE_LABELLED_ROWS 1

/* Library ABI version (CCE_ABI_VERSION).  No reference counterpart. */
int cce_abi_version(void);

/* Hex SHA-256 of the sources the library was compiled from (the kernel file
   and this header; "unknown" for a build that did not pass it).  No reference
   counterpart: the Python loader compares it with the source tree and
   refuses a library built from other sources. */
const char* cce_source_hash(void);

/* Message for the last non-zero return on this thread. */
const char* cce_last_error(void);

/*
 * Workspace bytes cce_forward needs for this problem.
 *
 * Two environment variables, read on every query and every call (so a query
 * and the call it sizes must see the same values), change the workspace
 * layout and so its size, never the results:
 *   CHRONICALS_CCE_ROW_GATHER  0: the labelled-rows GEMMs always read a
 *       gathered N x d bf16 copy of hidden; 1: they read hidden's rows in
 *       place wherever byte offsets into hidden fit 32 bits; unset: in place
 *       for hidden of 256 MiB to 2 GiB, the copy otherwise.
 *   CHRONICALS_CCE_G_BUDGET_MB (backward only) the memory budget of the two
 *       band-gradient buffers, in MiB (default 512); a smaller budget means
 *       more, smaller row blocks.
 */
int cce_forward_workspace_bytes(int64_t N, int64_t d, int64_t V, int reduction, int lse_rows, size_t* bytes);

/*
 * Forward.  Replaces CutCrossEntropyForward.forward
 * (chronicals/kernels/cut_cross_entropy.py:567-692) plus the reduction of
 * fused_linear_cross_entropy (chronicals/kernels/triton_kernels.py:2481-2491):
 *   lse[n]   = logsumexp_v (hidden[n] . weight[v] + bias[v])         (:627-671)
 *   row[n]   = valid ? (1-eps)*(lse - t) + eps*S + z*lse^2 : 0       (:674-686)
 *   S        = log(V)                  smoothing_form CCE_SMOOTH_LOGV (:677-679)
 *            = lse - mean_v(logit[n][v]) CCE_SMOOTH_UNIFORM, the loss of
 *              triton_fused_linear_cross_entropy (triton_kernels.py:3147-3263
 *              through _liger_ce_kernel, :2914-2956); the mean is
 *              hidden[n] . sum_v weight[v] / V (+ mean bias)
 *   loss_out = mean: sum(row)/max(n_valid,1); sum: sum(row); none: row[N]
 *   n_valid_out[0] = number of rows with label != ignore_index        (:618, :689)
 *   target_out[n] = hidden[n] . weight[label] + bias[label], 0 for ignored rows
 *                   and labels outside [0, V) (:663-668); may be NULL
 * lse_out [N] fp32 is what cce_backward consumes (the reference saves it at
 * :841).  loss_out holds 1 float (mean/sum) or N floats (none).  Both
 * smoothing forms have the gradient cce_backward computes.  lse_rows
 * (CCE_LSE_ALL_ROWS / CCE_LSE_LABELLED_ROWS) selects whether ignored rows get
 * their lse and target logit or 0; with CCE_LSE_LABELLED_ROWS and d a
 * multiple of 64 the logits GEMM runs only over the 256-row tiles that hold
 * labelled rows.
 */
int cce_forward(const void* hidden, const void* weight, const void* labels, int labels_int64,
                const float* bias, int64_t N, int64_t d, int64_t V, int64_t ignore_index,
                float label_smoothing, float z_loss_weight, int smoothing_form, int reduction, int lse_rows,
                float* loss_out, float* lse_out, float* target_out, int32_t* n_valid_out,
                void* workspace, size_t workspace_bytes, void* stream);

/*
 * cce_forward without a workspace argument: the same computation and results
 * (it runs cce_forward's kernels), with its scratch memory taken from a static
 * device array of CCE_NOALLOC_SCRATCH_BYTES that the library holds on each
 * device it runs on until the process ends.  No counterpart in the reference:
 * it serves callers that cannot allocate device memory (work under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation); the call
 * itself makes no device allocation and no allocating library call.
 * Its scratch need is cce_forward_workspace_bytes' less the N x d bf16 copy
 * of the hidden rows that a labelled-rows forward may take: it reads those
 * rows in place wherever byte offsets into hidden fit 32 bits (hidden below
 * 2 GiB), so its need grows with N only (8.4 MiB at N = 16384, d = 896 and
 * 17.5 MiB at N = 65536, d = 3584, V = 152k).  Problems needing more than
 * CCE_NOALLOC_SCRATCH_BYTES return CCE_ERR_WORKSPACE.  `stream` must belong
 * to the current device.  Every call on one device shares that device's
 * array, so calls whose work overlaps on one device (concurrent streams, or
 * host threads) race; calls ordered on one stream do not.  Nothing in the
 * array needs to start at zero: every scratch value a call reads, the same
 * call writes first.
 */
#define CCE_NOALLOC_SCRATCH_BYTES (64u << 20)
int cce_forward_noalloc(const void* hidden, const void* weight, const void* labels, int labels_int64,
                        const float* bias, int64_t N, int64_t d, int64_t V, int64_t ignore_index,
                        float label_smoothing, float z_loss_weight, int smoothing_form, int reduction, int lse_rows,
                        float* loss_out, float* lse_out, float* target_out, int32_t* n_valid_out, void* stream);

/* Workspace bytes cce_backward needs for this problem, chunk_size and these
   gradients (grad_*_dtype: CCE_DTYPE_BF16 or CCE_DTYPE_F32, as passed to
   cce_backward; fp32 gradients accumulate in place and need less). */
int cce_backward_workspace_bytes(int64_t N, int64_t d, int64_t V, int64_t chunk_size, int need_grad_hidden,
                                 int grad_hidden_dtype, int need_grad_weight, int grad_weight_dtype,
                                 size_t* bytes);

/*
 * Backward.  Replaces CutCrossEntropyBackward.backward
 * (chronicals/kernels/cut_cross_entropy.py:703-808) with the one-hot term
 * applied (as the reference's GPU path, :530-546, and
 * triton_kernels.py:2594-2601 do; its CPU path loses it at :773-780):
 *   G[n][v] = (P - (1-eps)*onehot - eps/V + 2z*lse*P) * valid * g_n
 *   g_n     = grad_out[0]/max(n_valid,1) (mean), grad_out[0] (sum), grad_out[n] (none)
 *   grad_hidden = G . weight  [N][d]    (:795)
 *   grad_weight = G^T . hidden [V][d]   (:798)
 *   grad_bias   = sum_n G      [V]      (:801-802)
 * Any of grad_hidden / grad_weight / grad_bias may be NULL to skip it (a
 * frozen lm_head skips grad_weight, as triton_kernels.py:3213 does).
 * grad_*_dtype selects CCE_DTYPE_BF16 or CCE_DTYPE_F32 output; grad_bias is
 * fp32.  The vocabulary is processed in bands of up to 8192 columns: the
 * reference's chunk_size argument (:1028), rounded up to a multiple of 256,
 * bounds the band from above (the partial band, if any, comes first); from
 * 1024 to 4095 rows the bands are up to 4x wider, while G and W^T of a band
 * take no more than at 4096 rows.  The rows are processed in blocks whose
 * band gradient (two bf16 buffers of rows x band) stays within 512 MiB, so
 * that memory does not grow with N; dW of a band accumulates over the
 * blocks.  fp32 gradients accumulate in place; bf16 ones in fp32 workspace.
 * Deterministic: every reduction runs in a fixed order, including the fp32
 * partials of dH when few rows make the library split each band's columns
 * over several workgroups.
 * grad_hidden and grad_weight double as scratch while the call's kernels run
 * (H^T, and each band's W^T, live in output memory that is not yet written),
 * so neither may overlap an input, and their contents are final only once
 * the stream has run past the call.
 */
int cce_backward(const float* grad_out, const void* hidden, const void* weight, const void* labels,
                 int labels_int64, const float* bias, const float* lse, const int32_t* n_valid,
                 int64_t N, int64_t d, int64_t V, int64_t ignore_index, float label_smoothing,
                 float z_loss_weight, int reduction, int64_t chunk_size, void* grad_hidden,
                 int grad_hidden_dtype, void* grad_weight, int grad_weight_dtype, float* grad_bias,
                 void* workspace, size_t workspace_bytes, void* stream);

/*
 * Cross-entropy over logits that already exist (no lm_head fusion): the
 * callers that hold logits.  Replaces the row computation of
 *   chunked_cross_entropy_loss  cut_cross_entropy.py:1169-1249  (CCE_SMOOTH_LOGV)
 *   _liger_ce_kernel            triton_kernels.py:2839-2963     (CCE_SMOOTH_UNIFORM)
 *   fused_cross_entropy_kernel  triton_kernels.py:141-210       (CCE_SMOOTH_UNIFORM)
 * For logits [N][ld] (row stride ld >= V elements, last dimension
 * contiguous; bf16, fp16 or fp32 per logits_dtype):
 *   lse[n] = log(sum_v exp(x[n][v]) + 1e-10)                   (:1206-1223)
 *   row[n] = valid ? (1-eps)*(lse - x[n][label]) + eps*S + z*lse^2 : 0
 *            S = log(V) (CCE_SMOOTH_LOGV, :1226-1246) or
 *            S = lse - sum_v x[n][v]/V (CCE_SMOOTH_UNIFORM, triton_kernels.py:2952-2956)
 *   loss   = mean: sum(row)/max(n_valid,1); sum: sum(row); none: row[N]
 * A label outside [0, V) that is not ignore_index has no target logit (the
 * chunked reference's gather would raise; the Triton kernels give the same
 * zero target).  Deterministic; workspace from
 * cce_logits_forward_workspace_bytes.
 */
int cce_logits_forward_workspace_bytes(int64_t N, int64_t V, int reduction, size_t* bytes);
int cce_logits_forward(const void* logits, int logits_dtype, int64_t ld, const void* labels, int labels_int64,
                       int64_t N, int64_t V, int64_t ignore_index, float label_smoothing, float z_loss_weight,
                       int smoothing_form, int reduction, float* loss_out, float* lse_out, int32_t* n_valid_out,
                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * Gradient of cce_logits_forward's loss with respect to the logits, for
 * valid rows (zero rows for ignored labels), p = softmax(x[n]):
 *   CCE_SMOOTH_LOGV:    g_n*(((1-eps) + 2z*lse[n])*p[v] - (1-eps)*[v == label])
 *                       (autograd through cut_cross_entropy.py:1169-1249;
 *                       eps*log V is a constant)
 *   CCE_SMOOTH_UNIFORM: g_n*((1 + 2z*lse[n])*p[v] - eps/V - (1-eps)*[v == label])
 *                       (triton_kernels.py:2930-2947, :197-206)
 * g_n as in cce_backward.  grad_logits has row stride ld_grad and element type
 * grad_dtype: the logits' type or CCE_DTYPE_F32.  grad_logits may be the
 * logits buffer itself (same type and stride): the gradient then overwrites
 * the logits, as _liger_ce_kernel does.
 */
int cce_logits_backward(const float* grad_out, const void* logits, int logits_dtype, int64_t ld, const void* labels,
                        int labels_int64, const float* lse, const int32_t* n_valid, int64_t N, int64_t V,
                        int64_t ignore_index, float label_smoothing, float z_loss_weight, int smoothing_form,
                        int reduction, void* grad_logits, int grad_dtype, int64_t ld_grad, void* stream);

/*
 * Loss and gradient in one kernel, for the callers whose reference computes
 * both in its forward: fused_cross_entropy_kernel (triton_kernels.py:141-210)
 * and _liger_ce_kernel with COMPUTE_GRADS (:2839-2958).  Computes what
 * cce_logits_forward does and, in the same pass over each row, writes the
 * gradient of cce_logits_backward with grad_out = 1 and g_n =
 * 1/max(n_valid,1) if grad_mean, else 1 (the reference kernels' 'mean' and
 * unscaled forms, :2946-2947, :197-206).  Each row is read twice (the second
 * time mostly from the memory-side cache) and its gradient written once.
 * grad_logits may be the logits buffer itself (same dtype and stride).
 * Workspace from cce_logits_forward_workspace_bytes.
 */
int cce_logits_forward_backward(const void* logits, int logits_dtype, int64_t ld, const void* labels,
                                int labels_int64, int64_t N, int64_t V, int64_t ignore_index, float label_smoothing,
                                float z_loss_weight, int smoothing_form, int reduction, int grad_mean,
                                float* loss_out, float* lse_out, int32_t* n_valid_out, void* grad_logits,
                                int grad_dtype, int64_t ld_grad, void* workspace, size_t workspace_bytes,
                                void* stream);

/*
 * Per-kernel timing for measurement tools (no counterpart in the reference).
 * While enabled, every GEMM launch of cce_forward / cce_backward and every
 * row-kernel launch of cce_logits_forward / _backward / _forward_backward is bracketed
 * by HIP events recorded on its stream.  cce_kernel_timing_read() waits for
 * the recorded events and returns, for one kernel kind, the summed
 * milliseconds, the launch count and the work of those launches — credited
 * (the algorithmic work: forward logits, dHidden, dWeight; the backward's
 * logits recompute is executed but not credited) and executed — then clears
 * that kind's record.  The work is MFMA FLOPs for the GEMM kinds and
 * algorithmic HBM bytes for the logits kinds.  credited_flops /
 * executed_flops may be NULL.  Kinds:
 */
#define CCE_KERNEL_FWD_LSE 0   /* forward GEMM + online logsumexp                 */
#define CCE_KERNEL_BWD_GRAD 1  /* backward recompute GEMM -> dLoss/dS             */
#define CCE_KERNEL_BWD_DH 2    /* dHidden GEMM (per vocabulary band)               */
#define CCE_KERNEL_BWD_DW 3    /* dWeight GEMM (per vocabulary band)               */
#define CCE_KERNEL_BWD_DHDW 4  /* dHidden + dWeight GEMMs in one launch            */
#define CCE_KERNEL_BWD_BAND 5  /* dHidden + dWeight of band b with the recompute
                                  of band b+1 in one launch                        */
#define CCE_KERNEL_LOGITS_FWD 6 /* logits-in forward row kernel (reads N*V)     */
#define CCE_KERNEL_LOGITS_BWD 7 /* logits-in backward row kernel (N*V in + out) */
#define CCE_KERNEL_LOGITS_FUSED 8 /* logits-in loss + gradient kernel (N*V in + out) */
#define CCE_KERNEL_KINDS 9
int cce_kernel_timing_enable(int enable);
int cce_kernel_timing_read(int kind, double* total_ms, int64_t* launches, double* credited_flops,
                           double* executed_flops);

#ifdef __cplusplus
}
#endif

#endif /* CHRONICALS_CCE_H */
