/*
 * fwloss.h -- C ABI of the MI355X (gfx950) Familywise (FW) loss library, libfwloss.so.
 *
 * For each row z (C fp32 logits) with label y the library computes the FW threshold
 *     tau = max_k (S_k - 1)/k,   S_k = sum of the k largest entries of z,
 * the support {j : z_j > tau} (strict), kappa = its size, the loss 1 - z_y + tau and the gradient
 *     grad_j = scale * ( [z_j > tau] / kappa - [j == y] ).
 * (Reference definition: reference_impl.py:11-35; closed form: src/cpu/fw_cpu.cpp:1-4.)
 *
 * Output conventions (every entry point):
 *   H[r]       largest float <= tau, so that for every float x:  x > H[r]  <=>  x > tau.  Any test
 *              "z > H" therefore selects exactly the support.
 *   losses[r]  (float)((1 - z_y) + tau), evaluated in fp64.
 *   kappa[r]   |{j : z_j > tau}|.
 *   mean_loss  (float)(sum_r losses[r] / N), summed in fp64 in a fixed order (deterministic).
 *   grad       inv = (float)(scale / kappa); grad[r,j] = z_j > tau ? inv : 0; grad[r,y] -= (float)scale.
 *              The ops that mirror the reference bake in scale = 1/N (mean reduction).
 * Threshold decisions are exact for rows whose fp64 partial sums are exact (every row whose
 * candidates (max-1, max] span fewer than 29 binades, which includes every finite row away from 0).
 *
 * Calling convention:
 *   - all pointers are device pointers; logits and grad are row-major [N, C], contiguous;
 *   - every call is asynchronous on `stream` and allocates nothing;
 *   - `workspace` is caller-provided device memory of at least fwl_workspace_bytes(N, C) bytes,
 *     8-byte aligned, with any contents: every call writes what it reads there before reading it
 *     (the mean's block partial sums, added by a one-block kernel after the rows; for few long rows
 *     the chunk thresholds and supports; for many long rows the support lists between the two
 *     passes).  No state survives from one call to the next.  Calls that run concurrently
 *     (different streams) must not share one workspace;
 *   - targets outside [0, C) do not fault: that row gets loss = NaN and no label term in grad;
 *   - NaN logits are never selected; rows without a finite maximum give kappa = 0, H = NaN;
 *   - the return value is FWL_OK or an fwl_status (argument errors are detected before launch);
 *   - calls are re-entrant: the dispatch switches of a call come from its fwl_options argument (the
 *     _ex entry points) or, for the others, from the process-wide defaults of fwl_set_params.
 */
#ifndef FWLOSS_H
#define FWLOSS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* hipStream_t;

enum fwl_status {
  FWL_OK = 0,
  FWL_ERR_INVALID_ARG = 1,  /* null pointer, N < 0, C < 1, C > 2^29 */
  FWL_ERR_WORKSPACE = 2,    /* workspace missing or smaller than fwl_workspace_bytes(N, C) */
  FWL_ERR_ALIGNMENT = 3,    /* logits/grad not aligned to their element size, targets not to 8 bytes */
  FWL_ERR_LAUNCH = 4,       /* the HIP runtime rejected a launch */
  FWL_ERR_DEVICE = 5        /* no usable gfx950 device current */
};

/* Element types of the logits accepted by fwl_forward_backward_typed. */
enum fwl_dtype {
  FWL_FLOAT32 = 0,
  FWL_BFLOAT16 = 1,   /* bfloat16 */
  FWL_FLOAT16 = 2     /* IEEE binary16 */
};

/* Dispatch switches of one call (the _ex entry points); NULL means the process-wide defaults of
 * fwl_set_params.  Each call reads only its own options, so calls with different options may run
 * at the same time from different host threads. */
typedef struct fwl_options {
  int path;       /* as fwl_set_params: 0 = automatic dispatch, 1-8 = a forced kernel family */
  int cand_cap;   /* LDS candidate capacity per wavefront of paths 2 and 4, in [64, 512]; 0 = 512 */
} fwl_options;

/* Human-readable text of a status code (static storage). */
const char* fwl_status_string(int status);

/* Bytes of device workspace the forward entry points need for an [N, C] problem: one fp64 per
 * block of the largest grid (>= 4096 blocks), rounded up to 256 bytes, then the larger of: 528
 * bytes per (row, chunk) for at most 128 rows of >= 24576 elements (the split rows), and 2056
 * bytes per row for >= 384 rows of >= 32000 elements, for batches of >= 32M elements in rows of
 * >= 8192, or for 8 rows per CU of >= 12000 elements (the fused op in two passes).  The answer follows the current fwl_set_params switches
 * (forcing path 7 needs the chunk scratch, forcing path 2 or 3 the two-pass scratch, for rows of
 * any length).  A smaller workspace is accepted: the mean needs only its first part, and without
 * room for the rest the one-pass kernels run. */
size_t fwl_workspace_bytes(int64_t N, int64_t C);

/* fwl_workspace_bytes for a call with these options (NULL: the process-wide defaults); 0 for
 * options out of range. */
size_t fwl_workspace_bytes_ex(int64_t N, int64_t C, const fwl_options* options);

/* Fused forward + backward: the whole hot path in one launch, reading logits once and writing the
 * dense gradient once.  mean_loss receives (float)(sum_r losses[r] / reduce_div) (reduce_div = N
 * for a mean, 1 for a sum).  Any of H, losses, kappa, mean_loss may be NULL.
 * Replaces the two-op sequence fw_radix_forward_small + fw_radix_backward_small
 * (src/cuda/fw_radix_argmax.cu:1381-1414, :1591-1609; driven by
 * benchmarks/cuda_benchmarks/CE_FW_perf.py:76-88) and the eager-gradient forward of the CPU
 * autograd Function (src/cpu/fw_cpu.cpp:721-741, scale as in :746-748). */
int fwl_forward_backward(const float* logits, const int64_t* targets, int64_t N, int64_t C,
                         double scale, double reduce_div, float* H, float* losses,
                         float* mean_loss, int32_t* kappa, float* grad, void* workspace,
                         size_t workspace_bytes, hipStream_t stream);

/* fwl_forward_backward for logits of element type `dtype` (enum fwl_dtype); grad has the same
 * element type.  16-bit logits are widened to fp32 exactly, every decision is the fp32 path's, and
 * the gradient values of the fp32 path are rounded to nearest-even on store; H, losses, mean_loss
 * and kappa are as for fp32 logits with the same values.  No reference counterpart: the reference
 * GPU ops accept fp32 only (src/cuda/fw_radix_argmax.cu:1385, :1421); this extends the fused op of
 * the CPU autograd path (src/cpu/fw_cpu.cpp:721-741), which dispatches on the logits' dtype
 * (fw_cpu.cpp:697-703). */
int fwl_forward_backward_typed(int dtype, const void* logits, const int64_t* targets, int64_t N,
                               int64_t C, double scale, double reduce_div, float* H, float* losses,
                               float* mean_loss, int32_t* kappa, void* grad, void* workspace,
                               size_t workspace_bytes, hipStream_t stream);

/* fwl_forward_backward_typed with a logits row stride and per-call options:
 *   ld        elements from one row of logits to the next (>= C; C for contiguous rows), so a
 *             column slice such as logits[:, 1:] needs no copy (grad stays contiguous [N, C]);
 *   losses64  optional fp64 per-row losses (1 - z_y) + tau, the value `losses` rounds; the
 *             reference CPU path returns its per-row losses in fp64 (src/cpu/fw_cpu.cpp:614,
 *             :750-757, fw_loss_grad);
 *   options   dispatch switches of this call (NULL: the fwl_set_params defaults).
 * Outputs as fwl_forward_backward_typed; every pointer output may be NULL but grad. */
int fwl_forward_backward_ex(int dtype, const void* logits, int64_t ld, const int64_t* targets, int64_t N,
                            int64_t C, double scale, double reduce_div, float* H, float* losses,
                            double* losses64, float* mean_loss, int32_t* kappa, void* grad,
                            void* workspace, size_t workspace_bytes, const fwl_options* options,
                            hipStream_t stream);

/* fwl_forward_backward_ex without the workspace arguments: it allocates nothing and takes no
 * workspace, for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation).  No counterpart in the reference, whose ops
 * allocate their outputs and scratch (src/cuda/fw_radix_argmax.cu:1390-1393, :1426-1453).  The
 * caller passes the inputs and outputs; the workspace is a static device array of
 * fwl_noalloc_scratch_bytes() bytes (64 MiB) in the library, one per device, looked up once per
 * device.  Calls on one device share it: calls that overlap on one device (several streams or
 * threads at once) race and give undefined results.  A call whose workspace (fwl_workspace_bytes_ex
 * with the same options) exceeds the array returns FWL_ERR_WORKSPACE before any launch: the mean
 * and overflow records need about 8 bytes per row, many long rows 2056 more (about 8M rows of short
 * rows, or 32000 rows of >= 32000 elements). */
size_t fwl_noalloc_scratch_bytes(void);
int fwl_forward_backward_noalloc(int dtype, const void* logits, int64_t ld, const int64_t* targets,
                                 int64_t N, int64_t C, double scale, double reduce_div, float* H,
                                 float* losses, double* losses64, float* mean_loss, int32_t* kappa,
                                 void* grad, const fwl_options* options, hipStream_t stream);

/* fwl_forward_backward for float64 logits (the reference CPU path's second dtype,
 * src/cpu/fw_cpu.cpp:697-703, run_generic<double>; the reference GPU ops take float32 only).
 * Every decision is taken in fp64: tau from fixed-point iterations t <- H({z > t}) with sums in a
 * fixed order; H[r] = tau (so z > H[r] is the support); losses, mean_loss and grad are fp64
 * (grad[r,j] = z_j > tau ? scale / kappa : 0, minus scale at the label).  mean_loss needs losses.
 * No workspace: the mean is reduced by a one-block kernel after the rows. */
int fwl_forward_backward_f64(const double* logits, const int64_t* targets, int64_t N, int64_t C,
                             double scale, double reduce_div, double* H, double* losses,
                             double* mean_loss, int32_t* kappa, double* grad, hipStream_t stream);

/* fwl_scale_grad for an fp64 gradient and fp64 factors (FWFunction::backward, fw_cpu.cpp:734-740). */
int fwl_scale_grad_f64(double* grad, const double* grad_output, int64_t go_stride, int64_t N,
                       int64_t C, hipStream_t stream);

/* Forward with the support mask: selected[r,j] = (z_j > tau) as bytes 0/1 (torch.bool layout).
 * Replaces fw_radix_forward_small (src/cuda/fw_radix_argmax.cu:1381-1414; binding.cpp:11):
 * outputs [H, losses, mean_loss, kappa, selected_logits]. */
int fwl_forward_small(const float* logits, const int64_t* targets, int64_t N, int64_t C,
                      float* H, float* losses, float* mean_loss, int32_t* kappa,
                      uint8_t* selected, void* workspace, size_t workspace_bytes,
                      hipStream_t stream);

/* grad[r,j] = (selected[r,j] ? (float)((1/N)/kappa[r]) : 0) - [j == y_r] * (float)(1/N).
 * Replaces fw_radix_backward_small (src/cuda/fw_radix_argmax.cu:1561-1609; binding.cpp:12). */
int fwl_backward_small(const int64_t* targets, const uint8_t* selected, const int32_t* kappa,
                       int64_t N, int64_t C, float* grad, hipStream_t stream);

/* Forward with candidate lists.  Row r's list (cand_values[r*C + p], cand_indices[r*C + p],
 * p < cand_counts[r]) holds exactly the support, so cand_counts[r] == kappa[r]; entries past the
 * count are left untouched.  The order of a list is deterministic, not sorted.
 * Replaces fw_radix_forward (src/cuda/fw_radix_argmax.cu:1417-1496; binding.cpp:9): outputs
 * [H, losses, mean_loss, kappa, candidate_buffer, candidate_indices, candidate_counts]. */
int fwl_forward_large(const float* logits, const int64_t* targets, int64_t N, int64_t C,
                      float* H, float* losses, float* mean_loss, int32_t* kappa,
                      float* cand_values, int32_t* cand_indices, int32_t* cand_counts,
                      void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Dense gradient from candidate lists: zeros, then (float)((1/N)/kappa[r]) at every listed index
 * whose listed value is > H[r], then -(float)(1/N) at y_r (added to the selected value when y_r is
 * selected, tested as logits[r, y_r] > H[r]).
 * Replaces fw_radix_backward (src/cuda/fw_radix_argmax.cu:1498-1559; binding.cpp:10). */
int fwl_backward_large(const float* logits, const int64_t* targets, const float* H,
                       const int32_t* kappa, const float* cand_values,
                       const int32_t* cand_indices, const int32_t* cand_counts, int64_t N,
                       int64_t C, float* grad, hipStream_t stream);

/* grad[r, :] *= grad_output[r * go_stride] for every row whose factor is not 1 (go_stride = 0: one
 * scalar for all rows, as for a 'mean'/'sum' loss; 1: one factor per row, as for 'none').  The
 * factor is read on the device, so the autograd backward needs no host synchronisation; rows with
 * factor 1 are not touched.  Counterpart of FWFunction::backward (src/cpu/fw_cpu.cpp:734-740),
 * which skips the multiply when grad_output == 1. */
int fwl_scale_grad(float* grad, const float* grad_output, int64_t go_stride, int64_t N, int64_t C,
                   hipStream_t stream);

/* fwl_scale_grad for a gradient of element type `dtype` (enum fwl_dtype): each element is widened
 * to fp32, multiplied, and rounded to nearest-even.  The backward of fwl_forward_backward_typed
 * (src/cpu/fw_cpu.cpp:734-740 scales in the logits' dtype). */
int fwl_scale_grad_typed(int dtype, void* grad, const float* grad_output, int64_t go_stride, int64_t N,
                         int64_t C, hipStream_t stream);

/* ---- The linear layer that produces the logits, fused with the loss ("LM head").
 * No counterpart in the reference: its losses take materialised logits (reference_impl.py:11-35,
 * src/cpu/fw_cpu.cpp:721-741, src/cuda/fw_radix_argmax.cu:1381-1496).  For hidden [N, d] and
 * weight [V, d], logits = hidden @ weight^T are handed over one vocabulary chunk at a time
 * (columns v0 .. v0 + Vc - 1), so no [N, V] tensor is needed:
 *   fwl_linear_begin    once per batch (state: fwl_linear_state_bytes(N) bytes, 16-byte aligned);
 *   fwl_linear_chunk    once per chunk (logits [N, Vc] with row stride ld, v0 + Vc <= V), in
 *                       any order, each column exactly once;
 *   fwl_linear_finish   H, losses, kappa and the support's columns (support[r * cap + p],
 *                       p < kappa[r], cap = fwl_linear_support_cap()) of every row.  Rows with
 *                       overflow[r] = 1 (more than cap entries within 1 of the maximum after
 *                       tightening, or no finite maximum) are not solved: the caller runs them
 *                       through fwl_forward_backward_typed on their materialised logits;
 *   fwl_linear_dhidden  dhidden[r] = sum_j g_rj weight[j] over the row's kappa + 1 non-zero
 *                       gradient columns (no GEMM), where g is the fused op's gradient with
 *                       scale s_r = row_scale[r * rs_stride];
 *   fwl_linear_coo      the (column, row) entries of g: row r's at offsets[r] (exclusive prefix
 *                       sum of kappa[r] + [label outside the support]), key = column * 2N + 2r
 *                       (+1 for a label entry), value g;
 *   fwl_linear_dweight  dweight[j] = sum of g * hidden[row] over column j's entries, given the
 *                       entries sorted by key (keys with a column outside [0, V) are skipped);
 *                       rows of dweight without entries are not written (zero-fill them first).
 * Every decision is the one fwl_forward_backward_typed takes on the same logits: H, losses and
 * kappa are bit-identical to it.  Element types as enum fwl_dtype (logits, weight, hidden and the
 * gradients share one). */
size_t fwl_linear_state_bytes(int64_t N);
int fwl_linear_support_cap(void);
int fwl_linear_begin(void* state, int64_t N, hipStream_t stream);
int fwl_linear_chunk(int dtype, const void* logits, int64_t N, int64_t Vc, int64_t ld, int64_t v0,
                     int64_t V, const int64_t* targets, void* state, hipStream_t stream);
int fwl_linear_finish(const void* state, const int64_t* targets, int64_t N, int64_t V, float* H,
                      float* losses, int32_t* kappa, int32_t* support, int32_t* overflow,
                      hipStream_t stream);
int fwl_linear_dhidden(int dtype, const void* weight, int64_t V, int64_t d, const int64_t* targets,
                       const int32_t* kappa, const int32_t* support, const float* row_scale,
                       int64_t rs_stride, int64_t N, void* dhidden, hipStream_t stream);
int fwl_linear_coo(const int64_t* targets, int64_t N, int64_t V, const int32_t* kappa,
                   const int32_t* support, const int64_t* offsets, const float* row_scale,
                   int64_t rs_stride, int64_t* keys, float* values, hipStream_t stream);
int fwl_linear_dweight(int dtype, const void* hidden, int64_t N, int64_t V, int64_t d,
                       const int64_t* keys, const float* values, int64_t P, void* dweight,
                       hipStream_t stream);

/* Process-wide default dispatch switches, the GPU counterpart of the reference CPU path's
 * set_params (src/cpu/fw_cpu.cpp:758-763, used by its tests to force each branch).  A call reads
 * the defaults once, at its start (atomically); a call that needs its own switches passes
 * fwl_options to an _ex entry point instead.
 *   path:      0 = automatic (7 for at most 128 rows of at least 96 KiB, 6 for short rows, 1 for
 *              C <= 2048 or C <= 1024 when rows are not 16-byte aligned, 4 for C <= 8192, else 2),
 *              1 = one wavefront per row with the row in registers (C <= 2048, or 1024 for rows
 *              that are not 16-byte aligned; larger C runs path 4),
 *              2 = one block per row, streamed, with LDS candidate lists,
 *              3 = path 2 with the overflow solve forced (rows solved in memory: a histogram
 *              pass, at most 4 refinements, a collect pass; a bounded bisection as last resort),
 *              4 = one wavefront per row, streamed, with an LDS candidate list,
 *              5 = path 4 with the overflow solve forced,
 *              6 = short rows: 16- or 32-lane segments of a wavefront, 4 or 2 rows per
 *              iteration (rows of up to 64 units; longer rows and candidate lists run path 1),
 *              7 = split rows: one block per (row, chunk of >= 4096 elements) streams the chunk
 *              and keeps its own support, then one block per row resolves their union (at most
 *              128 rows, and a workspace of fwl_workspace_bytes(N, C) taken with path 7 set;
 *              otherwise path 2 runs),
 *              8 = path 1 without line-aligned windows (path 1 reads and writes 16-byte aligned
 *              fp32 gradient rows through windows that start on the row's first 128-byte line
 *              boundary, where the logits and gradient share their offsets within a line).
 *   cand_cap:  LDS candidate capacity per wavefront of paths 2 and 4, in [64, 512] (512 =
 *              default); smaller values make rows overflow into the overflow solve sooner and
 *              shrink its LDS list, so that more rows take its refinement passes.
 * Returns FWL_ERR_INVALID_ARG for values out of range. */
int fwl_set_params(int path, int cand_cap);
int fwl_get_params(int* path, int* cand_cap);

#ifdef __cplusplus
}
#endif
#endif /* FWLOSS_H */
