/*
 * hilda_kernel_amd.h — C ABI of the MI355X (gfx950) operator hot path.
 *
 * Every entry point replaces one Triton launch site (or launch wrapper) of
 * kirsten-1/hilda-kernel; the citation in front of each declaration names the
 * reference code it stands in for (paths relative to triton-kernels/kernels/).
 *
 * Conventions
 *  - Plain pointers and sizes only. Device pointers are HIP device memory
 *    (torch tensors' data_ptr()); `stream` is a hipStream_t passed as void*.
 *  - The caller owns all memory. Scratch space an op needs is passed in as
 *    `workspace`, sized by the matching *_workspace_size() call.
 *  - No entry point synchronises the device or allocates device memory. The
 *    fused-linear entry points with gradients run their transposes on a
 *    second stream the library creates once per host thread and device
 *    (default priority, non-blocking; kept until the process ends), forked
 *    from `stream` and joined back to it with events before they return, so
 *    the caller sees one stream.
 *  - dtype codes: HK_F32 = 0, HK_F16 = 1, HK_BF16 = 2.
 *  - Return value: 0 on success; HK_EINVAL (-1) when an argument is rejected
 *    (checked before any HIP call, so this is testable without a GPU);
 *    a positive hipError_t when the HIP runtime reports an error.
 *    hk_last_error() returns the thread-local text of the last failure.
 */
#ifndef HILDA_KERNEL_AMD_H
#define HILDA_KERNEL_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HK_ABI_VERSION 2

#define HK_F32 0
#define HK_F16 1
#define HK_BF16 2
/* integer codes, used for masks */
#define HK_U8 3
#define HK_I32 4
#define HK_I64 5

/* loss reductions */
#define HK_REDUCTION_NONE 0
#define HK_REDUCTION_MEAN 1
#define HK_REDUCTION_SUM 2
#define HK_REDUCTION_BATCHMEAN 3 /* KLDiv only: sum / rows */

/* dW reduction path for the norm backward passes */
#define HK_DW_AUTO 0    /* partial (faster than atomic at every size)     */
#define HK_DW_ATOMIC 1  /* fp64 atomics into one [cols] accumulator       */
#define HK_DW_PARTIAL 2 /* per-row-group partial rows + a reduction pass  */

typedef void* hk_stream_t;

/* ----------------------------------------------------------------------- */
/* library                                                                 */
/* ----------------------------------------------------------------------- */
int hk_abi_version(void);
const char* hk_last_error(void);
/* Number of compute units of `device` (cached): the persistent grids and the
 * RMSNorm backward's row groups are sized by it (the reference reads
 * multi_processor_count for its dW path choice, rms_norm.py:325-326). */
int hk_device_cu_count(int device);

/* ----------------------------------------------------------------------- */
/* RMSNorm                                                                 */
/* ----------------------------------------------------------------------- */
/* Replaces _rms_norm_forward_kernel launch, rms_norm.py:293-304.
 * y[r,:] = ((x[r,:] * rstd[r]) rounded to dtype_x) * w ; rstd[r] = 1/sqrt(mean(x^2)+eps) */
int hk_rms_norm_fwd(void* y, float* rstd, const void* x, const void* w, int64_t rows, int64_t cols,
                    int64_t ld_x, int64_t ld_y, int dtype_x, int dtype_w, float eps, hk_stream_t stream);

/* Bytes of workspace hk_rms_norm_bwd / hk_fused_add_rms_norm_bwd need. */
size_t hk_rms_norm_bwd_workspace_size(int64_t rows, int64_t cols, int dtype_x, int dtype_w,
                                      int dw_mode, int device);

/* Replaces rms_norm_backward, rms_norm.py:309-359 (atomic kernel :152-193,
 * partial kernel :200-254 plus the torch sum/cast at :357-359).
 * dx = rstd*(dy*w) - rstd^3 * (sum(dy*w*x)/cols) * x ; dw = sum_r dy*x*rstd (cast to dtype_w). */
int hk_rms_norm_bwd(void* dx, void* dw, const void* dy, const void* x, const void* w, const float* rstd,
                    int64_t rows, int64_t cols, int64_t ld_dy, int64_t ld_x, int64_t ld_dx, int dtype_x,
                    int dtype_w, int dw_mode, void* workspace, size_t workspace_bytes, hk_stream_t stream);

/* No counterpart in the reference. hk_rms_norm_bwd for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): the same kernels and result, with the dW scratch in a
 * device array the library holds for each GPU it runs on (16 MiB, until the
 * process ends) instead of a workspace argument. Calls whose
 * hk_rms_norm_bwd_workspace_size exceeds 16 MiB are rejected with HK_EINVAL
 * (e.g. fp32 rows wider than 8192 columns on a 256-CU GPU). Allocates nothing.
 * Every call on one GPU uses that GPU's one array: calls that overlap on one
 * GPU (on different streams, or from host threads without ordering) race. */
int hk_rms_norm_bwd_noalloc(void* dx, void* dw, const void* dy, const void* x, const void* w, const float* rstd,
                            int64_t rows, int64_t cols, int64_t ld_dy, int64_t ld_x, int64_t ld_dx, int dtype_x,
                            int dtype_w, int dw_mode, hk_stream_t stream);

/* ----------------------------------------------------------------------- */
/* FusedAddRMSNorm                                                         */
/* ----------------------------------------------------------------------- */
/* Replaces _fused_add_rms_norm_fwd_kernel launch, fused_add_rms_norm.py:172-188.
 * s = x + r (rounded to dtype_x, stored); y = RMSNorm(s) * w. All four row
 * tensors share the row stride `ld`. */
int hk_fused_add_rms_norm_fwd(void* y, void* s, float* rstd, const void* x, const void* r, const void* w,
                              int64_t rows, int64_t cols, int64_t ld, int dtype_x, int dtype_w, float eps,
                              hk_stream_t stream);

/* Replaces fused_add_rms_norm_backward, fused_add_rms_norm.py:191-232.
 * dx = RMSNormBwd(dy; s) + ds_out (ds_out may be NULL); the same dx is the
 * gradient of both x and r. */
int hk_fused_add_rms_norm_bwd(void* dx, void* dw, const void* dy, const void* ds_out, const void* s,
                              const void* w, const float* rstd, int64_t rows, int64_t cols, int64_t ld,
                              int dtype_x, int dtype_w, int dw_mode, void* workspace, size_t workspace_bytes,
                              hk_stream_t stream);

/* ----------------------------------------------------------------------- */
/* RoPE                                                                    */
/* ----------------------------------------------------------------------- */
/* Replaces _rope_fwd_kernel launches (rope.py:95-106) for one tensor in
 * either direction: rope_forward (rope.py:113-136) with inverse = 0 and
 * rope_backward (rope.py:139-172) with inverse = 1 (sin negated in-kernel).
 * x / out: (B, H, T, D) logical with element strides s*; the last dim must
 * be contiguous. cos/sin: (cos_B, T', D/2) with cos_B in {1, B}, last dim
 * contiguous, rows indexed by t. */
int hk_rope(void* out, const void* in, const void* cos, const void* sin, int64_t B, int64_t H, int64_t T, int64_t D,
            int64_t in_sB, int64_t in_sH, int64_t in_sT, int64_t out_sB, int64_t out_sH, int64_t out_sT,
            int64_t cos_B, int64_t cos_sB, int64_t cos_sT, int dtype_x, int dtype_cs, int inverse,
            hk_stream_t stream);

/* Replaces the pair of _launch calls in rope_forward (rope.py:133-134) and
 * rope_backward (rope.py:169-170): q (B, Hq, T, D) and k (B, Hk, T, D), each
 * with its own input/output strides, rotated by the same cos/sin in one
 * launch. Arguments as for hk_rope. */
int hk_rope_qk(void* q_out, const void* q_in, int64_t Hq, int64_t q_in_sB, int64_t q_in_sH, int64_t q_in_sT,
               int64_t q_out_sB, int64_t q_out_sH, int64_t q_out_sT, void* k_out, const void* k_in, int64_t Hk,
               int64_t k_in_sB, int64_t k_in_sH, int64_t k_in_sT, int64_t k_out_sB, int64_t k_out_sH,
               int64_t k_out_sT, const void* cos, const void* sin, int64_t B, int64_t T, int64_t D, int64_t cos_B,
               int64_t cos_sB, int64_t cos_sT, int dtype_x, int dtype_cs, int inverse, hk_stream_t stream);

/* ----------------------------------------------------------------------- */
/* SwiGLU                                                                  */
/* ----------------------------------------------------------------------- */
/* Replaces _swiglu_fwd_kernel launch (swiglu.py:112-124) on n contiguous
 * elements: c = (silu(a) in fp32, rounded to dtype) * b. */
int hk_swiglu_fwd(void* c, const void* a, const void* b, int64_t n, int dtype, hk_stream_t stream);

/* Replaces _swiglu_bwd_kernel launch (swiglu.py:127-141); writes da and db to
 * separate buffers instead of over a and b:
 * db = dc * silu(a); da = dc * b * sig(a) * (1 + a * (1 - sig(a))). */
int hk_swiglu_bwd(void* da, void* db, const void* a, const void* b, const void* dc, int64_t n, int dtype,
                  hk_stream_t stream);

/* ----------------------------------------------------------------------- */
/* GeGLU (tanh-approximated GELU gate)                                     */
/* ----------------------------------------------------------------------- */
/* Replaces _geglu_fwd_kernel launch (geglu.py:131-143) on n contiguous
 * elements: c = (gelu_tanh(a) in fp32, rounded to dtype) * b, where
 * gelu_tanh(a) = 0.5 a (1 + tanh(sqrt(2/pi) (a + 0.044715 a^3))) (geglu.py:69-71). */
int hk_geglu_fwd(void* c, const void* a, const void* b, int64_t n, int dtype, hk_stream_t stream);

/* Replaces _geglu_bwd_kernel launch (geglu.py:146-159); writes da and db to
 * separate buffers instead of over a and b: db = dc * gelu_tanh(a),
 * da = dc * b * gelu_tanh'(a) (geglu.py:110-124). */
int hk_geglu_bwd(void* da, void* db, const void* a, const void* b, const void* dc, int64_t n, int dtype,
                 hk_stream_t stream);

/* ----------------------------------------------------------------------- */
/* KL divergence and JSD                                                   */
/* ----------------------------------------------------------------------- */
/* Replaces _kl_div_fwd_kernel launch + reduction (kl_div.py:114-138):
 * loss_rows[r] = sum_c t (log max(t, eps) - y), or e^t (t - y) with log_target
 * (y = y_pred log-probabilities, t = y_true); loss_out (nullable; unused for
 * HK_REDUCTION_NONE) = sum (SUM), sum / rows (BATCHMEAN) or
 * sum / (rows * cols) (MEAN). Rows have element strides ld_pred / ld_true. */
int hk_kl_div_fwd(float* loss_out, float* loss_rows, const void* y_pred, const void* y_true, int64_t rows,
                  int64_t cols, int64_t ld_pred, int64_t ld_true, int log_target, float eps, int reduction, int dtype,
                  hk_stream_t stream);

/* Replaces kl_div_backward (kl_div.py:141-166): dy_pred = -(t or e^t) * g * factor,
 * with g[r] per row (per_row = 1, the 'none' reduction) or g[0], read on the
 * device (the reference's float(grad_output) host read, :147-155, is gone). */
int hk_kl_div_bwd(void* dy_pred, const void* y_true, const float* g, int per_row, float factor, int64_t rows,
                  int64_t cols, int64_t ld_true, int64_t ld_out, int log_target, int dtype, hk_stream_t stream);

/* Bytes of device workspace hk_jsd_fwd needs when labels are given. */
size_t hk_jsd_workspace_size(void);

/* Replaces jsd_forward (jsd.py:97-135, kernel :30-90): X student and Y teacher
 * log-probabilities; per row the JSD(beta) loss and its gradient in X, both
 * divided by max(#labels != ignore_index, 1) (counted on the device; all rows
 * without labels); rows whose label is ignore_index get loss 0 and dX = 0.
 * loss_out (nullable) = sum of loss_rows. dX has X's dtype. */
int hk_jsd_fwd(float* loss_out, float* loss_rows, void* dX, const void* X, const void* Y, const int64_t* labels,
               int64_t ignore_index, float beta, int64_t rows, int64_t cols, int64_t ldx, int64_t ldy, int64_t ld_dx,
               int dtype, void* workspace, size_t workspace_bytes, hk_stream_t stream);

/* Bytes of device workspace hk_fused_linear_jsd needs for a call with the same
 * shape, chunk, budget, dtype, gradient and label choice and the same input
 * pointers (nullable: taken as 16-byte aligned); Ht: the teacher's hidden
 * size. 0 for an invalid shape or a budget no plan fits (see
 * hk_fused_linear_cross_entropy_workspace_size for chunk and budget). The
 * default budget here is at least what the reference's chunk loop holds at
 * once (fused_linear_jsd.py:133-135,159-203): c*V*22 bytes (16 for fp32) for
 * its chunk tensors, c = next_pow2(ceil(BT / ceil(V/H))) rows at most BT, and
 * V*H*es for its dlogits^T X product. The outputs are the reference's, so the
 * default peak memory stays at or below the reference's; without a
 * vocabulary-tiled plan, smaller budgets mean short row chunks whose dW pass
 * rewrites the whole weight gradient each chunk. */
size_t hk_fused_linear_jsd_workspace_size(int64_t BT, int64_t H, int64_t Ht, int64_t V, int64_t chunk,
                                          int64_t workspace_budget, int dtype, int with_grad, int with_labels,
                                          const void* s_input, const void* s_weight, const void* t_input,
                                          const void* t_weight);

/* No counterpart in the reference: the plan the call above sizes, in
 * hk_fused_linear_cross_entropy_plan's info[8] layout (never vocabulary
 * tiles). */
int hk_fused_linear_jsd_plan(int64_t BT, int64_t H, int64_t Ht, int64_t V, int64_t chunk, int64_t workspace_budget,
                             int dtype, int with_grad, int with_labels, const void* s_input, const void* s_weight,
                             const void* t_input, const void* t_weight, int64_t* info);

/* Replaces fused_linear_jsd_forward (fused_linear_jsd.py:114-205): per chunk,
 * student logits s_input[BT,H] * s_weight[V,H]^T and teacher logits
 * t_input[BT,Ht] * t_weight[V,Ht]^T on MFMA (fp32, bf16 or fp16), both
 * temperature log-softmaxes, JSD(beta) per row divided by
 * max(#labels != ignore_index, 1) (BT without labels), and (dinput, dweight
 * non-null) the student dlogits contracted into dinput [BT,H] and dweight
 * [V,H]. Rows labelled ignore_index are compacted away on the device before
 * the GEMMs. The teacher gets no gradient. *loss_out = the summed loss. Rows
 * are contiguous; any H, Ht and V. The chunk engine and its memory plans are
 * hk_fused_linear_cross_entropy's. */
int hk_fused_linear_jsd(float* loss_out, void* dinput, void* dweight, const void* s_input, const void* s_weight,
                        const void* t_input, const void* t_weight, const int64_t* labels, int64_t BT, int64_t H,
                        int64_t Ht, int64_t V, int64_t ignore_index, float beta, float temperature, int dtype,
                        int64_t chunk, int64_t workspace_budget, void* workspace, size_t workspace_bytes,
                        hk_stream_t stream);

/* ----------------------------------------------------------------------- */
/* FusedLinear-GRPO                                                        */
/* ----------------------------------------------------------------------- */
/* No counterpart in the reference: its GRPO op takes materialised logits
 * (grpo_loss.py:241-330). This is that op behind the lm_head, chunked like
 * fused_linear_cross_entropy_forward (fused_linear_cross_entropy.py:103-171),
 * so the (B, L+1, V) logits are never formed whole under the default budget.
 * Bytes of workspace it needs for a call with the same arguments (0 for an
 * invalid shape or a budget no plan fits; chunk and budget as for
 * hk_fused_linear_cross_entropy_workspace_size, the default budget at least
 * twice the weight's bytes, 2*V*H*es: without a vocabulary-tiled plan,
 * smaller budgets mean short row chunks whose dW pass rewrites the whole
 * weight gradient each chunk). */
size_t hk_fused_linear_grpo_workspace_size(int64_t B, int64_t L, int64_t H, int64_t V, int64_t chunk,
                                           int64_t workspace_budget, int dtype, int with_grad, const void* hidden,
                                           const void* weight);

/* No counterpart in the reference: the plan the call above sizes, in
 * hk_fused_linear_cross_entropy_plan's info[8] layout (rows per chunk over
 * the B*(L+1) positions; never vocabulary tiles). */
int hk_fused_linear_grpo_plan(int64_t B, int64_t L, int64_t H, int64_t V, int64_t chunk, int64_t workspace_budget,
                              int dtype, int with_grad, const void* hidden, const void* weight, int64_t* info);

/* hidden (B, L+1, H) and weight [V, H] (fp32, bf16 or fp16, contiguous, any H and V): logits =
 * hidden weight^T, then exactly hk_grpo_loss_fwd's loss, kl_mean, clip_ratio
 * and per-token rows, and with dhidden (B, L+1, H) / dweight [V, H] (both or
 * neither) the gradients of the loss at unit upstream gradient (zero rows of
 * dhidden at masked tokens and at position L). */
int hk_fused_linear_grpo(float* loss_out, float* kl_out, float* clip_out, float* lse_rows, float* loss_rows,
                         float* kl_rows, float* clip_rows, void* dhidden, void* dweight, const void* hidden,
                         const void* weight, const int64_t* ids, int64_t ids_sB, int64_t ids_sL,
                         const float* advantages, const float* old_logp, int64_t old_sB, int64_t old_sL,
                         const float* ref_logp, int64_t ref_sB, int64_t ref_sL, const void* mask, int mask_dtype,
                         int64_t mask_sB, int64_t mask_sL, int64_t B, int64_t L, int64_t H, int64_t V,
                         float temperature, float beta, float eps_low, float eps_high, int dtype, int64_t chunk,
                         int64_t workspace_budget, void* workspace, size_t workspace_bytes, hk_stream_t stream);

/* ----------------------------------------------------------------------- */
/* AttnRes (attention residuals over depth)                                */
/* ----------------------------------------------------------------------- */
/* Replaces attn_res_forward (attn_res.py:209-257, kernel :31-98): V holds
 * n_blocks stacked blocks [n_blocks, n_tokens, D]; per token
 * k_i = round(round(v_i * rstd_i) * w_norm), score_i = <w_query, k_i>,
 * alpha = softmax over blocks, out = sum_i alpha_i v_i (dtype of V).
 * alpha and rstd are [n_blocks, n_tokens] fp32 (saved for the backward).
 * 1 <= n_blocks <= 32; D a multiple of 16/sizeof(dtype), at most 2048 vectors of 16 bytes. */
int hk_attn_res_fwd(void* out, float* alpha, float* rstd, const void* V, const void* w_query, const void* w_norm,
                    int64_t n_blocks, int64_t n_tokens, int64_t D, float eps, int dtype, hk_stream_t stream);

/* Bytes of device workspace hk_attn_res_bwd needs (fp32 partial rows). */
size_t hk_attn_res_bwd_workspace_size(int64_t n_tokens, int64_t D);

/* Replaces attn_res_backward (attn_res.py:260-288, kernel :101-190): dV
 * [n_blocks, n_tokens, D] and dw_query / dw_norm [D] (dtype of the weights,
 * summed over tokens in fp64 from per-block fp32 partials instead of fp32
 * atomics). */
int hk_attn_res_bwd(void* dV, void* dw_query, void* dw_norm, const void* dh, const void* V, const void* w_query,
                    const void* w_norm, const float* alpha, const float* rstd, int64_t n_blocks, int64_t n_tokens,
                    int64_t D, int dtype, void* workspace, size_t workspace_bytes, hk_stream_t stream);

/* ----------------------------------------------------------------------- */
/* CrossEntropy                                                            */
/* ----------------------------------------------------------------------- */
/* Bytes of device workspace the CrossEntropy entry points use:
 * 256 + roundup(4 * rows, 256) for rows < 2^31 (256 beyond): 256 for the
 * counts, then the launch plan of hk_cross_entropy_fwd_grad (4 bytes a row),
 * which deals the rows that get a gradient out evenly over the GPU. A
 * workspace of 256 bytes or more but less than this is accepted and runs
 * without the plan. */
size_t hk_cross_entropy_workspace_size(int64_t rows);

/* Replaces cross_entropy_forward's training path (cross_entropy.py:206-236:
 * _n_valid_tensor :196-199, _ce_train_forward_kernel_ignore :114-166 and
 * _ce_train_forward_kernel_no_ignore :72-111, per_token_loss.sum() :236).
 * loss_rows[r] = (lse_r - x[r,t_r]) * s, dlogits[r,:] = (softmax_r - onehot_r) * s with
 * s = 1/max(n_valid,1) for mean, 1 otherwise; ignored rows: 0 and a zero row.
 * ignore_index == -1 means "ignore nothing". n_valid stays on the device.
 * loss_out (nullable) receives sum(loss_rows). */
int hk_cross_entropy_fwd_grad(void* dlogits, float* loss_rows, float* loss_out, const void* logits,
                              const int64_t* targets, int64_t rows, int64_t V, int64_t ld_logits, int64_t ld_dlogits,
                              int64_t ignore_index, int reduction, int dtype, void* workspace, size_t workspace_bytes,
                              hk_stream_t stream);

/* Replaces the inference path of cross_entropy_forward (cross_entropy.py:238-249,
 * _ce_forward_kernel :32-65): lse_rows, loss_rows = lse - x_t (0 if ignored);
 * loss_out (nullable) = sum, or sum / max(n_valid, 1) for mean. */
int hk_cross_entropy_fwd(float* lse_rows, float* loss_rows, float* loss_out, const void* logits,
                         const int64_t* targets, int64_t rows, int64_t V, int64_t ld_logits, int64_t ignore_index,
                         int reduction, int dtype, void* workspace, size_t workspace_bytes, hk_stream_t stream);

/* Replaces _ce_scale_grad_kernel (cross_entropy.py:173-189) and
 * _element_mul_kernel (fused_linear_cross_entropy.py:84-96):
 * out = in * g (g scalar or per row, read on the device), or in * g / g_prev
 * when g_prev is given (0 where g_prev is 0). With skip_if_one, out == in and
 * a scalar g == 1 the kernel returns without touching memory, which replaces
 * the host-synchronising torch.equal test at cross_entropy.py:202-203. */
int hk_scale_rows(void* out, const void* in, const float* g, const float* g_prev, int per_row, int skip_if_one,
                  int64_t rows, int64_t cols, int64_t ld_in, int64_t ld_out, int dtype, hk_stream_t stream);

/* ----------------------------------------------------------------------- */
/* GRPO                                                                    */
/* ----------------------------------------------------------------------- */
/* Replaces fused_selective_log_softmax (grpo_loss.py:65-80, kernel :29-62).
 * logits: (B, L+1, V) contiguous; logp[b,l] = x[b,l,id]/T - logsumexp(x[b,l,:]/T)
 * for l < L with id = ids[b*ids_sB + l*ids_sL]; 0 where mask == 0 (mask
 * nullable, dtype HK_F32/F16/BF16/U8/I32/I64, element strides). */
int hk_selective_log_softmax(float* logp, const void* logits, const int64_t* ids, int64_t ids_sB, int64_t ids_sL,
                             const void* mask, int mask_dtype, int64_t mask_sB, int64_t mask_sL, int64_t B, int64_t L,
                             int64_t V, float temperature, int dtype, hk_stream_t stream);

/* Bytes of device workspace hk_grpo_loss_fwd needs. */
size_t hk_grpo_workspace_size(int64_t B, int64_t L);

/* Replaces grpo_loss_forward (grpo_loss.py:241-297) and, fused into the same
 * pass at unit upstream gradient, grpo_loss_backward (grpo_loss.py:300-330).
 * Scalars loss_out, kl_out (nullable) and clip_out receive the reduced loss,
 * kl_mean and clip_ratio (grpo_loss.py:290-295); per-token lse/loss/kl/clipped rows
 * [B, L]; dlogits (nullable: forward only) is (B, L+1, V) with zero rows at
 * masked tokens and at position L. old_logp (nullable: on-policy) and
 * ref_logp (required when beta != 0) are fp32 with element strides. */
int hk_grpo_loss_fwd(void* dlogits, float* loss_out, float* kl_out, float* clip_out, float* lse_rows,
                     float* loss_rows, float* kl_rows, float* clip_rows, const void* logits, const int64_t* ids,
                     int64_t ids_sB, int64_t ids_sL, const float* advantages, const float* old_logp, int64_t old_sB,
                     int64_t old_sL, const float* ref_logp, int64_t ref_sB, int64_t ref_sL, const void* mask,
                     int mask_dtype, int64_t mask_sB, int64_t mask_sL, int64_t B, int64_t L, int64_t V,
                     float temperature, float beta, float eps_low, float eps_high, int dtype, void* workspace,
                     size_t workspace_bytes, hk_stream_t stream);

/* ----------------------------------------------------------------------- */
/* FusedLinearCrossEntropy                                                 */
/* ----------------------------------------------------------------------- */
/* Bytes of device workspace hk_fused_linear_cross_entropy needs for a call
 * with the same shape, chunk, budget, dtype and gradient choice and the same
 * hidden/weight pointers (nullable: taken as 16-byte aligned); 0 for an
 * invalid shape or a budget no plan fits.
 *   chunk: most rows per chunk (<= 0: 8192).
 *   workspace_budget: 0 selects the default budget: the larger of 40 MiB and
 *     what the reference's chunk costs (fused_linear_cross_entropy.py:112-114:
 *     C0 = next_pow2(ceil(BT / ceil(V / H))) rows, 64 to 8192, whose logits
 *     are about the size of the hidden states) in the leanest layout, plus an
 *     eighth of the chunk's logits bytes for split partial sums; < 0 no limit
 *     (the fastest plan); > 0 at most that many bytes. Within the budget the
 *     plan with the least modelled time is taken, except that a plan which
 *     sums dW in the 16-bit output across chunks gives way to one that sums it
 *     exactly (fp32, or written once) when that one is modelled at most 1.5x
 *     slower; for fp16 inputs such a plan is compared only with the plans
 *     that do not sum dW in the fp16 output over row chunks (there gradients
 *     scaled by 1/n fall in fp16's subnormal range), when one fits
 *     (hk_fused_linear_cross_entropy_plan reports the choice).
 *   Debugging override (all fused-linear ops, read at every call): the
 *   environment variable HILDA_FL_FORM="<defer|acc|out>,<wt|wmn>,<dt|dmn>"
 *   restricts the plan to that row-chunked form (dW deferred, in an fp32
 *   accumulator or in the output; W^T or W read MN-contiguous; D^T or D read
 *   MN-contiguous), the chunk still from the budget; "vtile,<acc|out>,<cols>"
 *   to the vocabulary-tiled plan with that dX sum and tile width. Calls
 *   without gradients ignore a row-chunked form; a form that does not parse,
 *   or does not apply to the call, fails it with HK_EINVAL. */
size_t hk_fused_linear_cross_entropy_workspace_size(int64_t BT, int64_t H, int64_t V, int64_t chunk,
                                                    int64_t workspace_budget, int dtype, int with_grad,
                                                    const void* hidden, const void* weight);

/* No counterpart in the reference: the plan the call above sizes, for
 * benchmarks and tests. info[8] = rows per chunk, chunks, dW mode (0: every
 * chunk's D^T kept and one dW GEMM after the loop; 1: an fp32 [V,H]
 * accumulator; 2: accumulated in the output, rounded per chunk for 16-bit
 * inputs; 3 and 4: vocabulary tiles, each tile's dW rows written once, dX
 * summed over the tiles in an fp32 buffer (3) or in the output (4); rows per
 * chunk and chunks are then the tile's columns and the tile count), W^T
 * materialised (else W read MN-contiguous), D^T materialised (else D read
 * MN-contiguous), dX split cap, workspace bytes, modelled ns. */
int hk_fused_linear_cross_entropy_plan(int64_t BT, int64_t H, int64_t V, int64_t chunk, int64_t workspace_budget,
                                       int dtype, int with_grad, const void* hidden, const void* weight,
                                       int64_t* info);

/* Replaces fused_linear_cross_entropy_forward (fused_linear_cross_entropy.py:103-171)
 * and its backward scaling (:192-210). hidden [BT,H], weight [V,H] (fp32, bf16
 * or fp16, contiguous, any H and V); targets [BT] int64; rows equal to
 * ignore_index are ignored. loss_rows[r] = CE of row r (scaled by
 * 1/max(n_valid,1) when gradients are computed with reduction mean);
 * loss_out (nullable) = sum, or mean over valid rows. With dhidden/dweight
 * (both or neither): the gradients of the reduced loss at unit upstream
 * gradient, each row's gradient further multiplied by row_scale[r] when
 * row_scale is given (reduction 'none' backward). Logits are produced a chunk
 * of rows at a time on MFMA (fp32 inputs on the fp32 MFMA), for the rows whose
 * target is not ignore_index only (compacted on the device), in the memory
 * plan workspace_budget selects (see the size query above). */
int hk_fused_linear_cross_entropy(float* loss_out, float* loss_rows, void* dhidden, void* dweight, const void* hidden,
                                  const void* weight, const int64_t* targets, const float* row_scale, int64_t BT,
                                  int64_t H, int64_t V, int64_t ignore_index, int reduction, int dtype, int64_t chunk,
                                  int64_t workspace_budget, void* workspace, size_t workspace_bytes,
                                  hk_stream_t stream);

/* ----------------------------------------------------------------------- */
/* Streaming copies (measurement references)                               */
/* ----------------------------------------------------------------------- */
#define HK_COPY_FLAT 0
#define HK_COPY_ROWS 1

/* No counterpart in the reference: a copy of rows * row_bytes bytes (rows of
 * whole 16-byte vectors, 16-byte aligned, no overlap) that a benchmark times
 * beside an HBM-bound op of the same bytes. HK_COPY_FLAT sweeps the buffer
 * with the whole GPU in one contiguous front (the fastest order measured);
 * HK_COPY_ROWS moves one row per CU at a time in the order of the
 * register-resident row kernels (row_bytes <= 384 KiB). */
int hk_stream_copy(void* dst, const void* src, int64_t rows, int64_t row_bytes, int mode, hk_stream_t stream);

/* No counterpart in the reference: an op's byte mix without its arithmetic,
 * timed beside it. n_read source streams and n_write destination streams of
 * `bytes` each (whole 16-byte vectors) start `stride` bytes apart (>= bytes, a
 * multiple of 16) from src and from dst (16-byte aligned, no overlap);
 * destination stream w receives the XOR of the source streams' vectors at the
 * same offset plus w in every 32-bit word. Flat order. 1 <= n_read <= 9,
 * 1 <= n_write <= 8. */
int hk_stream_mix(void* dst, const void* src, int64_t bytes, int64_t stride, int n_read, int n_write,
                  hk_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* HILDA_KERNEL_AMD_H */
