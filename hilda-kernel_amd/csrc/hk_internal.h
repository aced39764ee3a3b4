// Internal (non-ABI) launchers shared between translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hk {

// n_valid[0] = number of targets != ignore_index (all rows when has_ignore == 0)
int count_valid_launch(int* n_valid, const int64_t* targets, int64_t rows, int64_t ignore_index, int has_ignore,
                       hipStream_t st);

// Per-row CrossEntropy over logits rows. With dlogits: loss_rows = (lse - x_t) * s and
// dlogits = (softmax - onehot) * s * row_scale[r] (row_scale nullable), s = 1/max(n_valid,1)
// when scale_by_n_valid, else 1; ignored rows give 0 and a zero row. dlogits may alias logits.
// Without dlogits: loss_rows = lse - x_t (0 if ignored), no scaling.
// rows_lim (nullable): a device-side bound, only rows < *rows_lim - rows_off are processed.
// rowmap/n_live (nullable, with dlogits only; not with rows_lim): the plan of
// ce_plan_launch, whose live rows the grid deals out evenly.
int ce_rows_launch(void* dlogits, float* loss_rows, const void* logits, const int64_t* targets, int64_t rows,
                   int64_t V, int64_t ld_in, int64_t ld_out, int64_t ignore_index, int has_ignore, const int* n_valid,
                   int scale_by_n_valid, const float* row_scale, int dtype, hipStream_t st,
                   const int* rows_lim = nullptr, int64_t rows_off = 0, const int* rowmap = nullptr,
                   const int* n_live = nullptr);

// The CrossEntropy plan (one block): *n_valid = rows whose target is not
// ignored; rowmap[0 .. *n_live) = rows with a gradient (target not ignored and
// in [0, V)), in order. rows < 2^31.
int ce_plan_launch(int* n_valid, int* rowmap, int* n_live, const int64_t* targets, int64_t rows, int64_t V,
                   int64_t ignore_index, int has_ignore, hipStream_t st);

// Stable compaction of the rows whose target is not ignore_index: rowmap[0 .. n)
// the live rows in order, inv[r] their place (-1 for ignored rows), *n_live = n.
int ce_compact_launch(int* rowmap, int* inv, int* n_live, const int64_t* targets, int64_t rows,
                      int64_t ignore_index, hipStream_t st);

// out[0] = sum(v[0:n]) (fp64 accumulation), / max(n_valid, 1) when divide
int sum_rows_launch(float* out, const float* v, int64_t n, const int* n_valid, int divide, hipStream_t st);

// out = scale * sum(v[0..n)), one block.
int scaled_sum_rows_launch(float* out, const float* v, int64_t n, float scale, hipStream_t st);

// FusedLinearJSD row step on rows x cols student logits ls and teacher logits
// lt (row stride ld, dtype of the ABI): loss_rows = JSD(beta) of the
// temperature log-softmaxes / n, n = max(*n_valid, 1) with labels, else n_all;
// with write, ls is overwritten with the student dlogits. Rows labelled
// ignore_index get loss 0 and zero dlogits. rows_lim (nullable): a device-side
// bound, only rows < *rows_lim - rows_off are processed.
int jsd_logits_launch(float* loss_rows, void* ls, const void* lt, const int64_t* labels, int64_t ignore_index,
                      const int* n_valid, int64_t n_all, float beta, float temperature, int64_t rows, int64_t cols,
                      int64_t ld, int write, int dtype, hipStream_t st, const int* rows_lim = nullptr,
                      int64_t rows_off = 0);

// GRPO's per-call inputs (kernels/grpo_loss.py:241-297): ids, old/ref log-probs
// (fp32, nullable) and mask (any HK_ dtype, nullable) with element strides;
// advantages [B] fp32.
struct GrpoInputs {
  const int64_t* ids;
  int64_t ids_sB, ids_sL;
  const float* adv;
  const float* old_logp;
  int64_t old_sB, old_sL;
  const float* ref_logp;
  int64_t ref_sB, ref_sL;
  const void* mask;
  int mask_dt;
  int64_t mask_sB, mask_sL;
  int64_t B, L, V;
  float temperature, beta, eps_lo, eps_hi;
};

// Argument checks shared by the GRPO entry points: HK_OK, or HK_EINVAL with the message set.
int grpo_check(const GrpoInputs& in);

// Bytes of GRPO scratch (16-byte aligned): token records and per-token results for B x L tokens.
size_t grpo_scratch_bytes(int64_t B, int64_t L);

// Token records (id, old/ref, advantage, mask, mask / (len_b * B) / T) into scratch.
int grpo_prep_launch(const GrpoInputs& in, void* scratch, hipStream_t st);

// Rows [row0, row0 + nrows) of the B x (L+1) logits rows, `logits` pointing at
// row row0 (row stride ld, 0: the width): per-token results into scratch and,
// with dlogits (may alias logits), the gradient rows at unit upstream
// gradient. With rowmap (a compaction, see grpo_compact_launch) row q of the
// launch is position rowmap[row0 + q], and only q < *n_live - row0 exist.
// width (0: V): the row elements read, V or more when the columns past V hold
// -inf (their probability and gradient are then exactly 0).
int grpo_rows_launch(void* dlogits, const void* logits, int64_t row0, int64_t nrows, const GrpoInputs& in,
                     void* scratch, int dtype, hipStream_t st, const int* rowmap = nullptr,
                     const int* n_live = nullptr, int64_t width = 0, int64_t ld = 0);

// Stable compaction of the live positions (l < L, mask != 0) of the B x (L+1)
// rows: rowmap, inv and *n_live as for ce_compact_launch.
int grpo_compact_launch(int* rowmap, int* inv, int* n_live, const GrpoInputs& in, hipStream_t st);

// The reductions (loss, kl_mean, clip_ratio) and the per-token rows [B, L].
int grpo_finalize_launch(const GrpoInputs& in, const void* scratch, float* loss_out, float* kl_out, float* clip_out,
                         float* lse_rows, float* loss_rows, float* kl_rows, float* clip_rows, hipStream_t st);

}  // namespace hk
