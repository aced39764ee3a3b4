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
int ce_rows_launch(void* dlogits, float* loss_rows, const void* logits, const int64_t* targets, int64_t rows,
                   int64_t V, int64_t ld_in, int64_t ld_out, int64_t ignore_index, int has_ignore, const int* n_valid,
                   int scale_by_n_valid, const float* row_scale, int dtype, hipStream_t st);

// out[0] = sum(v[0:n]) (fp64 accumulation), / max(n_valid, 1) when divide
int sum_rows_launch(float* out, const float* v, int64_t n, const int* n_valid, int divide, hipStream_t st);

// out = scale * sum(v[0..n)), one block.
int scaled_sum_rows_launch(float* out, const float* v, int64_t n, float scale, hipStream_t st);

// FusedLinearJSD row step on rows x cols student logits ls and teacher logits
// lt (row stride ld, dtype of the ABI): loss_rows = JSD(beta) of the
// temperature log-softmaxes / n, n = max(*n_valid, 1) with labels, else n_all;
// with write, ls is overwritten with the student dlogits. Rows labelled
// ignore_index get loss 0 and zero dlogits.
int jsd_logits_launch(float* loss_rows, void* ls, const void* lt, const int64_t* labels, int64_t ignore_index,
                      const int* n_valid, int64_t n_all, float beta, float temperature, int64_t rows, int64_t cols,
                      int64_t ld, int write, int dtype, hipStream_t st);

}  // namespace hk
