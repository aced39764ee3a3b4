// FusedLinearCrossEntropy, FusedLinearJSD and FusedLinear-GRPO for gfx950:
// lm_head GEMMs on MFMA (bf16/fp16, or fp32 for fp32 inputs) with the loss
// gradient produced chunk by chunk, so the full (BT, V) logits never exist.
//
// Per chunk of C rows (fused_linear_cross_entropy.py:130-161):
//   logits_c = X_c W^T          into the chunk buffer [C, ldl]
//   row step                    the loss and, with gradients, D_c over the logits
//   dX_c     = D_c W            A = D_c [C, V], B = W^T [H, V] or W read MN-contiguous
//   dW      += D_c^T X_c        A = D_c^T [V, C] or D_c read MN-contiguous, B = X_c^T [H, C]
//
// How much memory that takes is a plan (FlPlan), chosen per call from a byte
// budget by a cost model. The forms, from most to least memory:
//   * every chunk's D_c^T kept side by side and dW one GEMM over all rows
//     after the loop (deferred): no dW read-modify-write, a (V, BT) buffer;
//   * dW accumulated across chunks in an fp32 [V, H] buffer;
//   * dW accumulated in the output itself (fp32 inputs: an exact fp32 sum;
//     16-bit inputs: rounded per chunk, as the reference's bf16 addmm does);
// each with W^T (a weight-sized copy) or W read MN-contiguous by the dX GEMM
// (ds_read_b64_tr_b16), and D_c^T (a chunk-sized copy) or D_c read
// MN-contiguous by the dW GEMM. The default budget is what the reference's
// chunk (fused_linear_cross_entropy.py:112-114: chunk logits about the size of
// the hidden states) costs, in the leanest form.
//
// Rows that need no logits (ignored targets or labels, masked GRPO positions)
// are compacted away on the device first; each chunk gathers its live rows,
// and the GEMMs, transposes and row kernels read the live count from device
// memory, so the host never waits.
//
// Any H and V: the chunk buffer's row stride is V rounded up to 64 (its
// columns past V are -inf or zero, see EpiLogits, and zero past the row
// step's width), hidden rows are gathered into rows of H rounded up to 8
// (zero filled), the weight is copied once into such rows when H is not a
// multiple of 8 or it is not 16-byte aligned, and the output epilogues store
// element by element where a row is not 16-byte aligned.
#include "hk_common.h"
#include "hk_internal.h"
#include "gemm_nt.h"
#include "../../include/hilda_kernel_amd.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <type_traits>
#include <vector>

namespace hk {
namespace {

using gemm::f32x4_t;
struct NoPrior {};

// n (<= 4) fp32 values stored at p in T: one 8- (16-bit) or 16-byte (fp32)
// store when n == 4 and vec (the address is aligned for it), else element by element.
template <typename T>
__device__ __forceinline__ void store4(T* p, const float* v, int n, bool vec) {
  if (n == 4 && vec) {
    if constexpr (sizeof(T) == 4) *reinterpret_cast<f32x4_t*>(p) = f32x4_t{v[0], v[1], v[2], v[3]};
    else *reinterpret_cast<u32x2*>(p) = u32x2{gemm::pack2<T>(v[0], v[1]), gemm::pack2<T>(v[2], v[3])};
  } else {
    for (int e = 0; e < n; ++e) p[e] = from_f32<T>(v[e]);
  }
}

// n (<= 4) values of T at p widened to fp32 (zeros past n); one load when n == 4 and vec.
template <typename T>
__device__ __forceinline__ f32x4_t load4(const T* p, int n, bool vec) {
  f32x4_t x = {0.f, 0.f, 0.f, 0.f};
  if (n == 4 && vec) {
    if constexpr (sizeof(T) == 4) {
      x = *reinterpret_cast<const f32x4_t*>(p);
    } else {
      struct alignas(8) Q { T v[4]; };
      const Q q = *reinterpret_cast<const Q*>(p);
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = to_f32<T>(q.v[e]);
    }
  } else {
    for (int e = 0; e < n; ++e) x[e] = to_f32<T>(p[e]);
  }
  return x;
}

// The logits GEMM's epilogue: C (T) = acc in 16-byte chunks (ldc a multiple of
// 8, C 16-byte aligned). The chunk that straddles column N is completed with
// `pad` past N: -inf for the CrossEntropy and GRPO row steps, which then read
// the row to the next multiple of 16 bytes (a -inf logit has probability 0,
// so the loss is unchanged and its gradient entry is 0), 0 for the JSD step.
template <typename T>
struct EpiLogits {
  using Stage = T;
  using Prior = NoPrior;
  static constexpr bool kReads = false;
  T* C;
  int64_t ldc;
  float pad;
  __device__ __forceinline__ Prior load(int, int, int) const { return {}; }
  __device__ __forceinline__ void store(int row, int col, const T* v, int n, const Prior&) const {
    constexpr int E = 16 / (int)sizeof(T);
    T* p = C + (int64_t)row * ldc + col;
    if (n == E) {
      *reinterpret_cast<u32x4*>(p) = *reinterpret_cast<const u32x4*>(v);
    } else {
      const T fill = from_f32<T>(pad);
      for (int e = 0; e < E; ++e) p[e] = e < n ? v[e] : fill;
    }
  }
};

// The dX GEMM's epilogue (M = chunk rows, N = the padded hidden size). GEMM row
// r goes to row rows[r] of C (rows nullable: row r); only columns < cols are
// stored. Unsplit (the GEMM's split count is 1) it stores the tile; split, split
// s stores fp32 partial sums at part + (s * m + row) * ld (m the GEMM's bounded
// row count, ld its N) and splitk_sum_kernel adds them up.
template <typename T>
struct EpiDx {
  using Stage = float;
  using Prior = NoPrior;
  static constexpr bool kReads = false;
  T* C;
  int64_t ldc;
  const int* rows;
  float* part;
  int64_t ld;   // a multiple of 4
  int cols;
  bool vec;     // C rows 8-byte (16-bit) / 16-byte (fp32) aligned at every 4th column
  int split = 0, nsplit = 1, m = 0;
  __device__ __forceinline__ void set_split(int s, int ns, int bounded_m) {
    split = s;
    nsplit = ns;
    m = bounded_m;
  }
  __device__ __forceinline__ Prior load(int, int, int) const { return {}; }
  __device__ __forceinline__ void store(int row, int col, const float* v, int n, const Prior&) const {
    if (nsplit == 1) {
      n = min(n, cols - col);
      if (n > 0) store4<T>(C + (int64_t)(rows ? rows[row] : row) * ldc + col, v, n, vec);
      return;
    }
    float* p = part + ((int64_t)split * m + row) * ld + col;
    if (n == 4) {
      *reinterpret_cast<f32x4_t*>(p) = f32x4_t{v[0], v[1], v[2], v[3]};
    } else {
      for (int e = 0; e < n; ++e) p[e] = v[e];
    }
  }
};

// The dW GEMM's epilogue (M = vocabulary rows, N = the padded hidden size);
// rows < rows_lim and columns < cols_lim are kept. MODE:
//   0: out = v                       (one chunk, or the deferred GEMM)
//   1: out = out + v                 (accumulation in the output, rounded per chunk)
//   2: acc = v,  3: acc += v         (the fp32 accumulator, chunks before the last)
//   4: out = acc + v                 (the last chunk)
template <typename T, int MODE>
struct EpiDw {
  using Stage = float;
  using Prior = f32x4_t;
  static constexpr bool kReads = MODE == 1 || MODE == 3 || MODE == 4;
  T* out;
  int64_t ldo;
  float* acc;
  int64_t lda;  // a multiple of 4
  int rows_lim, cols_lim;
  bool vec;     // out rows aligned for 4-element stores
  const int* inv_n = nullptr;  // nullable: the values are multiplied by 1 / max(*inv_n, 1) first
  __device__ __forceinline__ Prior load(int row, int col, int n) const {
    if (row >= rows_lim || col >= cols_lim) return Prior{0.f, 0.f, 0.f, 0.f};
    n = min(n, cols_lim - col);
    if constexpr (MODE == 1) return load4<T>(out + (int64_t)row * ldo + col, n, vec);
    const float* p = acc + (int64_t)row * lda + col;
    if (n == 4) return *reinterpret_cast<const f32x4_t*>(p);
    Prior x = {0.f, 0.f, 0.f, 0.f};
    for (int e = 0; e < n; ++e) x[e] = p[e];
    return x;
  }
  __device__ __forceinline__ void store(int row, int col, const float* v, int n, const Prior& x) const {
    if (row >= rows_lim || col >= cols_lim) return;
    n = min(n, cols_lim - col);
    const float f = inv_n ? 1.f / (float)max(*inv_n, 1) : 1.f;
    float r[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = kReads ? x[e] + v[e] * f : v[e] * f;
    if constexpr (MODE == 2 || MODE == 3) {
      float* p = acc + (int64_t)row * lda + col;
      if (n == 4) {
        *reinterpret_cast<f32x4_t*>(p) = f32x4_t{r[0], r[1], r[2], r[3]};
      } else {
        for (int e = 0; e < n; ++e) p[e] = r[e];
      }
    } else {
      store4<T>(out + (int64_t)row * ldo + col, r, n, vec);
    }
  }
};

// Rows [0, rows) of out (row stride ldo, width wo; 16-byte aligned rows when
// VEC): row i is input row src(i) = rowmap[row0 + i] (rowmap nullable: row0 + i)
// for i below the live rows (*n_live - row0, or live_rows - row0 without
// n_live), its w elements followed by zeros up to wo; the rows after are zero.
// VEC: the input rows are 16-byte aligned with w a multiple of 16 bytes.
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void gather_rows_kernel(T* __restrict__ out, int64_t ldo, int64_t wo,
                                                          const T* __restrict__ in, int64_t ldi, int64_t w,
                                                          const int* __restrict__ rowmap,
                                                          const int* __restrict__ n_live, int64_t live_rows,
                                                          int64_t row0, int64_t rows) {
  constexpr int E = 16 / (int)sizeof(T);
  const int64_t lv = n_live ? (int64_t)*n_live : live_rows;
  const int64_t live = std::max<int64_t>(0, std::min<int64_t>(rows, lv - row0));
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    T* o = out + r * ldo;
    int64_t c0 = 0;
    if (r < live) {
      const T* s = in + (int64_t)(rowmap ? rowmap[row0 + r] : row0 + r) * ldi;
      if constexpr (VEC) {
        for (int64_t j = threadIdx.x; j < w / E; j += 256)
          reinterpret_cast<u32x4*>(o)[j] = reinterpret_cast<const u32x4*>(s)[j];
      } else {
        for (int64_t j = threadIdx.x; j < w; j += 256) o[j] = s[j];
      }
      c0 = w;
    }
    // zeros from c0 (a row start or w) to wo: elements up to a 16-byte boundary, then 16-byte stores
    const int64_t cv = std::min<int64_t>(wo, (c0 + E - 1) / E * E);
    for (int64_t j = c0 + threadIdx.x; j < cv; j += 256) o[j] = from_f32<T>(0.f);
    for (int64_t j = cv / E + threadIdx.x; j < wo / E; j += 256) reinterpret_cast<u32x4*>(o)[j] = u32x4{0, 0, 0, 0};
  }
}

// Per-row CE inputs of the compacted rows: targets and the optional row scale.
__global__ __launch_bounds__(256) void gather_ce_kernel(int64_t* __restrict__ t_out, float* __restrict__ s_out,
                                                        const int64_t* __restrict__ t_in,
                                                        const float* __restrict__ s_in, const int* __restrict__ rowmap,
                                                        const int* __restrict__ n_live) {
  const int64_t n = *n_live;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int r = rowmap[i];
    t_out[i] = t_in[r];
    if (s_in) s_out[i] = s_in[r];
  }
}

// Columns [c0, c1) of `rows` rows (row stride ld) set to zero.
template <typename T>
__global__ __launch_bounds__(256) void zero_cols_kernel(T* __restrict__ p, int64_t ld, int64_t c0, int64_t c1,
                                                        int64_t rows) {
  const int64_t w = c1 - c0, n = rows * w;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / w;
    p[r * ld + c0 + (i - r * w)] = from_f32<T>(0.f);
  }
}

// Rows of the original order after a compacted pass: dead rows (inv[r] < 0)
// get a zero dX row of H elements (when dX) and loss 0; live rows take their
// loss from the compacted losses (when loss_rows). VEC: dX rows are whole
// 16-byte aligned vectors.
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void finish_rows_kernel(T* __restrict__ dX, int64_t H,
                                                          float* __restrict__ loss_rows,
                                                          const float* __restrict__ loss_c,
                                                          const int* __restrict__ inv, int64_t rows) {
  constexpr int E = 16 / (int)sizeof(T);
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const int k = inv[r];
    if (loss_rows && threadIdx.x == 0) loss_rows[r] = k >= 0 ? loss_c[k] : 0.f;
    if (dX && k < 0) {
      if constexpr (VEC) {
        for (int64_t w = threadIdx.x; w < H / E; w += 256) reinterpret_cast<u32x4*>(dX + r * H)[w] = u32x4{0, 0, 0, 0};
      } else {
        for (int64_t w = threadIdx.x; w < H; w += 256) dX[r * H + w] = from_f32<T>(0.f);
      }
    }
  }
}

// out[c, r] = in[r, c] for a rows x cols matrix of a 16-bit type (row strides
// ld_in, ld_out, both multiples of 8; cols a multiple of 8); output columns r
// in [rows, rows_pad) are written as zeros (rows_pad a multiple of 8).
// 16-byte global loads and stores, the tile staged in LDS (layout below).
// With lim (a compacted input whose first *lim - lim_off rows are live), rows
// past that are read as zeros and zeros are written up to the next multiple
// of 64 of the bound, both relative to lim_off and absolute: what a GEMM
// whose K is cut by the same bound reads (at least 64 columns).
template <typename T>
__global__ __launch_bounds__(512) void transpose_kernel(T* __restrict__ out, const T* __restrict__ in, int64_t rows,
                                                        int64_t rows_pad, int64_t cols, int64_t ld_in,
                                                        int64_t ld_out, const int* __restrict__ lim,
                                                        int64_t lim_off) {
  static_assert(sizeof(T) == 2, "16-bit elements");
  // 128 x 128 tiles: 256-byte runs on both sides (a 64 x 64 tile's 128-byte
  // input runs from 256 KB rows ran at 2.3 TB/s). Lane (q, k) of unit i loads
  // input rows 2q and 2q+1 at 16-byte column chunk k; each column's pair of
  // elements becomes one 32-bit word (v_perm), stored column-major: word
  // (column j, pair q) at j*64 + (((q >> 2) ^ (j >> 3)) << 2 | (q & 3)). The XOR
  // of 4-word groups keeps the word writes (16 chunks of a wave, 16 groups) and
  // the 16-byte reads (16 lanes of one column, 16 groups) free of bank conflicts.
  __shared__ __attribute__((aligned(16))) uint32_t tile[128 * 64];
  const int t = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.y * 128, c0 = (int64_t)blockIdx.x * 128;
  if (lim) {
    const int64_t n = *lim, v = n - lim_off;
    rows = std::max<int64_t>(0, std::min<int64_t>(rows, v));
    const int64_t z = std::max<int64_t>(64, std::max<int64_t>((v + 63) / 64 * 64, (n + 63) / 64 * 64 - lim_off));
    rows_pad = std::min<int64_t>(rows_pad, z);
    if (r0 >= rows_pad) return;  // uniform
  }
  const int k = t & 15;
  u32x4 va[2], vb[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int q = (t >> 4) + 32 * i;
    const int64_t r = r0 + 2 * q, c = c0 + 8 * k;
    va[i] = u32x4{0u, 0u, 0u, 0u};
    vb[i] = u32x4{0u, 0u, 0u, 0u};
    if (c < cols) {
      if (r < rows) va[i] = *reinterpret_cast<const u32x4*>(in + r * ld_in + c);
      if (r + 1 < rows) vb[i] = *reinterpret_cast<const u32x4*>(in + (r + 1) * ld_in + c);
    }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int q = (t >> 4) + 32 * i;
    const int slot = (((q >> 2) ^ k) << 2) | (q & 3);  // j >> 3 == k for the 8 columns of chunk k
    const uint32_t a[4] = {va[i].x, va[i].y, va[i].z, va[i].w};
    const uint32_t b[4] = {vb[i].x, vb[i].y, vb[i].z, vb[i].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      // low half: row 2q's element of column 8k + e, high half: row 2q+1's
      const uint32_t w = __builtin_amdgcn_perm(b[e >> 1], a[e >> 1], (e & 1) ? 0x07060302u : 0x05040100u);
      tile[(8 * k + e) * 64 + slot] = w;
    }
  }
  __syncthreads();
  const int m = t & 15;  // output chunk: rows 8m .. 8m+7 of the tile, words 4m .. 4m+3
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int j = (t >> 4) + 32 * i;
    const int64_t c = c0 + j, r = r0 + 8 * m;
    const u32x4 v = *reinterpret_cast<const u32x4*>(tile + j * 64 + ((m ^ (j >> 3)) << 2));
    if (c < cols && r < rows_pad) *reinterpret_cast<u32x4*>(out + c * ld_out + r) = v;
  }
}

// The fp32 form of transpose_kernel (same arguments and zero padding): 64x64
// tiles of 16-byte (4-element) loads and stores, staged in LDS with a pitch of
// 65 floats so the column reads of a wave fall in distinct banks.
__global__ __launch_bounds__(256) void transpose32_kernel(float* __restrict__ out, const float* __restrict__ in,
                                                          int64_t rows, int64_t rows_pad, int64_t cols, int64_t ld_in,
                                                          int64_t ld_out, const int* __restrict__ lim,
                                                          int64_t lim_off) {
  constexpr int P = 65;
  __shared__ float tile[64 * P];
  const int t = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  if (lim) {
    const int64_t n = *lim, v = n - lim_off;
    rows = std::max<int64_t>(0, std::min<int64_t>(rows, v));
    const int64_t z = std::max<int64_t>(64, std::max<int64_t>((v + 63) / 64 * 64, (n + 63) / 64 * 64 - lim_off));
    rows_pad = std::min<int64_t>(rows_pad, z);
    if (r0 >= rows_pad) return;  // uniform
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int rr = t / 16 + 16 * k, cc = (t % 16) * 4;
    const int64_t r = r0 + rr, c = c0 + cc;
    f32x4_t v = {0.f, 0.f, 0.f, 0.f};
    if (r < rows && c < cols) v = *reinterpret_cast<const f32x4_t*>(in + r * ld_in + c);
#pragma unroll
    for (int e = 0; e < 4; ++e) tile[rr * P + cc + e] = v[e];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int oc = t / 16 + 16 * k, oq = (t % 16) * 4;
    const int64_t c = c0 + oc, r = r0 + oq;
    if (c < cols && r < rows_pad)
      *reinterpret_cast<f32x4_t*>(out + c * ld_out + r) =
          f32x4_t{tile[oq * P + oc], tile[(oq + 1) * P + oc], tile[(oq + 2) * P + oc], tile[(oq + 3) * P + oc]};
  }
}

// C[rows ? rows[r] : r, 0:cols) = sum over the splits of the partials (rounded
// once to T), 4 columns a thread, for r below the device-bounded M. The split
// count is the GEMM's own (auto_splits of its bounded tiles); unsplit, the
// GEMM stored C itself and this returns at once. Partials have row stride N.
template <typename T>
__global__ __launch_bounds__(256) void splitk_sum_kernel(T* __restrict__ C, int64_t ldc, const int* __restrict__ rows,
                                                         const float* __restrict__ part, int M, int N, int KT,
                                                         int max_s, const int* lim, int lim_off, int cols, int vec) {
  if (lim) M = min(M, max(0, *lim - lim_off));
  const int S = gemm::auto_splits(((M + 255) / 256) * ((N + 255) / 256), KT, max_s);
  if (S == 1) return;
  const int n4 = (cols + 3) / 4;
  const int64_t total = (int64_t)M * n4, stride = (int64_t)M * N;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int r = (int)(i / n4), c = (int)(i - (int64_t)r * n4) * 4;
    const float* p = part + (int64_t)r * N + c;
    f32x4_t a = *reinterpret_cast<const f32x4_t*>(p);
    for (int s = 1; s < S; ++s) a += *reinterpret_cast<const f32x4_t*>(p + s * stride);
    const float v[4] = {a[0], a[1], a[2], a[3]};
    store4<T>(C + (int64_t)(rows ? rows[r] : r) * ldc + c, v, min(4, cols - c), vec != 0);
  }
}


// ---------------------------------------------------------------------------
// Vocabulary-tiled CrossEntropy row passes. The logits tile holds every row's
// columns [v0, v0 + w) (row stride ld); logits are scaled by log2(e) into
// base 2. VtRow is a row's state across the tiles: the running maximum m,
// the sum sx of 2^(z - m) over the columns seen that are not the target, and
// the target logit zt (-inf until its tile). After vt_finalize_kernel: m holds
// the base-2 log-sum-exp and sx 1 - p_target (formed from the other columns'
// mass, so a peaked row keeps its small target gradient exact).
// ---------------------------------------------------------------------------
struct VtRow {
  float m, sx, zt, pad;
};

constexpr int kVtLanes = 256;  // four waves a block, one row a wave at a time

// One wave a row (grid-stride over the rows): per lane an online maximum and
// sum of 2^(z - m) over the row's 16-byte vectors (the target column left
// out), then the wave's (max, sum) by DPP reductions; merged into the row state.
template <typename T>
__global__ __launch_bounds__(kVtLanes) void vt_lse_kernel(const T* __restrict__ L, int64_t ld, int64_t w, int64_t v0,
                                                        const int64_t* __restrict__ targets, int64_t ignore_index,
                                                        VtRow* __restrict__ state, int64_t rows, int first) {
  constexpr int E = 16 / (int)sizeof(T);
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t nw = (int64_t)gridDim.x * (kVtLanes / kWave);
  const float ninf = -__builtin_huge_valf();
  for (int64_t r = (int64_t)blockIdx.x * (kVtLanes / kWave) + threadIdx.x / kWave; r < rows; r += nw) {
    const int64_t t = targets[r];
    if (t == ignore_index) continue;  // uniform in the wave
    const int64_t tl = t - v0;         // the target's column in this tile, if it is here
    const T* row = L + r * ld;
    float m = ninf, sx = 0.f, zt = ninf;
    for (int64_t j0 = (int64_t)lane * E; j0 < w; j0 += kWave * E) {
      float x[E];
      if (j0 + E <= w) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(row + j0);
        const T* e = reinterpret_cast<const T*>(&v);
#pragma unroll
        for (int i = 0; i < E; ++i) x[i] = to_f32<T>(e[i]) * kLog2e;
      } else {
#pragma unroll
        for (int i = 0; i < E; ++i) x[i] = j0 + i < w ? to_f32<T>(row[j0 + i]) * kLog2e : ninf;
      }
      float cm = m;
#pragma unroll
      for (int i = 0; i < E; ++i) cm = fmaxf(cm, x[i]);
      float cs = 0.f;
#pragma unroll
      for (int i = 0; i < E; ++i) {
        if (j0 + i == tl) zt = x[i];
        else cs += exp2_fast(x[i] - cm);
      }
      sx = (sx > 0.f ? sx * exp2_fast(m - cm) : 0.f) + cs;
      m = cm;
    }
    const float M = wave_max(m);
    sx = wave_sum(sx > 0.f ? sx * exp2_fast(m - M) : 0.f);
    zt = wave_max(zt);
    if (lane == 0) {
      VtRow q = first ? VtRow{ninf, 0.f, ninf, 0.f} : state[r];
      const float Mn = fmaxf(q.m, M);
      q.sx = (q.sx > 0.f ? q.sx * exp2_fast(q.m - Mn) : 0.f) + (sx > 0.f ? sx * exp2_fast(M - Mn) : 0.f);
      q.m = Mn;
      if (tl >= 0 && tl < w) q.zt = zt;
      state[r] = q;
    }
  }
}

// Per row after the last tile: loss (times s when scale), and the state turned
// into (base-2 log-sum-exp, 1 - p_target).
__global__ __launch_bounds__(256) void vt_finalize_kernel(VtRow* __restrict__ state, float* __restrict__ loss_rows,
                                                          const int64_t* __restrict__ targets, int64_t ignore_index,
                                                          const int* __restrict__ n_valid, int scale, int64_t rows) {
  const float s = scale ? 1.f / (float)max(*n_valid, 1) : 1.f;
  for (int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x; r < rows; r += (int64_t)gridDim.x * 256) {
    if (targets[r] == ignore_index) {
      loss_rows[r] = 0.f;
      continue;
    }
    VtRow q = state[r];
    const float et = exp2_fast(q.zt - q.m);
    const float tot = q.sx + et;
    const float lse2 = q.m + log2_fast(tot);
    loss_rows[r] = (lse2 - q.zt) * kLn2 * s;
    state[r] = VtRow{lse2, q.sx / tot, q.zt, 0.f};
  }
}

// The gradient tile in place, one wave a row: D = (p - onehot) * g with
// g = s * row_scale[r] (s = 1 / max(n_valid, 1) when scale), the target entry
// -(1 - p_t) * g; columns [w, wz) and ignored rows are zero.
template <typename T>
__global__ __launch_bounds__(kVtLanes) void vt_grad_kernel(T* __restrict__ L, int64_t ld, int64_t w, int64_t wz,
                                                         int64_t v0, const int64_t* __restrict__ targets,
                                                         int64_t ignore_index, const VtRow* __restrict__ state,
                                                         const int* __restrict__ n_valid, int scale,
                                                         const float* __restrict__ row_scale, int64_t rows) {
  constexpr int E = 16 / (int)sizeof(T);
  const float s = scale ? 1.f / (float)max(*n_valid, 1) : 1.f;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t nw = (int64_t)gridDim.x * (kVtLanes / kWave);
  for (int64_t r = (int64_t)blockIdx.x * (kVtLanes / kWave) + threadIdx.x / kWave; r < rows; r += nw) {
    T* row = L + r * ld;
    const int64_t t = targets[r];
    const bool dead = t == ignore_index;
    const VtRow q = dead ? VtRow{0.f, 0.f, 0.f, 0.f} : state[r];
    const float g = dead ? 0.f : s * (row_scale ? row_scale[r] : 1.f);
    const int64_t tl = t - v0;
    for (int64_t j0 = (int64_t)lane * E; j0 < wz; j0 += kWave * E) {
      T out[E];
      if (j0 + E <= w && !dead) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(row + j0);
        const T* e = reinterpret_cast<const T*>(&v);
#pragma unroll
        for (int i = 0; i < E; ++i) {
          const float d = j0 + i == tl ? -q.sx * g : exp2_fast(to_f32<T>(e[i]) * kLog2e - q.m) * g;
          out[i] = from_f32<T>(d);
        }
      } else {
#pragma unroll
        for (int i = 0; i < E; ++i) {
          const int64_t j = j0 + i;
          float d = 0.f;
          if (!dead && j < w) d = j == tl ? -q.sx * g : exp2_fast(to_f32<T>(row[j]) * kLog2e - q.m) * g;
          out[i] = from_f32<T>(d);
        }
      }
      if (j0 + E <= wz) {
        *reinterpret_cast<u32x4*>(row + j0) = *reinterpret_cast<const u32x4*>(out);
      } else {
        for (int i = 0; i < E && j0 + i < wz; ++i) row[j0 + i] = out[i];
      }
    }
  }
}

// The tile's target entries set to zero (after the tile's dW GEMM has read them):
// dX is then summed across the tiles from softmax terms alone, of like size, and
// vt_target_dx_kernel adds each row's target term once at the end.
template <typename T>
__global__ __launch_bounds__(256) void vt_drop_targets_kernel(T* __restrict__ L, int64_t ld, int64_t w, int64_t v0,
                                                              const int64_t* __restrict__ targets,
                                                              int64_t ignore_index, int64_t rows) {
  for (int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x; r < rows; r += (int64_t)gridDim.x * 256) {
    const int64_t t = targets[r];
    if (t != ignore_index && t >= v0 && t < v0 + w) L[r * ld + (t - v0)] = from_f32<T>(0.f);
  }
}

// dX[r] = s * (dX[r] - (1 - p_target) * row_scale[r] * W[target]) for every live row, in fp32, rounded once
// (one block a row): dX was summed in the output without s (s = 1 / max(n_valid, 1) when scale), which keeps
// fp16 sums out of the subnormal range (unscaled, they stay below twice the largest |W|).
template <typename T>
__global__ __launch_bounds__(256) void vt_target_dx_kernel(T* __restrict__ dX, int64_t H, const T* __restrict__ W,
                                                           int64_t ldw, const int64_t* __restrict__ targets,
                                                           int64_t ignore_index, int64_t V,
                                                           const VtRow* __restrict__ state,
                                                           const int* __restrict__ n_valid, int scale,
                                                           const float* __restrict__ row_scale, int64_t rows) {
  const float s = scale ? 1.f / (float)max(*n_valid, 1) : 1.f;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const int64_t t = targets[r];
    if (t == ignore_index || t < 0 || t >= V) continue;
    const float c = -state[r].sx * (row_scale ? row_scale[r] : 1.f);
    const T* wr = W + t * ldw;
    T* o = dX + r * H;
    for (int64_t j = threadIdx.x; j < H; j += 256)
      o[j] = from_f32<T>(s * (to_f32<T>(o[j]) + c * to_f32<T>(wr[j])));
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

template <typename T, class Epi>
int launch_gemm(const T* A, const T* B, int M, int N, int K, int64_t lda, int64_t ldb, Epi epi, hipStream_t st,
                const int* lim = nullptr, int lim_off = 0, bool lim_k = false, int ksplit = 1, int kb = 0) {
  return gemm::launch<T>(A, B, M, N, K, lda, ldb, epi, st, lim, lim_off, lim_k, ksplit, 0, kb);
}

// An MN-contiguous operand (16-bit inputs only: the plans never take one for fp32).
template <typename T, bool AMN, bool BMN, class Epi>
int launch_gemm_mn(const T* A, const T* B, int M, int N, int K, int64_t lda, int64_t ldb, Epi epi, hipStream_t st,
                   const int* lim = nullptr, int lim_off = 0, bool lim_k = false, int ksplit = 1, int kb = 0,
                   int ka = 0) {
  if constexpr (sizeof(T) == 2) {
    return gemm::launch<T, gemm::CfgFor<T>, AMN, BMN>(A, B, M, N, K, lda, ldb, epi, st, lim, lim_off, lim_k, ksplit,
                                                      ka, kb);
  } else {
    set_error("internal: an MN-contiguous fp32 operand");
    return HK_EINVAL;
  }
}

template <typename T>
int launch_transpose(T* out, const T* in, int64_t rows, int64_t rows_pad, int64_t cols, int64_t ld_in,
                     int64_t ld_out, hipStream_t st, const int* lim = nullptr, int64_t lim_off = 0) {
  if (rows_pad == 0 || cols == 0) return HK_OK;
  HK_REQUIRE(cols % 8 == 0 && rows_pad % 8 == 0 && ld_in % 8 == 0 && ld_out % 8 == 0 && aligned_to(in, 16) &&
                 aligned_to(out, 16),
             "transpose: 16-byte rows and chunks expected");
  if constexpr (sizeof(T) == 4) {
    const dim3 grid((unsigned)cdiv(cols, 64), (unsigned)cdiv(rows_pad, 64));
    hipLaunchKernelGGL(transpose32_kernel, grid, dim3(256), 0, st, out, in, rows, rows_pad, cols, ld_in, ld_out, lim,
                       lim_off);
    return check_launch("transpose32_kernel");
  } else {
    const dim3 grid((unsigned)cdiv(cols, 128), (unsigned)cdiv(rows_pad, 128));
    hipLaunchKernelGGL((transpose_kernel<T>), grid, dim3(512), 0, st, out, in, rows, rows_pad, cols, ld_in, ld_out,
                       lim, lim_off);
    return check_launch("transpose_kernel");
  }
}

int64_t pad8(int64_t x) { return (x + 7) & ~(int64_t)7; }
int64_t pad64(int64_t x) { return (x + 63) & ~(int64_t)63; }
size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Input dtypes of the fused-linear ops: bf16 and fp16 (16-bit MFMA) and fp32 (fp32 MFMA).
bool fl_dtype_ok(int dt) { return dt == HK_BF16 || dt == HK_F16 || dt == HK_F32; }
int fl_esize(int dt) { return dt == HK_F32 ? 4 : 2; }

// f(Tag<T>) for the dtype (checked by fl_dtype_ok)
template <typename T> struct Tag { using type = T; };
template <typename F>
int fl_dispatch(int dt, F&& f) {
  if (dt == HK_BF16) return f(Tag<__bf16>{});
  if (dt == HK_F16) return f(Tag<_Float16>{});
  return f(Tag<float>{});
}

// Leading dimension of the transposed GEMM operands (X^T, D^T): 128 bytes past
// the K extent, so the rows of a tile's panel do not all start at the same
// large power-of-two offset.
int64_t ld_t(int64_t k) { return pad8(k) + 64; }

// Rows of out from rows of in (see gather_rows_kernel).
template <typename T>
int gather_rows(T* out, int64_t ldo, int64_t wo, const T* in, int64_t ldi, int64_t w, const int* rowmap,
                const int* n_live, int64_t live_rows, int64_t row0, int64_t rows, hipStream_t st) {
  if (rows <= 0) return HK_OK;
  constexpr int E = 16 / (int)sizeof(T);
  const dim3 grid((unsigned)std::min<int64_t>(rows, 8192));
  if (w % E == 0 && ldi % E == 0 && aligned_to(in, 16))
    hipLaunchKernelGGL((gather_rows_kernel<T, true>), grid, dim3(256), 0, st, out, ldo, wo, in, ldi, w, rowmap, n_live,
                       live_rows, row0, rows);
  else
    hipLaunchKernelGGL((gather_rows_kernel<T, false>), grid, dim3(256), 0, st, out, ldo, wo, in, ldi, w, rowmap,
                       n_live, live_rows, row0, rows);
  return check_launch("gather_rows_kernel");
}

template <typename T>
int zero_cols(T* p, int64_t ld, int64_t c0, int64_t c1, int64_t rows, hipStream_t st) {
  if (c1 <= c0 || rows <= 0) return HK_OK;
  const int64_t n = (c1 - c0) * rows;
  hipLaunchKernelGGL((zero_cols_kernel<T>), dim3((unsigned)std::min<int64_t>(cdiv(n, 256), 4096)), dim3(256), 0, st, p,
                     ld, c0, c1, rows);
  return check_launch("zero_cols_kernel");
}

// Zero dX rows of the dead rows and, with loss_rows, the losses back in the original order.
template <typename T>
int finish_rows(T* dX, float* loss_rows, const float* loss_c, const int* inv, int64_t BT, int64_t H,
                hipStream_t st) {
  if (BT == 0 || (!dX && !loss_rows)) return HK_OK;
  constexpr int E = 16 / (int)sizeof(T);
  const dim3 grid((unsigned)std::min<int64_t>(BT, 4096));
  if (!dX || (H % E == 0 && aligned_to(dX, 16)))
    hipLaunchKernelGGL((finish_rows_kernel<T, true>), grid, dim3(256), 0, st, dX, H, loss_rows, loss_c, inv, BT);
  else
    hipLaunchKernelGGL((finish_rows_kernel<T, false>), grid, dim3(256), 0, st, dX, H, loss_rows, loss_c, inv, BT);
  return check_launch("finish_rows_kernel");
}

// ---------------------------------------------------------------------------
// The plan
// ---------------------------------------------------------------------------

enum DwMode { kDwDefer = 0, kDwAcc = 1, kDwOut = 2 };

// What a fused-linear op asks of the chunk engine.
struct FlShape {
  int64_t BT, H, V;
  int es;
  bool grad;
  bool compact;        // live rows compacted through a row map (CE, GRPO, JSD with labels)
  bool x_ok;           // hidden rows readable in place: 16-byte aligned, H a multiple of 8
  bool w_ok;           // weight rows readable in place: the same for W
  bool ce;             // room for the compacted CrossEntropy targets, row scales and losses
  size_t fixed_extra;  // the row step's own scratch, bytes
  size_t row_extra;    // and per chunk row
  int64_t chunk_cap;   // rows per chunk at most (<= 0: no cap below 8192)
  bool vt_ok = false;  // the vocabulary-tiled plan applies (CrossEntropy on 16-bit inputs)
  bool f16 = false;    // fp16 inputs (see fl_plan)
  size_t default_floor = 0;  // the default budget is at least this many bytes
};

struct FlPlan {
  int64_t C = 0, nch = 0;
  int64_t Hp = 0;   // H rounded up to 8: the hidden rows' width in the GEMMs
  int64_t V8 = 0;   // V rounded up to 8: rows of D^T, M of an MN-contiguous dW GEMM
  int64_t Vr = 0;   // the CE / GRPO row steps' width: V rounded up to a 16-byte multiple
  int64_t ldl = 0;  // chunk buffer row stride: V rounded up to 64 (the dX GEMM's K)
  bool gather = false, wpad = false, wt = false, dt = false;
  int dw = kDwOut;
  int ksplit = 1;   // most K splits of the dX GEMM
  size_t nvalid = 0, nlive = 0, rowmap = 0, inv = 0, tc = 0, sc = 0, lc = 0;
  size_t xg = 0, xt = 0, lg = 0, wtp = 0, wp = 0, dtp = 0, acc = 0, part = 0, extra = 0, total = 0;
  double cost = 0;
  // the vocabulary-tiled plan: tiles of Vt vocabulary columns over every row
  // (the logits tile [BT, Vt] at lg), per-row state at vst, the hidden rows
  // padded at xg when they cannot be read in place; dw = kDwAcc sums dX in an
  // fp32 [BT, Hp] buffer at acc, kDwOut in the output
  bool vtile = false;
  int64_t Vt = 0, ntiles = 0;
  size_t vst = 0;
};

int dx_bk(int es) { return es == 4 ? gemm::F32Cfg::BK : gemm::DefaultCfg::BK; }

// fp32 partial-sum bytes the dX GEMM of a chunk of up to C rows can need with at
// most smax splits: the largest splits x rows over the row counts it may be cut to.
size_t dx_part_bytes(int64_t C, int64_t Hp, int64_t ldl, int bk, int smax) {
  if (smax <= 1) return 0;
  size_t best = 0;
  const int64_t ntn = cdiv(Hp, 256), kt = ldl / bk;
  for (int64_t mt = 1; mt <= cdiv(C, 256); ++mt) {
    const int s = gemm::auto_splits((int)(mt * ntn), (int)kt, smax);
    if (s > 1) best = std::max(best, (size_t)s * (size_t)std::min<int64_t>(C, mt * 256) * Hp * 4);
  }
  return best;
}

// The workspace layout of one candidate (C rows a chunk, the forms, the split cap).
FlPlan fl_layout(const FlShape& s, int64_t C, bool wt, bool dt, int dw, int smax) {
  FlPlan p;
  p.C = C;
  p.nch = s.BT > 0 ? cdiv(s.BT, C) : 0;
  p.Hp = pad8(s.H);
  p.V8 = pad8(s.V);
  p.Vr = (s.V + 16 / s.es - 1) / (16 / s.es) * (16 / s.es);
  p.ldl = pad64(s.V);
  p.gather = s.compact || !s.x_ok;
  p.wpad = !s.w_ok;
  p.wt = s.grad && wt;
  p.dt = s.grad && dt;
  p.dw = dw;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += align256(bytes);
    return o;
  };
  const size_t es = (size_t)s.es, bt = (size_t)std::max<int64_t>(s.BT, 1);
  p.nvalid = take(256);
  p.nlive = take(256);
  if (s.compact) {
    p.rowmap = take(bt * 4);
    p.inv = take(bt * 4);
  }
  if (s.ce) {
    p.tc = take(bt * 8);
    p.sc = take(bt * 4);
    p.lc = take(bt * 4);
  }
  p.lg = take((size_t)C * p.ldl * es);
  if (p.gather) p.xg = take((size_t)C * p.Hp * es);
  if (p.wpad) p.wp = take((size_t)s.V * p.Hp * es);
  if (s.grad) {
    const bool defer = dw == kDwDefer;
    p.xt = take((size_t)p.Hp * ld_t(defer ? s.BT : C) * es);
    if (p.wt) p.wtp = take((size_t)p.Hp * p.ldl * es);
    if (p.dt) p.dtp = take((size_t)p.V8 * ld_t(defer ? s.BT : C) * es);
    if (dw == kDwAcc) p.acc = take((size_t)s.V * p.Hp * 4);
    const size_t pb = dx_part_bytes(C, p.Hp, p.ldl, dx_bk(s.es), smax);
    p.ksplit = pb ? smax : 1;
    p.part = pb ? take(pb) : 0;
  }
  p.extra = take(s.fixed_extra + (size_t)C * s.row_extra);
  p.total = off;
  return p;
}

// The vocabulary-tiled candidate: tiles of Vt columns (a multiple of 256) over
// all BT rows; dX summed in fp32 (dw = kDwAcc) or in the output (kDwOut).
FlPlan vt_layout(const FlShape& s, int64_t Vt, int dw) {
  FlPlan p;
  p.vtile = true;
  p.Vt = Vt;
  p.ntiles = cdiv(s.V, Vt);
  p.C = Vt;
  p.nch = p.ntiles;
  p.Hp = pad8(s.H);
  p.V8 = pad8(s.V);
  p.Vr = (s.V + 16 / s.es - 1) / (16 / s.es) * (16 / s.es);
  p.ldl = Vt;
  p.gather = !s.x_ok;
  p.wpad = !s.w_ok;
  p.dw = dw;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += align256(bytes);
    return o;
  };
  const size_t es = (size_t)s.es, bt = (size_t)std::max<int64_t>(s.BT, 1);
  p.nvalid = take(256);
  p.nlive = take(256);
  p.vst = take(bt * 16);
  p.lg = take(bt * (size_t)Vt * es);
  if (p.gather) p.xg = take(bt * (size_t)p.Hp * es);
  if (p.wpad) p.wp = take((size_t)s.V * p.Hp * es);
  if (s.grad && dw == kDwAcc && p.ntiles > 1) p.acc = take(bt * (size_t)p.Hp * 4);
  p.total = off;
  return p;
}

// Modelled time of a vocabulary-tiled candidate: the logits GEMM twice (the
// log-sum-exp pass, then the gradient pass), the dW GEMM with both operands
// MN-contiguous, the dX GEMM with W MN-contiguous, idle CUs when a GEMM has
// fewer than 256 tiles, the row passes' HBM bytes and dX's read-modify-writes.
double vt_cost(const FlShape& s, const FlPlan& p) {
  const double Rg = 1.25e15, Rm = 5.0e12, pen = 1.2, launch = 5e-6;
  const double es = s.es, BT = (double)s.BT, Hp = (double)p.Hp, V = (double)s.V;
  const double F = 2.0 * BT * Hp * V;
  // a GEMM of `tiles` 256x256 tiles takes whole waves of 256 (one workgroup a CU)
  auto fill = [](int64_t tiles) {
    tiles = std::max<int64_t>(tiles, 1);
    return (double)(cdiv(tiles, 256) * 256) / (double)tiles;
  };
  const int64_t tb = cdiv(s.BT, 256), tv = cdiv(p.Vt, 256), th = cdiv(p.Hp, 256);
  double t = F / Rg * fill(tb * tv) + BT * V * es / Rm + p.ntiles * 3 * launch;
  if (p.gather) t += 2.0 * es * BT * Hp / Rm;
  if (p.wpad) t += 2.0 * es * V * Hp / Rm;
  if (s.grad) {
    t += F / Rg * fill(tb * tv) + 2.0 * BT * V * es / Rm;
    t += F / Rg * fill(tv * th) * pen * pen;
    t += F / Rg * fill(tb * th) * pen;
    const double nt = (double)p.ntiles;
    t += (p.dw == kDwAcc ? 8.0 * BT * Hp * (nt - 1) : 2.0 * es * BT * Hp * (nt - 1)) / Rm;
    t += p.ntiles * 4 * launch;
  }
  return t;
}

// Modelled time (seconds) of a candidate: GEMMs at a kk-kernel rate, 15% more
// for a GEMM with an MN-contiguous operand, tile waste of a short chunk, a dX
// GEMM that leaves CUs idle, and the HBM bytes of the transposes, the dW
// read-modify-writes, the split partials and the gathers, plus launches.
double fl_cost(const FlShape& s, const FlPlan& p) {
  const double Rg = 1.25e15, Rm = 5.0e12, pen = 1.2, launch = 5e-6;
  const double es = s.es, BT = (double)s.BT, Hp = (double)p.Hp, V = (double)s.V;
  const double F = 2.0 * BT * Hp * V;
  // row waste of a chunk's last 256-row tile, and whole waves of 256 workgroups (one a CU)
  const double q = (double)(cdiv(p.C, 256) * 256) / (double)p.C;
  auto waves = [](int64_t wgs) {
    wgs = std::max<int64_t>(wgs, 1);
    return (double)(cdiv(wgs, 256) * 256) / (double)wgs;
  };
  const double nch = (double)p.nch;
  double t = F / Rg * q * waves(cdiv(p.C, 256) * cdiv(s.V, 256)) + nch * 6 * launch;
  if (p.gather) t += 2.0 * es * BT * Hp / Rm;
  if (p.wpad) t += 2.0 * es * V * Hp / Rm;
  if (s.grad) {
    const int64_t tiles = cdiv(p.C, 256) * cdiv(p.Hp, 256);
    const int sp = gemm::auto_splits((int)tiles, (int)(p.ldl / dx_bk(s.es)), p.ksplit);
    t += F / Rg * q * waves(tiles * sp) * (p.wt ? 1.0 : pen);
    if (sp > 1) t += nch * 2.0 * sp * (double)p.C * Hp * 4 / Rm;
    t += F / Rg * waves(cdiv(s.V, 256) * cdiv(p.Hp, 256)) * (p.dt ? 1.0 : pen);
    double rmw = es * V * Hp;
    if (p.dw == kDwAcc && p.nch > 1) rmw = 8.0 * V * Hp * (nch - 1) + es * V * Hp;
    if (p.dw == kDwOut) rmw = es * V * Hp * (2 * nch - 1);
    t += rmw / Rm;
    if (p.wt) t += 2.0 * es * V * Hp / Rm;
    if (p.dt) t += 2.0 * es * BT * (double)p.V8 / Rm;
    t += 2.0 * es * BT * Hp / Rm + nch * 4 * launch;
  }
  return t;
}

// The reference's chunk rule (fused_linear_cross_entropy.py:112-114): chunk
// logits about the size of the hidden states; at least 64 and at most 8192 rows.
int64_t ref_chunk(int64_t BT, int64_t H, int64_t V) {
  const int64_t per = std::max<int64_t>(1, cdiv(BT, cdiv(V, H)));
  int64_t c = 1;
  while (c < per) c <<= 1;
  return std::min<int64_t>(8192, std::max<int64_t>(64, c));
}

// Candidates in order of preference for a given chunk size (the leanest last).
template <typename F>
void fl_forms(const FlShape& s, int64_t nch, F&& f) {
  if (!s.grad) {
    f(false, false, kDwOut);
    return;
  }
  const bool mn_ok = s.es == 2;  // MN-contiguous operands are 16-bit only
  for (int dw : {kDwDefer, kDwAcc, kDwOut}) {
    if (dw == kDwDefer && nch < 2) continue;
    if (dw == kDwAcc && (nch < 2 || s.es == 4)) continue;  // fp32: the output is the fp32 accumulator
    for (int wt = 1; wt >= 0; --wt)
      for (int dt = 1; dt >= 0; --dt) {
        if ((!wt || !dt) && !mn_ok) continue;
        if (dw == kDwDefer && !dt) continue;
        f(wt != 0, dt != 0, dw);
      }
  }
}

// A debugging override of the form (like MIOpen's MIOPEN_DEBUG_* variables):
// HILDA_FL_FORM="<dw>,<w>,<d>" with dw one of defer / acc / out, w one of wt /
// wmn, d one of dt / dmn restricts the plan to that row-chunked form (the chunk
// still from the budget); "vtile,<acc|out>,<columns>" to the vocabulary-tiled
// plan with that dX sum and tile width (a multiple of 256). Returns false when
// unset; *bad when it does not parse. *vt: the tile width (0: row chunks).
bool forced_form(int* dw, bool* wt, bool* dt, int64_t* vt, bool* bad) {
  const char* e = std::getenv("HILDA_FL_FORM");
  *bad = false;
  *vt = 0;
  if (!e || !*e) return false;
  char a[16] = {0}, b[16] = {0}, c[16] = {0};
  if (std::sscanf(e, "%15[^,],%15[^,],%15s", a, b, c) != 3) {
    *bad = true;
    return true;
  }
  const std::string sa(a), sb(b), sc(c);
  if (sa == "vtile") {
    *dw = sb == "acc" ? kDwAcc : sb == "out" ? kDwOut : -1;
    *vt = std::atoll(c);
    *bad = *dw < 0 || *vt <= 0 || *vt % 256 != 0 || *vt > 8192;
    return true;
  }
  *dw = sa == "defer" ? kDwDefer : sa == "acc" ? kDwAcc : sa == "out" ? kDwOut : -1;
  *wt = sb == "wt";
  *dt = sc == "dt";
  *bad = *dw < 0 || (sb != "wt" && sb != "wmn") || (sc != "dt" && sc != "dmn");
  return true;
}

// Default budget floor: below this much chunk memory there is nothing worth
// saving, and small problems then run in one chunk (or with an fp32 dW
// accumulator). 40 MiB keeps the reference's tightest memory config
// (bench_fused_linear_ce.py:270-274: N 4096, V 128256, fp16) 47.7% below the
// unfused path, the low end of the reference's claim (README.md:42).
constexpr size_t kSmallWorkspace = (size_t)40 << 20;

// A plan that sums dW (and dX) in fp32 is taken over a faster one that sums in
// the 16-bit output unless it is modelled this much slower.
constexpr double kExactSlack = 1.5;

// dW summed in fp32 (or computed whole): every form but accumulation in a
// 16-bit output over several chunks.
bool exact_dw(const FlShape& s, const FlPlan& p) { return !s.grad || p.dw != kDwOut || p.nch <= 1 || s.es == 4; }
// (a vocabulary-tiled plan writes dW once; its dX is summed across the tiles in the same ways)

// The plan for a byte budget: budget == 0 the default (at most the larger of
// kSmallWorkspace and what the reference's chunk costs in the leanest form),
// budget < 0 unlimited, else at most `budget` bytes. Within the budget: the
// fastest candidate by fl_cost (vt_cost) whose sums are in fp32, unless the
// fastest of all, which accumulates in the 16-bit output (the reference's
// arithmetic, fused_linear_cross_entropy.py:161), is modelled more than
// kExactSlack times faster. HK_EINVAL when nothing fits.
int fl_plan(const FlShape& s, int64_t budget, FlPlan* out) {
  int f_dw = 0;
  int64_t f_vt = 0;
  bool f_wt = false, f_dt = false, f_bad = false;
  const bool forced = forced_form(&f_dw, &f_wt, &f_dt, &f_vt, &f_bad) && (s.grad || f_vt > 0);
  HK_REQUIRE(!f_bad, "HILDA_FL_FORM: expected <defer|acc|out>,<wt|wmn>,<dt|dmn> or vtile,<acc|out>,<columns>");
  const int64_t cmax_rows = std::min<int64_t>(8192, s.chunk_cap > 0 ? s.chunk_cap : 8192);
  const int64_t cmax = std::max<int64_t>(8, std::min<int64_t>(cmax_rows & ~(int64_t)7, pad8(std::max<int64_t>(s.BT, 1))));
  const int smax_full = s.grad ? (int)std::max<int64_t>(1, std::min<int64_t>(8, pad64(s.V) / dx_bk(s.es) / 16)) : 1;
  auto lean = [&](int64_t C, int sm) {
    const bool mn_ok = s.es == 2;
    return fl_layout(s, C, !mn_ok, !mn_ok, kDwOut, sm);
  };
  size_t cap;
  if (budget == 0) {
    const int64_t C0 = std::min<int64_t>(cmax, ref_chunk(s.BT, s.H, s.V));
    // the reference's chunk logits, the gathered rows and their transpose, and an
    // eighth of the chunk's bytes for the dX GEMM's split partials
    const FlPlan b = lean(C0, 1);
    cap = std::max({kSmallWorkspace, s.default_floor, b.total + (size_t)C0 * pad64(s.V) * s.es / 8});
  } else {
    cap = budget < 0 ? SIZE_MAX : (size_t)budget;
  }
  // the fastest candidate overall, the fastest whose dW (and dX) are summed in fp32, and (fp16 inputs) the
  // fastest that does not sum dW in the fp16 output over several chunks: gradients scaled by 1/n sit in
  // fp16's subnormal range there, where each rounding costs percent-level error (the vocabulary-tiled plan
  // sums dX unscaled, which stays in the normal range)
  bool found = false, found_ex = false, found_safe = false;
  FlPlan best, best_ex, best_safe;
  auto consider = [&](const FlPlan& p) {
    auto better = [&](const FlPlan& a, const FlPlan& b) {
      return a.cost < b.cost || (a.cost == b.cost && a.total < b.total);
    };
    if (!found || better(p, best)) {
      best = p;
      found = true;
    }
    if (exact_dw(s, p) && (!found_ex || better(p, best_ex))) {
      best_ex = p;
      found_ex = true;
    }
    const bool risky = s.f16 && !p.vtile && !exact_dw(s, p);
    if (!risky && (!found_safe || better(p, best_safe))) {
      best_safe = p;
      found_safe = true;
    }
  };
  std::vector<int64_t> cs;
  for (int64_t C = cmax; C >= 8; C = (C > 64 ? (C - 1) / 64 * 64 : C / 2 & ~(int64_t)7)) {
    cs.push_back(C);
    if (C <= 8) break;
  }
  for (int64_t C : cs) {
    const int64_t nch = s.BT > 0 ? cdiv(s.BT, C) : 0;
    fl_forms(s, nch, [&](bool wt, bool dt, int dw) {
      if (forced && (f_vt > 0 || dw != f_dw || wt != f_wt || dt != f_dt)) return;
      for (int sm = smax_full; sm >= 1; sm = sm > 1 ? sm / 2 : 0) {
        FlPlan p = fl_layout(s, C, wt, dt, dw, sm);
        if (p.total > cap) continue;
        p.cost = fl_cost(s, p);
        consider(p);
        break;  // fewer splits only if more do not fit
      }
    });
  }
  if (s.vt_ok && s.BT > 0 && (forced ? f_vt > 0 : s.chunk_cap <= 0)) {
    const int64_t vmax = std::min<int64_t>(8192, (s.V + 255) / 256 * 256);
    for (int64_t Vt = vmax; Vt >= 256; Vt -= 256)
      for (int dw : {kDwAcc, kDwOut}) {
        if (forced && (Vt != f_vt || dw != f_dw)) continue;
        FlPlan p = vt_layout(s, Vt, dw);
        if (p.total > cap) continue;
        p.cost = vt_cost(s, p);
        consider(p);
      }
  }
  if (!found && forced) {
    set_error("HILDA_FL_FORM: the forced form does not apply to this call (dtype, chunk count or budget)");
    return HK_EINVAL;
  }
  if (!found) {
    const FlPlan small = lean(cs.back(), 1);
    set_error("workspace budget %lld bytes is below the smallest plan (%zu bytes)", (long long)budget, small.total);
    return HK_EINVAL;
  }
  // fp32 sums unless they cost more than half as much time again as the fastest plan (fp16: the fastest
  // plan without fp16 dW sums over chunks, when one fits)
  const FlPlan& fast = s.f16 && found_safe ? best_safe : best;
  *out = found_ex && best_ex.cost <= kExactSlack * fast.cost ? best_ex : fast;
  return HK_OK;
}

// ---------------------------------------------------------------------------
// The chunk loop shared by the fused-linear losses.
//
// X [BT, H] (row stride H) and W [V, H] are the caller's hidden states and
// weight. With rowmap, the rows are compacted first: rowmap[i] is compacted
// row i's original row, *n_live (device memory) their count; each chunk
// gathers its live rows (zero rows after them) and every GEMM is cut to the
// live rows on the device (tiles past them exit, the dW GEMM's K stops at
// them); dX_c is stored straight into the original rows and the caller zeroes
// the dead rows of dX. Without rowmap (n_live null too) every row is live.
//
// row_step(Lg, r0, cs): the chunk's logits Lg (compacted rows r0 .. r0 + cs,
// row stride plan.ldl) to row losses and, with gradients, the dlogits D_c
// written over them (zero past the row step's width). pad: what the logits
// epilogue writes past V in the straddling 16-byte chunk.
template <typename T, class RowStep>
int chunked_lm_head(const T* X, const T* W, int64_t BT, int64_t H, int64_t V, char* ws, const FlPlan& p, bool grad,
                    T* dX, T* dWo, const int* n_live, const int* rowmap, float pad, RowStep&& row_step,
                    hipStream_t st) {
  constexpr int E = 16 / (int)sizeof(T);
  const int64_t C = p.C, Hp = p.Hp, ldl = p.ldl;
  const bool defer = grad && p.dw == kDwDefer;
  T* Lg = (T*)(ws + p.lg);
  T* Xg = p.gather ? (T*)(ws + p.xg) : nullptr;
  T* Wp = p.wpad ? (T*)(ws + p.wp) : nullptr;
  T* Wt = p.wt ? (T*)(ws + p.wtp) : nullptr;
  T* Xt = grad ? (T*)(ws + p.xt) : nullptr;
  T* Dt = p.dt ? (T*)(ws + p.dtp) : nullptr;
  float* acc = (grad && p.dw == kDwAcc) ? (float*)(ws + p.acc) : nullptr;
  const T* Wk = p.wpad ? Wp : W;  // K-contiguous weight rows
  const int64_t ldw = p.wpad ? Hp : H;
  int rc = HK_OK;
  if (p.wpad) {  // the weight rows at a 16-byte multiple, zero filled past H
    rc = gather_rows<T>(Wp, Hp, Hp, W, H, H, nullptr, nullptr, V, 0, V, st);
    if (rc) return rc;
  }
  // the chunk buffer's columns the row step never writes are the dX GEMM's K padding: zero
  rc = zero_cols<T>(Lg, ldl, p.Vr, ldl, C, st);
  if (rc) return rc;
  // The transposes (HBM-bound) run on a side stream beside the GEMMs
  // (MFMA-bound; a transpose workgroup fits in the registers and LDS a GEMM
  // workgroup leaves free on its CU): W^T beside the first chunk's logits, each
  // chunk's X^T and D^T beside its dX GEMM. `side_pending`: the side stream
  // holds work the caller's stream has not joined yet.
  hipStream_t side = nullptr;
  bool side_pending = false;
  if (grad) {
    const int dev = current_device();
    side = dev >= 0 ? side_stream(dev) : nullptr;
    if (!side) return HK_EINVAL;
  }
  auto fork = [&]() { return stream_after(side, st); };
  auto join = [&]() {
    if (!side_pending) return HK_OK;
    side_pending = false;
    return stream_after(st, side);
  };
  // An error return also leaves the caller's stream ordered after the side
  // stream's work: the caller may free the workspace as soon as we return.
  struct JoinOnExit {
    hipStream_t st, side;
    bool& pending;
    ~JoinOnExit() {
      if (pending) (void)stream_after(st, side);
    }
  } join_on_exit{st, side, side_pending};
  if (grad && p.wt) {
    rc = fork();
    if (rc) return rc;
    rc = launch_transpose<T>(Wt, Wk, V, ldl, Hp, ldw, ldl, side);  // W^T [Hp, ldl], zero columns past V
    if (rc) return rc;
    side_pending = true;
  }
  const int64_t BTp = pad8(BT), ldxt = ld_t(defer ? BT : C);
  const bool dvec = H % 4 == 0 && aligned_to(dX, 16);    // 4-element stores of dX rows
  const bool wvec = H % 4 == 0 && aligned_to(dWo, 16);   // and of dW rows
  const int kt_dx = (int)(ldl / gemm::CfgFor<T>::BK);
  for (int64_t ci = 0; ci < p.nch; ++ci) {
    const int64_t r0 = ci * C;
    const int64_t cs = std::min<int64_t>(C, BT - r0);
    if (ci > 0) {  // the previous chunk's transposes still read Xg and Lg
      rc = join();
      if (rc) return rc;
    }
    // the chunk's hidden rows, K-contiguous
    const T* Xc = X + r0 * H;
    int64_t ldxc = H;
    if (p.gather) {
      rc = gather_rows<T>(Xg, Hp, Hp, X, H, H, rowmap, n_live, BT, r0, cs, st);
      if (rc) return rc;
      Xc = Xg;
      ldxc = Hp;
    }
    // logits_c = X_c W^T (live rows only)
    rc = launch_gemm<T>(Xc, Wk, (int)cs, (int)V, (int)Hp, ldxc, ldw, EpiLogits<T>{Lg, ldl, pad}, st, n_live,
                        (int)r0);
    if (rc) return rc;
    rc = row_step(Lg, r0, cs);
    if (rc) return rc;
    if (!grad) continue;
    // X_c^T (zeros past the live rows) into X^T: columns [r0, r0 + cs) of [Hp, BT] when
    // deferred, else [Hp, C]; and D_c^T when materialised: into columns [r0, r0 + cs) of
    // D^T [V8, BTp] (zeros past the live rows) when deferred, else D^T [V8, C]. On the
    // side stream, beside the dX GEMM, which also only reads the chunk.
    const int64_t csp = pad8(cs);
    {
      rc = join();  // W^T, which the dX GEMM reads
      if (rc) return rc;
      rc = fork();
      if (rc) return rc;
      T* xt_dst = defer ? Xt + r0 : Xt;
      const int64_t xrp = defer ? (ci + 1 < p.nch ? cs : BTp - r0) : csp;
      rc = launch_transpose<T>(xt_dst, Xc, cs, xrp, Hp, ldxc, ldxt, side, n_live, r0);
      if (rc) return rc;
      if (defer) rc = launch_transpose<T>(Dt + r0, Lg, cs, xrp, p.V8, ldl, ldxt, side, n_live, r0);
      else if (p.dt) rc = launch_transpose<T>(Dt, Lg, cs, csp, p.V8, ldl, ldxt, side, n_live, r0);
      if (rc) return rc;
      side_pending = true;
    }
    // dX_c = D_c W, stored into the live rows' original places; a short chunk
    // splits K (= ldl) and sums the splits' fp32 partials in a second pass
    T* dst = rowmap ? dX : dX + r0 * H;
    const int* map = rowmap ? rowmap + r0 : nullptr;
    float* part = p.ksplit > 1 ? (float*)(ws + p.part) : nullptr;
    const EpiDx<T> edx{dst, H, map, part, Hp, (int)H, dvec};
    if (p.wt)
      rc = launch_gemm<T>(Lg, Wt, (int)cs, (int)Hp, (int)ldl, ldl, ldl, edx, st, n_live, (int)r0, false, p.ksplit);
    else  // W [V, ldw] read MN-contiguous: k = the vocabulary row, past V zero
      rc = launch_gemm_mn<T, false, true>(Lg, Wk, (int)cs, (int)Hp, (int)ldl, ldl, ldw, edx, st, n_live, (int)r0,
                                          false, p.ksplit, (int)V);
    if (rc) return rc;
    if (p.ksplit > 1) {
      const int64_t work = cs * cdiv(H, 4);
      hipLaunchKernelGGL((splitk_sum_kernel<T>), dim3((unsigned)std::min<int64_t>(cdiv(work, 256), 8192)), dim3(256),
                         0, st, dst, H, map, part, (int)cs, (int)Hp, kt_dx, p.ksplit, n_live, (int)r0, (int)H,
                         dvec ? 1 : 0);
      rc = check_launch("splitk_sum_kernel");
      if (rc) return rc;
    }
    if (defer) continue;
    // dW (+)= D_c^T X_c; K = cs is padded to a multiple of 8 with zeros on both operands, and cut
    // on the device to the live rows
    rc = join();
    if (rc) return rc;
    auto dw_gemm = [&](auto epi) {
      if (p.dt)
        return launch_gemm<T>(Dt, Xt, (int)V, (int)Hp, (int)csp, ldxt, ldxt, epi, st, n_live, (int)r0, true);
      // D_c [cs, ldl] read MN-contiguous (k = the chunk row, m = the vocabulary column); its rows stop at
      // cs (the chunk buffer's rows past it were never written), or at the live rows on the device
      return launch_gemm_mn<T, true, false>(Lg, Xt, (int)p.V8, (int)Hp, (int)csp, ldl, ldxt, epi, st, n_live,
                                            (int)r0, true, 1, 0, (int)cs);
    };
    const int vl = (int)V, hl = (int)H;
    if (p.nch == 1) rc = dw_gemm(EpiDw<T, 0>{dWo, H, nullptr, Hp, vl, hl, wvec});
    else if (p.dw == kDwOut) rc = ci == 0 ? dw_gemm(EpiDw<T, 0>{dWo, H, nullptr, Hp, vl, hl, wvec})
                                          : dw_gemm(EpiDw<T, 1>{dWo, H, nullptr, Hp, vl, hl, wvec});
    else if (ci == 0) rc = dw_gemm(EpiDw<T, 2>{dWo, H, acc, Hp, vl, hl, wvec});
    else if (ci + 1 < p.nch) rc = dw_gemm(EpiDw<T, 3>{dWo, H, acc, Hp, vl, hl, wvec});
    else rc = dw_gemm(EpiDw<T, 4>{dWo, H, acc, Hp, vl, hl, wvec});
    if (rc) return rc;
  }
  rc = join();  // (also leaves no work of this call behind on the side stream)
  if (rc) return rc;
  if (defer && p.nch > 0) {
    rc = launch_gemm<T>(Dt, Xt, (int)V, (int)Hp, (int)BTp, ldxt, ldxt,
                        EpiDw<T, 0>{dWo, H, nullptr, Hp, (int)V, (int)H, wvec}, st, n_live, 0, true);
    if (rc) return rc;
  }
  if (grad && p.nch == 0 && V > 0) {
    // no rows: the weight gradient is zero (dX is empty)
    rc = zero_cols<T>(dWo, H, 0, H, V, st);
    if (rc) return rc;
  }
  (void)E;
  return rc;
}


// The vocabulary-tiled plan for CrossEntropy (p.vtile). Pass 1, per tile of
// Vt vocabulary columns: the logits of every row for those columns (the same
// GEMM as the row-chunked plans, so the same logits bit for bit), folded into
// each row's running log-sum-exp. Then the losses. Pass 2, per tile: the
// logits again, the gradient tile D in place, dW of the tile's vocabulary rows
// as one GEMM over all BT rows (written once, summed in fp32), and dX += D W_t,
// summed across the tiles in an fp32 buffer or in the output. No rows are
// compacted: ignored rows have zero gradient rows. n_valid is counted already.
template <typename T>
int vtiled_ce(const T* X, const T* W, int64_t BT, int64_t H, int64_t V, char* ws, const FlPlan& p, bool grad, T* dX,
              T* dWo, const int64_t* targets, int64_t ignore_index, const int* n_valid, bool mean,
              const float* row_scale, float* loss_rows, hipStream_t st) {
  const int64_t Hp = p.Hp, Vt = p.Vt;
  T* Lt = (T*)(ws + p.lg);
  VtRow* state = (VtRow*)(ws + p.vst);
  float* acc = (grad && p.dw == kDwAcc && p.ntiles > 1) ? (float*)(ws + p.acc) : nullptr;
  int rc = HK_OK;
  const T* Xk = X;
  int64_t ldx = H;
  if (p.gather) {  // hidden rows at a 16-byte multiple, zero filled past H
    rc = gather_rows<T>((T*)(ws + p.xg), Hp, Hp, X, H, H, nullptr, nullptr, BT, 0, BT, st);
    if (rc) return rc;
    Xk = (const T*)(ws + p.xg);
    ldx = Hp;
  }
  const T* Wk = W;
  int64_t ldw = H;
  if (p.wpad) {
    rc = gather_rows<T>((T*)(ws + p.wp), Hp, Hp, W, H, H, nullptr, nullptr, V, 0, V, st);
    if (rc) return rc;
    Wk = (const T*)(ws + p.wp);
    ldw = Hp;
  }
  const int dev = current_device();
  const int cu = dev >= 0 ? cu_count(dev) : 256;
  const dim3 rgrid((unsigned)std::min<int64_t>(BT, (int64_t)(cu > 0 ? cu : 256) * 8));
  auto logits = [&](int64_t v0, int64_t w) {
    return launch_gemm<T>(Xk, Wk + v0 * ldw, (int)BT, (int)w, (int)Hp, ldx, ldw,
                          EpiLogits<T>{Lt, Vt, -__builtin_huge_valf()}, st);
  };
  for (int64_t ti = 0; ti < p.ntiles; ++ti) {
    const int64_t v0 = ti * Vt, w = std::min<int64_t>(Vt, V - v0);
    rc = logits(v0, w);
    if (rc) return rc;
    hipLaunchKernelGGL((vt_lse_kernel<T>), rgrid, dim3(kVtLanes), 0, st, Lt, Vt, w, v0, targets, ignore_index, state,
                       BT, ti == 0 ? 1 : 0);
    rc = check_launch("vt_lse_kernel");
    if (rc) return rc;
  }
  const bool scale = grad && mean;
  hipLaunchKernelGGL(vt_finalize_kernel, dim3((unsigned)std::min<int64_t>(cdiv(BT, 256), 4096)), dim3(256), 0, st,
                     state, loss_rows, targets, ignore_index, n_valid, scale ? 1 : 0, BT);
  rc = check_launch("vt_finalize_kernel");
  if (rc || !grad) return rc;
  const bool dvec = H % 4 == 0 && aligned_to(dX, 16);
  const bool wvec = H % 4 == 0 && aligned_to(dWo, 16);
  // dX summed in the output over several tiles: D without the 1/n of 'mean' (applied by dW's epilogue and
  // by the last pass over dX), and without its target entries (see vt_drop_targets_kernel)
  const bool out_sum = p.ntiles > 1 && !acc;
  const int* dw_scale = out_sum && scale ? n_valid : nullptr;
  for (int64_t ti = 0; ti < p.ntiles; ++ti) {
    const int64_t v0 = ti * Vt, w = std::min<int64_t>(Vt, V - v0), w8 = pad8(w);
    rc = logits(v0, w);
    if (rc) return rc;
    hipLaunchKernelGGL((vt_grad_kernel<T>), rgrid, dim3(kVtLanes), 0, st, Lt, Vt, w, w8, v0, targets, ignore_index,
                       state, n_valid, scale && !out_sum ? 1 : 0, row_scale, BT);
    rc = check_launch("vt_grad_kernel");
    if (rc) return rc;
    // dW of the tile's rows: D [BT, w8] (k = the row, m = the tile column) and X [BT, Hp] (k = the row,
    // n = the hidden column), both read MN-contiguous; K = BT
    rc = launch_gemm_mn<T, true, true>(Lt, Xk, (int)w8, (int)Hp, (int)BT, Vt, ldx,
                                       EpiDw<T, 0>{dWo + v0 * H, H, nullptr, Hp, (int)w, (int)H, wvec, dw_scale},
                                       st);
    if (rc) return rc;
    if (out_sum) {
      // summed in the 16-bit output: the softmax terms only (see vt_drop_targets_kernel)
      hipLaunchKernelGGL((vt_drop_targets_kernel<T>), dim3((unsigned)std::min<int64_t>(cdiv(BT, 256), 4096)),
                         dim3(256), 0, st, Lt, Vt, w, v0, targets, ignore_index, BT);
      rc = check_launch("vt_drop_targets_kernel");
      if (rc) return rc;
    }
    // dX (+)= D W_t: D K-contiguous (K = w8, zero past w), W_t's rows read MN-contiguous (k past w zero)
    auto dx_gemm = [&](auto epi) {
      return launch_gemm_mn<T, false, true>(Lt, Wk + v0 * ldw, (int)BT, (int)Hp, (int)w8, Vt, ldw, epi, st, nullptr,
                                            0, false, 1, (int)w);
    };
    const int bl = (int)BT, hl = (int)H;
    if (p.ntiles == 1) rc = dx_gemm(EpiDw<T, 0>{dX, H, nullptr, Hp, bl, hl, dvec});
    else if (!acc) rc = ti == 0 ? dx_gemm(EpiDw<T, 0>{dX, H, nullptr, Hp, bl, hl, dvec})
                                : dx_gemm(EpiDw<T, 1>{dX, H, nullptr, Hp, bl, hl, dvec});
    else if (ti == 0) rc = dx_gemm(EpiDw<T, 2>{dX, H, acc, Hp, bl, hl, dvec});
    else if (ti + 1 < p.ntiles) rc = dx_gemm(EpiDw<T, 3>{dX, H, acc, Hp, bl, hl, dvec});
    else rc = dx_gemm(EpiDw<T, 4>{dX, H, acc, Hp, bl, hl, dvec});
    if (rc) return rc;
  }
  if (out_sum) {
    hipLaunchKernelGGL((vt_target_dx_kernel<T>), rgrid, dim3(256), 0, st, dX, H, Wk, ldw, targets, ignore_index, V,
                       state, n_valid, scale ? 1 : 0, row_scale, BT);
    rc = check_launch("vt_target_dx_kernel");
  }
  return rc;
}

// Shape checks shared by the fused-linear entry points.
int fl_check_dims(int64_t BT, int64_t H, int64_t V) {
  HK_REQUIRE(BT >= 0 && H > 0 && V > 0, "invalid shape BT=%lld H=%lld V=%lld", (long long)BT, (long long)H,
             (long long)V);
  HK_REQUIRE(BT < (1LL << 31) - 8192 && H < (1LL << 30) && V < (1LL << 31) - 4096, "dimension too large");
  return HK_OK;
}

FlShape flce_shape(int64_t BT, int64_t H, int64_t V, int dtype, bool grad, int64_t chunk, const void* hidden,
                   const void* weight) {
  FlShape s{};
  s.BT = BT;
  s.H = H;
  s.V = V;
  s.es = fl_esize(dtype);
  s.grad = grad;
  s.compact = true;
  // (rows of a multiple of 8 elements: the padded width Hp is then H itself)
  s.x_ok = H % 8 == 0 && (!hidden || aligned_to(hidden, 16));
  s.w_ok = H % 8 == 0 && (!weight || aligned_to(weight, 16));
  s.ce = true;
  s.chunk_cap = chunk;
  s.vt_ok = s.es == 2;  // (the tiled dW GEMM reads both operands MN-contiguous: 16-bit only)
  s.f16 = dtype == HK_F16;
  return s;
}

}  // namespace
}  // namespace hk

namespace hk {
namespace {
// Default-budget floor of FusedLinear-GRPO (no vocabulary-tiled plan and no
// reference to follow): twice the bytes of the weight (the size of its
// gradient, which the op allocates anyway, twice over). Below it the plans
// fall back to short chunks, whose dW GEMM re-reads and rewrites the whole
// weight gradient every chunk: at B 16, L+1 1024, H 4096, V 151936 bf16 95 ms
// with a 150 MB plan, 44 ms at the floor, 36 ms with no limit.
size_t weight_pair_bytes(int64_t V, int64_t H, int es) { return 2 * (size_t)V * (size_t)pad8(H) * (size_t)es; }

// Default-budget floor of FusedLinearJSD: what the reference's chunk loop
// holds at once (fused_linear_jsd.py:133-135,159-203) in its dW product: per
// logit of a chunk of the reference's rows, the student and teacher logits in
// the input dtype, their fp32 log-softmax copies, the fp32 dX and dlogits and
// the dlogits cast back (22 bytes; 16 for fp32 inputs, whose .float() and
// .to() return the tensor itself), plus the [V, H] product dlogits^T X before
// it is added into grad_weight. The op's outputs are the reference's, so a
// workspace within this keeps its peak memory at or below the reference's.
// (Smaller budgets mean short chunks: BT 8192, H 4096, V 128256 bf16 ran
// 60 ms at 256 MiB, 38 ms at 1 GiB, 35 ms at 1.5 GiB, 31 ms with no limit.)
size_t jsd_reference_bytes(int64_t BT, int64_t H, int64_t V, int es) {
  // the reference's chunk rows, unclamped (fused_linear_jsd.py:133-135), at most BT
  const int64_t per = std::max<int64_t>(1, cdiv(BT, cdiv(V, H)));
  int64_t c = 1;
  while (c < per) c <<= 1;
  c = std::min<int64_t>(c, BT);
  return (size_t)c * (size_t)V * (es == 4 ? 16 : 22) + (size_t)V * (size_t)H * (size_t)es;
}

struct JsdExtra {
  size_t lc, labc, lt, xtc, wtp, total;
};
JsdExtra jsd_extra(int64_t BT, int64_t Ht, int64_t V, int64_t C, int es, bool t_gather, bool t_wpad) {
  JsdExtra e{};
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += align256(bytes);
    return o;
  };
  const size_t bt = (size_t)std::max<int64_t>(BT, 1);
  e.lc = take(bt * 4);
  e.labc = take(bt * 8);
  e.lt = take((size_t)C * pad64(V) * es);
  e.xtc = t_gather ? take((size_t)C * pad8(Ht) * es) : 0;
  e.wtp = t_wpad ? take((size_t)V * pad8(Ht) * es) : 0;
  e.total = off;
  return e;
}

FlShape fljsd_shape(int64_t BT, int64_t H, int64_t Ht, int64_t V, int dtype, bool grad, int64_t chunk, bool labels,
                    const void* s_in, const void* s_w, const void* t_in, const void* t_w, bool* t_gather,
                    bool* t_wpad) {
  FlShape s{};
  s.BT = BT;
  s.H = H;
  s.V = V;
  s.es = fl_esize(dtype);
  s.grad = grad;
  s.compact = labels;
  s.x_ok = H % 8 == 0 && (!s_in || aligned_to(s_in, 16));
  s.w_ok = H % 8 == 0 && (!s_w || aligned_to(s_w, 16));
  *t_gather = labels || Ht % 8 != 0 || (t_in && !aligned_to(t_in, 16));
  *t_wpad = Ht % 8 != 0 || (t_w && !aligned_to(t_w, 16));
  const JsdExtra e0 = jsd_extra(BT, Ht, V, 0, s.es, *t_gather, *t_wpad);
  s.f16 = dtype == HK_F16;
  s.fixed_extra = e0.total + 4 * 256;
  s.row_extra = (size_t)pad64(V) * s.es + (*t_gather ? (size_t)pad8(Ht) * s.es : 0);
  s.chunk_cap = chunk;
  s.default_floor = jsd_reference_bytes(BT, H, V, s.es);
  return s;
}
}  // namespace
namespace {
FlShape flgrpo_shape(int64_t B, int64_t L, int64_t H, int64_t V, int dtype, bool grad, int64_t chunk,
                     const void* hidden, const void* weight) {
  FlShape s = flce_shape(B * (L + 1), H, V, dtype, grad, chunk, hidden, weight);
  s.ce = false;
  s.vt_ok = false;
  s.fixed_extra = grpo_scratch_bytes(B, L);
  s.default_floor = weight_pair_bytes(V, H, s.es);
  return s;
}
}  // namespace
}  // namespace hk

namespace hk {
namespace {
// The plan queries' info[8] (the layout the header gives).
void plan_info(const FlPlan& p, int64_t* info) {
  info[0] = p.C;
  info[1] = p.nch;
  info[2] = p.vtile ? 3 + (p.dw == kDwAcc ? 0 : 1) : p.dw;
  info[3] = p.wt ? 1 : 0;
  info[4] = p.dt ? 1 : 0;
  info[5] = p.ksplit;
  info[6] = (int64_t)p.total;
  info[7] = (int64_t)(p.cost * 1e9);
}
}  // namespace
}  // namespace hk

using namespace hk;

extern "C" {

size_t hk_fused_linear_cross_entropy_workspace_size(int64_t BT, int64_t H, int64_t V, int64_t chunk,
                                                    int64_t workspace_budget, int dtype, int with_grad,
                                                    const void* hidden, const void* weight) {
  if (!fl_dtype_ok(dtype) || fl_check_dims(BT, H, V) != HK_OK) return 0;
  FlPlan p;
  if (fl_plan(flce_shape(BT, H, V, dtype, with_grad != 0, chunk, hidden, weight), workspace_budget, &p) != HK_OK)
    return 0;
  return p.total;
}

int hk_fused_linear_cross_entropy_plan(int64_t BT, int64_t H, int64_t V, int64_t chunk, int64_t workspace_budget,
                                       int dtype, int with_grad, const void* hidden, const void* weight,
                                       int64_t* info) {
  HK_REQUIRE(fl_dtype_ok(dtype), "fused linear cross entropy supports fp32, bf16 and fp16 (got %d)", dtype);
  if (const int rc = fl_check_dims(BT, H, V)) return rc;
  HK_REQUIRE(info, "null pointer argument");
  FlPlan p;
  if (const int rc = fl_plan(flce_shape(BT, H, V, dtype, with_grad != 0, chunk, hidden, weight), workspace_budget,
                             &p))
    return rc;
  plan_info(p, info);
  return HK_OK;
}

int hk_fused_linear_cross_entropy(float* loss_out, float* loss_rows, void* dhidden, void* dweight, const void* hidden,
                                  const void* weight, const int64_t* targets, const float* row_scale, int64_t BT,
                                  int64_t H, int64_t V, int64_t ignore_index, int reduction, int dtype, int64_t chunk,
                                  int64_t workspace_budget, void* workspace, size_t workspace_bytes,
                                  hk_stream_t stream) {
  HK_REQUIRE(fl_dtype_ok(dtype), "fused linear cross entropy supports fp32, bf16 and fp16 (got %d)", dtype);
  if (const int rc = fl_check_dims(BT, H, V)) return rc;
  HK_REQUIRE(reduction >= HK_REDUCTION_NONE && reduction <= HK_REDUCTION_SUM, "invalid reduction %d", reduction);
  const bool grad = dhidden != nullptr || dweight != nullptr;
  HK_REQUIRE(!grad || (dhidden && dweight), "dhidden and dweight are computed together");
  HK_REQUIRE(loss_rows && hidden && weight && targets, "null pointer argument");
  const int es = fl_esize(dtype);
  HK_REQUIRE(aligned_to(hidden, es) && aligned_to(weight, es) &&
                 (!grad || (aligned_to(dhidden, es) && aligned_to(dweight, es))),
             "hidden, weight and gradients must be aligned to their element size");
  FlPlan lay;
  if (const int rc = fl_plan(flce_shape(BT, H, V, dtype, grad, chunk, hidden, weight), workspace_budget, &lay))
    return rc;
  HK_REQUIRE(workspace && workspace_bytes >= lay.total, "workspace too small: need %zu bytes, got %zu", lay.total,
             workspace_bytes);
  HK_REQUIRE(aligned_to(workspace, 256), "workspace must be 256-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  int* n_valid = (int*)(ws + lay.nvalid);
  int* n_live = (int*)(ws + lay.nlive);
  int* rowmap = (int*)(ws + lay.rowmap);
  int* inv = (int*)(ws + lay.inv);
  int64_t* tc = (int64_t*)(ws + lay.tc);
  float* sc = (float*)(ws + lay.sc);
  float* lc = (float*)(ws + lay.lc);
  // every target equal to ignore_index is ignored (fused_linear_cross_entropy.py:121,62-65);
  // unlike the CrossEntropy op, -1 is not a "no ignore" sentinel here
  const int has_ignore = 1;

  auto run = [&](auto tag) -> int {
    using T = typename decltype(tag)::type;
    int rc = HK_OK;
    if (lay.vtile) {
      rc = count_valid_launch(n_valid, targets, BT, ignore_index, has_ignore, st);
      if (rc) return rc;
      rc = vtiled_ce<T>((const T*)hidden, (const T*)weight, BT, H, V, ws, lay, grad, (T*)dhidden, (T*)dweight,
                        targets, ignore_index, n_valid, reduction == HK_REDUCTION_MEAN, row_scale, loss_rows, st);
      if (rc) return rc;
      if (!loss_out) return HK_OK;
      const bool divide = !grad && reduction == HK_REDUCTION_MEAN;
      return sum_rows_launch(loss_out, loss_rows, BT, divide ? n_valid : nullptr, divide, st);
    }
    if (BT > 0) {
      rc = count_valid_launch(n_valid, targets, BT, ignore_index, has_ignore, st);
      if (rc) return rc;
      // the non-ignored rows, compacted: their targets and row scales (each chunk gathers its hidden rows)
      rc = ce_compact_launch(rowmap, inv, n_live, targets, BT, ignore_index, st);
      if (rc) return rc;
      hipLaunchKernelGGL(gather_ce_kernel, dim3((unsigned)std::min<int64_t>(cdiv(BT, 256), 1024)), dim3(256), 0, st,
                         tc, sc, targets, row_scale, rowmap, n_live);
      rc = check_launch("gather_ce_kernel");
      if (rc) return rc;
    }
    // per-row loss of the compacted rows; with gradients, D_c = (softmax - onehot) * s * row_scale
    // written over the logits (the -inf padding past V to the row width gives exact zeros)
    auto ce_step = [&](T* Lg, int64_t r0, int64_t cs) {
      return ce_rows_launch(grad ? (void*)Lg : nullptr, lc + r0, Lg, tc + r0, cs, lay.Vr, lay.ldl, lay.ldl,
                            ignore_index, has_ignore, n_valid, grad && reduction == HK_REDUCTION_MEAN,
                            row_scale ? sc + r0 : nullptr, dtype, st, n_live, r0);
    };
    rc = chunked_lm_head<T>((const T*)hidden, (const T*)weight, BT, H, V, ws, lay, grad, (T*)dhidden, (T*)dweight,
                            n_live, rowmap, -__builtin_huge_valf(), ce_step, st);
    if (rc) return rc;
    // losses back in row order (ignored rows 0); ignored rows of dhidden are zero
    rc = finish_rows<T>(grad ? (T*)dhidden : nullptr, loss_rows, lc, inv, BT, H, st);
    if (rc) return rc;
    if (loss_out) {
      // with gradients the rows already carry 1/max(n_valid,1) for 'mean'; without, divide here
      const bool divide = !grad && reduction == HK_REDUCTION_MEAN && BT > 0;
      return sum_rows_launch(loss_out, loss_rows, BT, divide ? n_valid : nullptr, divide, st);
    }
    return HK_OK;
  };
  return fl_dispatch(dtype, run);
}

// ---------------------------------------------------------------------------
// FusedLinearJSD: the engine with a row step that runs the teacher GEMM on the
// chunk's (gathered) teacher rows into a second chunk buffer, then one row
// kernel (both temperature log-softmaxes, JSD, the student dlogits).
// Extra workspace: per-row losses and compacted labels (BT each), the teacher
// logits chunk and gathered teacher rows (per chunk row) and a padded copy of
// the teacher weight when its rows are not 16-byte multiples.
// ---------------------------------------------------------------------------

size_t hk_fused_linear_jsd_workspace_size(int64_t BT, int64_t H, int64_t Ht, int64_t V, int64_t chunk,
                                          int64_t workspace_budget, int dtype, int with_grad, int with_labels,
                                          const void* s_input, const void* s_weight, const void* t_input,
                                          const void* t_weight) {
  if (!fl_dtype_ok(dtype) || Ht <= 0 || Ht >= (1LL << 30) || fl_check_dims(BT, H, V) != HK_OK) return 0;
  bool tg, tw;
  FlPlan p;
  if (fl_plan(fljsd_shape(BT, H, Ht, V, dtype, with_grad != 0, chunk, with_labels != 0, s_input, s_weight, t_input,
                          t_weight, &tg, &tw),
              workspace_budget, &p) != HK_OK)
    return 0;
  return p.total;
}

int hk_fused_linear_jsd_plan(int64_t BT, int64_t H, int64_t Ht, int64_t V, int64_t chunk, int64_t workspace_budget,
                             int dtype, int with_grad, int with_labels, const void* s_input, const void* s_weight,
                             const void* t_input, const void* t_weight, int64_t* info) {
  HK_REQUIRE(fl_dtype_ok(dtype), "fused linear JSD supports fp32, bf16 and fp16 (got %d)", dtype);
  if (const int rc = fl_check_dims(BT, H, V)) return rc;
  HK_REQUIRE(Ht > 0 && Ht < (1LL << 30), "invalid teacher hidden size Ht=%lld", (long long)Ht);
  HK_REQUIRE(info, "null pointer argument");
  bool tg, tw;
  FlPlan p;
  if (const int rc = fl_plan(fljsd_shape(BT, H, Ht, V, dtype, with_grad != 0, chunk, with_labels != 0, s_input,
                                         s_weight, t_input, t_weight, &tg, &tw),
                             workspace_budget, &p))
    return rc;
  plan_info(p, info);
  return HK_OK;
}

int hk_fused_linear_jsd(float* loss_out, void* dinput, void* dweight, const void* s_input, const void* s_weight,
                        const void* t_input, const void* t_weight, const int64_t* labels, int64_t BT, int64_t H,
                        int64_t Ht, int64_t V, int64_t ignore_index, float beta, float temperature, int dtype,
                        int64_t chunk, int64_t workspace_budget, void* workspace, size_t workspace_bytes,
                        hk_stream_t stream) {
  HK_REQUIRE(fl_dtype_ok(dtype), "fused linear JSD supports fp32, bf16 and fp16 (got %d)", dtype);
  if (const int rc = fl_check_dims(BT, H, V)) return rc;
  HK_REQUIRE(Ht > 0 && Ht < (1LL << 30), "invalid teacher hidden size Ht=%lld", (long long)Ht);
  HK_REQUIRE(beta >= 0.f && beta <= 1.f, "beta must lie in [0, 1] (got %g)", (double)beta);
  HK_REQUIRE(temperature > 0.f, "temperature must be positive (got %g)", (double)temperature);
  const bool grad = dinput != nullptr || dweight != nullptr;
  HK_REQUIRE(!grad || (dinput && dweight), "dinput and dweight are computed together");
  HK_REQUIRE(loss_out && s_input && s_weight && t_input && t_weight, "null pointer argument");
  const int es = fl_esize(dtype);
  HK_REQUIRE(aligned_to(s_input, es) && aligned_to(s_weight, es) && aligned_to(t_input, es) &&
                 aligned_to(t_weight, es) && (!grad || (aligned_to(dinput, es) && aligned_to(dweight, es))),
             "inputs, weights and gradients must be aligned to their element size");
  bool t_gather, t_wpad;
  const FlShape shp = fljsd_shape(BT, H, Ht, V, dtype, grad, chunk, labels != nullptr, s_input, s_weight, t_input,
                                  t_weight, &t_gather, &t_wpad);
  FlPlan lay;
  if (const int rc = fl_plan(shp, workspace_budget, &lay)) return rc;
  HK_REQUIRE(workspace && workspace_bytes >= lay.total, "workspace too small: need %zu bytes, got %zu", lay.total,
             workspace_bytes);
  HK_REQUIRE(aligned_to(workspace, 256), "workspace must be 256-byte aligned");
  const JsdExtra je = jsd_extra(BT, Ht, V, lay.C, es, t_gather, t_wpad);
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  char* ex = ws + lay.extra;
  int* n_valid = (int*)(ws + lay.nvalid);
  // with labels the ignored rows are compacted away (the engine's row map and live count)
  int* n_live = labels ? (int*)(ws + lay.nlive) : nullptr;
  int* rowmap = labels ? (int*)(ws + lay.rowmap) : nullptr;
  int* inv = labels ? (int*)(ws + lay.inv) : nullptr;
  float* lc = (float*)(ex + je.lc);
  int64_t* labc = (int64_t*)(ex + je.labc);
  const int64_t Htp = pad8(Ht), ldl = lay.ldl;

  auto run = [&](auto tag) -> int {
    using T = typename decltype(tag)::type;
    const T* Xs = (const T*)s_input;
    const T* Xt_in = (const T*)t_input;
    T* Lt = (T*)(ex + je.lt);
    T* Xtc = t_gather ? (T*)(ex + je.xtc) : nullptr;
    T* Wtp = t_wpad ? (T*)(ex + je.wtp) : nullptr;
    const T* Wt_k = t_wpad ? Wtp : (const T*)t_weight;
    const int64_t ldwt = t_wpad ? Htp : Ht;
    int rc = HK_OK;
    if (t_wpad) {
      rc = gather_rows<T>(Wtp, Htp, Htp, (const T*)t_weight, Ht, Ht, nullptr, nullptr, V, 0, V, st);
      if (rc) return rc;
    }
    if (labels && BT > 0) {
      // n counts the labels that are not ignore_index over all BT rows (fused_linear_jsd.py:137-141)
      rc = count_valid_launch(n_valid, labels, BT, ignore_index, 1, st);
      if (rc) return rc;
      rc = ce_compact_launch(rowmap, inv, n_live, labels, BT, ignore_index, st);
      if (rc) return rc;
      hipLaunchKernelGGL(gather_ce_kernel, dim3((unsigned)std::min<int64_t>(cdiv(BT, 256), 1024)), dim3(256), 0, st,
                         labc, nullptr, labels, nullptr, rowmap, n_live);
      rc = check_launch("gather_ce_kernel");
      if (rc) return rc;
    }
    // row step: the teacher logits of the chunk's rows (fused_linear_jsd.py:159-160), then the log-softmaxes,
    // JSD and, with gradients, the student dlogits over the student logits (:163-199); both chunk
    // buffers hold zeros past V, which the row kernel does not read
    auto jsd_step = [&](T* Ls, int64_t r0, int64_t cs) {
      const T* xt = Xt_in + r0 * Ht;
      int64_t ldx = Ht;
      if (t_gather) {
        int r = gather_rows<T>(Xtc, Htp, Htp, Xt_in, Ht, Ht, rowmap, n_live, BT, r0, cs, st);
        if (r) return r;
        xt = Xtc;
        ldx = Htp;
      }
      int r = launch_gemm<T>(xt, Wt_k, (int)cs, (int)V, (int)Htp, ldx, ldwt, EpiLogits<T>{Lt, ldl, 0.f}, st, n_live,
                             (int)r0);
      if (r) return r;
      return jsd_logits_launch(lc + r0, Ls, Lt, labels ? labc + r0 : nullptr, ignore_index, n_valid, BT, beta,
                               temperature, cs, V, ldl, grad ? 1 : 0, dtype, st, n_live, r0);
    };
    if (BT > 0) {
      rc = zero_cols<T>(Lt, ldl, V, ldl, lay.C, st);
      if (rc) return rc;
    }
    rc = chunked_lm_head<T>(Xs, (const T*)s_weight, BT, H, V, ws, lay, grad, (T*)dinput, (T*)dweight, n_live, rowmap,
                            0.f, jsd_step, st);
    if (rc) return rc;
    float* lrows = lc;
    if (labels) {
      // losses back in row order (ignored rows 0); ignored rows of dinput are zero
      float* rows_out = (float*)(ex + je.labc);  // the compacted labels are no longer needed
      rc = finish_rows<T>(grad ? (T*)dinput : nullptr, rows_out, lc, inv, BT, H, st);
      if (rc) return rc;
      lrows = rows_out;
    }
    // the rows already carry 1/n (:190)
    return scaled_sum_rows_launch(loss_out, lrows, BT, 1.0f, st);
  };
  return fl_dispatch(dtype, run);
}

// ---------------------------------------------------------------------------
// FusedLinear-GRPO
// ---------------------------------------------------------------------------

size_t hk_fused_linear_grpo_workspace_size(int64_t B, int64_t L, int64_t H, int64_t V, int64_t chunk,
                                           int64_t workspace_budget, int dtype, int with_grad, const void* hidden,
                                           const void* weight) {
  if (B <= 0 || L < 0 || B > (1LL << 31) || L > (1LL << 31) || !fl_dtype_ok(dtype) ||
      fl_check_dims(B * (L + 1), H, V) != HK_OK)
    return 0;
  FlPlan p;
  if (fl_plan(flgrpo_shape(B, L, H, V, dtype, with_grad != 0, chunk, hidden, weight), workspace_budget, &p) != HK_OK)
    return 0;
  return p.total;
}

int hk_fused_linear_grpo_plan(int64_t B, int64_t L, int64_t H, int64_t V, int64_t chunk, int64_t workspace_budget,
                              int dtype, int with_grad, const void* hidden, const void* weight, int64_t* info) {
  HK_REQUIRE(B > 0 && L >= 0 && B <= (1LL << 31) && L <= (1LL << 31), "invalid shape B=%lld L=%lld", (long long)B,
             (long long)L);
  HK_REQUIRE(fl_dtype_ok(dtype), "fused linear GRPO supports fp32, bf16 and fp16 (got %d)", dtype);
  if (const int rc = fl_check_dims(B * (L + 1), H, V)) return rc;
  HK_REQUIRE(info, "null pointer argument");
  FlPlan p;
  if (const int rc = fl_plan(flgrpo_shape(B, L, H, V, dtype, with_grad != 0, chunk, hidden, weight),
                             workspace_budget, &p))
    return rc;
  plan_info(p, info);
  return HK_OK;
}

int hk_fused_linear_grpo(float* loss_out, float* kl_out, float* clip_out, float* lse_rows, float* loss_rows,
                         float* kl_rows, float* clip_rows, void* dhidden, void* dweight, const void* hidden,
                         const void* weight, const int64_t* ids, int64_t ids_sB, int64_t ids_sL,
                         const float* advantages, const float* old_logp, int64_t old_sB, int64_t old_sL,
                         const float* ref_logp, int64_t ref_sB, int64_t ref_sL, const void* mask, int mask_dtype,
                         int64_t mask_sB, int64_t mask_sL, int64_t B, int64_t L, int64_t H, int64_t V,
                         float temperature, float beta, float eps_low, float eps_high, int dtype, int64_t chunk,
                         int64_t workspace_budget, void* workspace, size_t workspace_bytes, hk_stream_t stream) {
  HK_REQUIRE(fl_dtype_ok(dtype), "fused linear GRPO supports fp32, bf16 and fp16 (got %d)", dtype);
  const GrpoInputs in{ids,    ids_sB, ids_sL, advantages, old_logp, old_sB,      old_sL, ref_logp,
                      ref_sB, ref_sL, mask,   mask_dtype, mask_sB,  mask_sL,     B,      L,
                      V,      temperature,    beta,       eps_low,  eps_high};
  if (const int rc = grpo_check(in)) return rc;
  if (const int rc = fl_check_dims(B * (L + 1), H, V)) return rc;
  const bool grad = dhidden != nullptr || dweight != nullptr;
  HK_REQUIRE(!grad || (dhidden && dweight), "dhidden and dweight are computed together");
  HK_REQUIRE(loss_out && clip_out && hidden && weight && (L == 0 || (lse_rows && loss_rows && kl_rows && clip_rows)),
             "null pointer argument");
  const int es = fl_esize(dtype);
  HK_REQUIRE(aligned_to(hidden, es) && aligned_to(weight, es) &&
                 (!grad || (aligned_to(dhidden, es) && aligned_to(dweight, es))),
             "hidden, weight and gradients must be aligned to their element size");
  const int64_t BT = B * (L + 1);
  FlPlan lay;
  if (const int rc = fl_plan(flgrpo_shape(B, L, H, V, dtype, grad, chunk, hidden, weight), workspace_budget, &lay))
    return rc;
  HK_REQUIRE(workspace && workspace_bytes >= lay.total, "workspace too small: need %zu bytes, got %zu", lay.total,
             workspace_bytes);
  HK_REQUIRE(aligned_to(workspace, 256), "workspace must be 256-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  void* scratch = ws + lay.extra;
  int* n_live = (int*)(ws + lay.nlive);
  int* rowmap = (int*)(ws + lay.rowmap);
  int* inv = (int*)(ws + lay.inv);
  auto run = [&](auto tag) -> int {
    using T = typename decltype(tag)::type;
    int rc = grpo_prep_launch(in, scratch, st);
    if (rc) return rc;
    // the live positions (l < L, mask != 0), compacted: only their logits are computed
    rc = grpo_compact_launch(rowmap, inv, n_live, in, st);
    if (rc) return rc;
    // compacted row q of a chunk is position rowmap[r0 + q]: the GRPO row kernel
    // writes that token's results and, with gradients, its dlogits over the logits
    auto grpo_step = [&](T* Lg, int64_t r0, int64_t cs) {
      return grpo_rows_launch(grad ? (void*)Lg : nullptr, Lg, r0, cs, in, scratch, dtype, st, rowmap, n_live, lay.Vr,
                              lay.ldl);
    };
    rc = chunked_lm_head<T>((const T*)hidden, (const T*)weight, BT, H, V, ws, lay, grad, (T*)dhidden, (T*)dweight,
                            n_live, rowmap, -__builtin_huge_valf(), grpo_step, st);
    if (rc) return rc;
    // masked tokens and position L: zero rows of dhidden
    rc = finish_rows<T>(grad ? (T*)dhidden : nullptr, nullptr, nullptr, inv, BT, H, st);
    if (rc) return rc;
    return grpo_finalize_launch(in, scratch, loss_out, kl_out, clip_out, lse_rows, loss_rows, kl_rows, clip_rows,
                                st);
  };
  return fl_dispatch(dtype, run);
}

}  // extern "C"
