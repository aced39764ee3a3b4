// KL divergence and Jensen-Shannon divergence for gfx950: one pass over each
// row, HBM-bound, loss and gradient in the same pass where the reference does.
//
//   kl_div_fwd_kernel  per-row sum of t (log max(t, eps) - y), or e^t (t - y)
//                      for log targets (kernels/kl_div.py:40-67)
//   kl_div_bwd_kernel  dy = -t * s, or -e^t * s (kl_div.py:87-107), s per row
//                      or scalar, read on the device
//   jsd_kernel         per-row JSD(beta) loss / n and its gradient in X, with
//                      ignored rows zeroed (kernels/jsd.py:30-90)
//   jsd_logits_kernel  the FusedLinearJSD row step on a chunk of student and
//                      teacher logits: temperature log-softmax of both, JSD,
//                      and the student dlogits written over its logits
//                      (kernels/fused_linear_jsd.py:46-108,159-199)
//
// One block per row; each lane keeps 4 16-byte vectors per input in flight,
// and the row sums are block reductions.
#include "hk_common.h"
#include "hk_internal.h"
#include "../../include/hilda_kernel_amd.h"

#include <type_traits>

namespace hk {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kUnroll = 4;

template <bool LOGT>
__device__ __forceinline__ float kl_term(float y, float t, float eps) {
  if constexpr (LOGT) return exp_fast(t) * (t - y);
  else return t * (log_fast(fmaxf(t, eps)) - y);
}

// Visit row elements: f(width, x[], y[], first column) for VEC-wide packs
// (U packs of each row issued first), then width-1 calls for the tail. NT
// lanes share the row.
template <typename T, int VEC, int NT = kThreads, int U = kUnroll, class F>
__device__ __forceinline__ void row_pairs(const T* __restrict__ a, const T* __restrict__ b, int64_t cols, F&& f) {
  const int64_t nvec = VEC > 1 ? cols / VEC : 0;
  for (int64_t base = threadIdx.x; base < nvec; base += (int64_t)NT * U) {
    Pack<T, VEC> av[U], bv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = base + (int64_t)u * NT;
      if (i < nvec) {
        av[u] = load_pack<T, VEC>(a + i * VEC);
        bv[u] = load_pack<T, VEC>(b + i * VEC);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = base + (int64_t)u * NT;
      if (i < nvec) {
        float x[VEC], y[VEC];
        unpack(av[u], x);
        unpack(bv[u], y);
        f(std::integral_constant<int, VEC>{}, x, y, i * VEC);
      }
    }
  }
  for (int64_t c = nvec * VEC + threadIdx.x; c < cols; c += NT) {
    float x[VEC], y[VEC];
    x[0] = to_f32<T>(a[c]);
    y[0] = to_f32<T>(b[c]);
    f(std::integral_constant<int, 1>{}, x, y, c);
  }
}

template <typename T, int VEC, bool LOGT>
__global__ __launch_bounds__(kThreads) void kl_div_fwd_kernel(float* __restrict__ loss_rows,
                                                              const T* __restrict__ yp, const T* __restrict__ yt,
                                                              int64_t cols, int64_t ldp, int64_t ldt, float eps) {
  __shared__ float red[kWaves];
  const int64_t row = blockIdx.x;
  float acc = 0.f;
  row_pairs<T, VEC>(yp + row * ldp, yt + row * ldt, cols, [&](auto wc, const float* y, const float* t, int64_t) {
    constexpr int W = decltype(wc)::value;
#pragma unroll
    for (int e = 0; e < W; ++e) acc += kl_term<LOGT>(y[e], t[e], eps);
  });
  acc = block_sum<kWaves>(acc, red);
  if (threadIdx.x == 0) loss_rows[row] = acc;
}

// dy[row] = -(t or e^t) * g[row or 0] * factor
template <typename T, int VEC, bool LOGT>
__global__ __launch_bounds__(kThreads) void kl_div_bwd_kernel(T* __restrict__ dy, const T* __restrict__ yt,
                                                              const float* __restrict__ g, int per_row, float factor,
                                                              int64_t cols, int64_t ldt, int64_t ldo) {
  const int64_t row = blockIdx.x;
  const float s = -g[per_row ? row : 0] * factor;
  const T* t = yt + row * ldt;
  T* o = dy + row * ldo;
  const int64_t nvec = VEC > 1 ? cols / VEC : 0;
  for (int64_t base = threadIdx.x; base < nvec; base += (int64_t)kThreads * kUnroll) {
    Pack<T, VEC> tv[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + (int64_t)u * kThreads;
      if (i < nvec) tv[u] = load_pack<T, VEC>(t + i * VEC);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + (int64_t)u * kThreads;
      if (i < nvec) {
        float x[VEC];
        unpack(tv[u], x);
#pragma unroll
        for (int e = 0; e < VEC; ++e) x[e] = (LOGT ? exp_fast(x[e]) : x[e]) * s;
        store_pack<T, VEC>(o + i * VEC, pack<T, VEC>(x));
      }
    }
  }
  for (int64_t c = nvec * VEC + threadIdx.x; c < cols; c += kThreads) {
    const float x = to_f32<T>(t[c]);
    o[c] = from_f32<T>((LOGT ? exp_fast(x) : x) * s);
  }
}

// The same with one scalar s over a contiguous array of n packs (the usual
// 'batchmean' / 'sum' / 'mean' call): a flat walk, one 256-lane block a CU, U
// packs of a lane in flight, the shape of the fastest streaming copy (the
// per-row walk above runs this 1-read 1-write stream about 10% slower).
template <typename T, int VEC, bool LOGT, int U = 4>
__global__ __launch_bounds__(kThreads) void kl_div_bwd_flat_kernel(T* __restrict__ dy, const T* __restrict__ yt,
                                                                   const float* __restrict__ g, float factor,
                                                                   int64_t n) {
  const float s = -g[0] * factor;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  auto scale = [&](const Pack<T, VEC>& v) {
    float x[VEC];
    unpack(v, x);
#pragma unroll
    for (int e = 0; e < VEC; ++e) x[e] = (LOGT ? exp_fast(x[e]) : x[e]) * s;
    return pack<T, VEC>(x);
  };
  int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  for (; i + (U - 1) * stride < n; i += U * stride) {  // whole passes: loads unconditional
    Pack<T, VEC> v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = load_pack<T, VEC>(yt + (i + u * stride) * VEC);
#pragma unroll
    for (int u = 0; u < U; ++u) store_pack<T, VEC>(dy + (i + u * stride) * VEC, scale(v[u]));
  }
  for (; i < n; i += stride) store_pack<T, VEC>(dy + i * VEC, scale(load_pack<T, VEC>(yt + i * VEC)));
}

// JSD(beta) of teacher P = e^Y and student Q = e^X, both log-probabilities:
// MODE 0 (beta = 0): KL(P||Q) = sum P (Y - X),        dX = -P
// MODE 1 (beta = 1): KL(Q||P) = sum Q (X - Y),        dX = Q (X - Y + 1)
// MODE 2:            beta KL(P||M) + (1-beta) KL(Q||M), M = beta P + (1-beta) Q,
//                    dX = (1-beta) Q (X - log M)
// One element: adds its loss term to *acc and returns dX (unscaled).
template <int MODE>
__device__ __forceinline__ float jsd_elem(float x, float y, float beta, float* acc) {
  if constexpr (MODE == 0) {
    const float p = exp_fast(y);
    *acc += p * (y - x);
    return -p;
  } else if constexpr (MODE == 1) {
    const float q = exp_fast(x);
    *acc += q * (x - y);
    return q * (x - y + 1.0f);
  } else {
    const float q = exp_fast(x), p = exp_fast(y);
    const float lm = log_fast(beta * p + (1.0f - beta) * q);
    *acc += beta * p * (y - lm) + (1.0f - beta) * q * (x - lm);
    return (1.0f - beta) * q * (x - lm);
  }
}

// MODE 2 in base 2, the form jsd_kernel streams (fewer VALU slots an element:
// the kernel is close to VALU-bound at HBM speed): with x2 = x log2(e),
// y2 = y log2(e), t = (1-beta) q and lm2 = log2(beta p + t),
//   loss term = ln2 (t (x2 - lm2) + beta p (y2 - lm2)),
//   dX / n    = q (x2 - lm2) kg, kg = (1-beta) ln2 / n.
// Adds t (x2 - lm2) to *acc_t and p (y2 - lm2) to *acc_p; returns dX / n.
__device__ __forceinline__ float jsd_mix_elem2(float x, float y, float beta, float c1, float kg, float* acc_t,
                                               float* acc_p) {
  const float x2 = x * kLog2e, y2 = y * kLog2e;
  const float q = exp2_fast(x2), p = exp2_fast(y2);
  const float t = c1 * q;
  const float lm2 = log2_fast(fmaf(beta, p, t));
  const float dx2 = x2 - lm2, dy2 = y2 - lm2;
  *acc_t = fmaf(t, dx2, *acc_t);
  *acc_p = fmaf(p, dy2, *acc_p);
  return (q * kg) * dx2;
}

// Loss and dX are divided by n = max(n_valid, 1) (all rows without labels).
// One 256-lane workgroup a CU walks rows r, r + grid, ...: four waves a CU with
// 8 packs of each row in flight a lane; a workgroup per row (up to 32 waves a
// CU) measured 3.4% slower at [8192, 128256] bf16, as streaming copies slow
// down with more waves a CU.
constexpr int kJsdUnroll = 8;
template <typename T, int VEC, int MODE>
__global__ __launch_bounds__(kThreads) void jsd_kernel(float* __restrict__ loss_rows, T* __restrict__ dX,
                                                       const T* __restrict__ X, const T* __restrict__ Y,
                                                       const int64_t* __restrict__ labels, int64_t ignore_index,
                                                       const int* __restrict__ n_valid, int64_t rows, float beta,
                                                       int64_t cols, int64_t ldx, int64_t ldy, int64_t ldd) {
  __shared__ float red[kWaves];
  const float n = labels != nullptr ? (float)max(*n_valid, 1) : (float)rows;
  const float inv_n = 1.0f / n;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {  // uniform over the block
  T* d = dX + row * ldd;
  if (labels != nullptr && labels[row] == ignore_index) {
    for (int64_t c = threadIdx.x; c < cols; c += kThreads) d[c] = from_f32<T>(0.f);
    if (threadIdx.x == 0) loss_rows[row] = 0.f;
    continue;
  }
  float acc = 0.f, acc_p = 0.f;  // MODE 2: acc sums t (x2 - lm2), acc_p sums p (y2 - lm2)
  const float c1 = 1.0f - beta, kg = c1 * kLn2 * inv_n;
  row_pairs<T, VEC, kThreads, kJsdUnroll>(X + row * ldx, Y + row * ldy, cols,
                                          [&](auto wc, const float* x, const float* y, int64_t c0) {
    constexpr int W = decltype(wc)::value;
    float g[W];
#pragma unroll
    for (int e = 0; e < W; ++e) {
      if constexpr (MODE == 2) g[e] = jsd_mix_elem2(x[e], y[e], beta, c1, kg, &acc, &acc_p);
      else g[e] = jsd_elem<MODE>(x[e], y[e], beta, &acc) * inv_n;
    }
    if constexpr (W == VEC && VEC > 1) {
      store_pack<T, VEC>(d + c0, pack<T, VEC>(g));
    } else {
#pragma unroll
      for (int e = 0; e < W; ++e) d[c0 + e] = from_f32<T>(g[e]);
    }
  });
  if constexpr (MODE == 2) acc = kLn2 * fmaf(beta, acc_p, acc);
  acc = block_sum<kWaves>(acc, red);
  if (threadIdx.x == 0) loss_rows[row] = acc * inv_n;
  }
}

// (max, sum) pair of a log-sum-exp in base 2, merged over the block: every
// lane gets lse2 = m + log2(s). red holds 2 * NT/64 floats.
template <int NT>
__device__ __forceinline__ float block_lse2(float m, float s, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float om = __shfl_xor(m, o), os = __shfl_xor(s, o);
    const float M = fmaxf(m, om);
    s = M == -INFINITY ? 0.f : s * exp2_fast(m - M) + os * exp2_fast(om - M);
    m = M;
  }
  constexpr int NW = NT / kWave;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  if (lane == 0) {
    red[2 * wave] = m;
    red[2 * wave + 1] = s;
  }
  __syncthreads();
  float M = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) M = fmaxf(M, red[2 * i]);
  float S = 0.f;
#pragma unroll
  for (int i = 0; i < NW; ++i) S += red[2 * i + 1] * exp2_fast(red[2 * i] - M);
  __syncthreads();
  return M + log2_fast(S);
}

constexpr int kLogitLanes = 512;

// One row of student logits ls and teacher logits lt (temperature T): with
// x = ls/T - lse(ls/T) and y = lt/T - lse(lt/T), loss_rows[r] = JSD(beta)/n
// and, when WRITE, ls is overwritten with the student dlogits
// (dX - e^x sum(dX)) / T, dX = dJSD/dx / n (fused_linear_jsd.py:81-108), in
// the input dtype as the reference rounds them (:201).
// Three passes over the two rows: the two log-sum-exps, then the loss and
// sum(dX), then the dlogits (dX recomputed exactly as in the second pass).
// Rows labelled ignore_index get loss 0 and zero dlogits.
template <typename T, int VEC, int MODE, bool WRITE>
__global__ __launch_bounds__(kLogitLanes) void jsd_logits_kernel(float* __restrict__ loss_rows, T* __restrict__ ls,
                                                                 const T* __restrict__ lt,
                                                                 const int64_t* __restrict__ labels,
                                                                 int64_t ignore_index, const int* __restrict__ n_valid,
                                                                 int64_t n_all, float beta, float inv_temp,
                                                                 int64_t cols, int64_t ld,
                                                                 const int* __restrict__ rows_lim, int64_t rows_off) {
  constexpr int NW = kLogitLanes / kWave;
  __shared__ float red[2 * NW];
  const int64_t row = blockIdx.x;
  if (rows_lim && row >= (int64_t)*rows_lim - rows_off) return;  // past a device-side bound (uniform)
  T* s = ls + row * ld;
  const T* t = lt + row * ld;
  if (labels != nullptr && labels[row] == ignore_index) {
    if constexpr (WRITE)
      for (int64_t c = threadIdx.x; c < cols; c += kLogitLanes) s[c] = from_f32<T>(0.f);
    if (threadIdx.x == 0) loss_rows[row] = 0.f;
    return;
  }
  const float inv_n = 1.0f / (labels != nullptr ? (float)max(*n_valid, 1) : (float)n_all);
  const float c2 = inv_temp * kLog2e;
  float ms = -INFINITY, ss = 0.f, mt = -INFINITY, st = 0.f;
  row_pairs<T, VEC, kLogitLanes>(s, t, cols, [&](auto wc, const float* a, const float* b, int64_t) {
    constexpr int W = decltype(wc)::value;
    float pa = -INFINITY, pb = -INFINITY;
#pragma unroll
    for (int e = 0; e < W; ++e) {
      pa = fmaxf(pa, a[e] * c2);
      pb = fmaxf(pb, b[e] * c2);
    }
    const float na = fmaxf(ms, pa), nb = fmaxf(mt, pb);
    float sa = 0.f, sb = 0.f;
#pragma unroll
    for (int e = 0; e < W; ++e) {
      sa += exp2_fast(fmaf(a[e], c2, -na));
      sb += exp2_fast(fmaf(b[e], c2, -nb));
    }
    ss = ss * exp2_fast(ms - na) + sa;
    st = st * exp2_fast(mt - nb) + sb;
    ms = na;
    mt = nb;
  });
  // natural log-softmax: x = ls/T - lse_s
  const float lse_s = block_lse2<kLogitLanes>(ms, ss, red) * kLn2;
  const float lse_t = block_lse2<kLogitLanes>(mt, st, red) * kLn2;
  float acc = 0.f, sdx = 0.f;
  row_pairs<T, VEC, kLogitLanes>(s, t, cols, [&](auto wc, const float* a, const float* b, int64_t) {
    constexpr int W = decltype(wc)::value;
#pragma unroll
    for (int e = 0; e < W; ++e)
      sdx += jsd_elem<MODE>(fmaf(a[e], inv_temp, -lse_s), fmaf(b[e], inv_temp, -lse_t), beta, &acc);
  });
  acc = block_sum<NW>(acc, red);
  if (threadIdx.x == 0) loss_rows[row] = acc * inv_n;
  if constexpr (WRITE) {
    sdx = block_sum<NW>(sdx, red);
    row_pairs<T, VEC, kLogitLanes>(s, t, cols, [&](auto wc, const float* a, const float* b, int64_t c0) {
      constexpr int W = decltype(wc)::value;
      float o[W];
#pragma unroll
      for (int e = 0; e < W; ++e) {
        float dummy = 0.f;
        const float x = fmaf(a[e], inv_temp, -lse_s);
        const float dx = jsd_elem<MODE>(x, fmaf(b[e], inv_temp, -lse_t), beta, &dummy);
        o[e] = (dx - exp_fast(x) * sdx) * inv_n * inv_temp;
      }
      if constexpr (W == VEC && VEC > 1) {
        store_pack<T, VEC>(s + c0, pack<T, VEC>(o));
      } else {
#pragma unroll
        for (int e = 0; e < W; ++e) s[c0 + e] = from_f32<T>(o[e]);
      }
    });
  }
}

// out = scale * sum(v[0..n))
__global__ __launch_bounds__(1024) void scaled_sum_kernel(float* __restrict__ out, const float* __restrict__ v,
                                                          int64_t n, float scale) {
  __shared__ float red[16];
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += 1024) s += v[i];
  s = block_sum<16>(s, red);
  if (threadIdx.x == 0) *out = s * scale;
}

template <typename T> struct Tag { using type = T; };

template <typename F>
int dispatch_t(int dt, F&& f) {
  switch (dt) {
    case kF32: return f(Tag<float>{});
    case kF16: return f(Tag<_Float16>{});
    case kBF16: return f(Tag<__bf16>{});
  }
  set_error("invalid dtype code %d", dt);
  return HK_EINVAL;
}

// VEC-wide access is possible when every row start is 16-byte aligned
template <typename T>
bool rows_vec_ok(const void* p, int64_t ld) {
  return aligned_to(p, 16) && (ld * (int64_t)sizeof(T)) % 16 == 0;
}

int scaled_sum_launch(float* out, const float* v, int64_t n, float scale, hipStream_t st) {
  hipLaunchKernelGGL(scaled_sum_kernel, dim3(1), dim3(1024), 0, st, out, v, n, scale);
  return check_launch("scaled_sum_kernel");
}

}  // namespace

int jsd_logits_launch(float* loss_rows, void* ls, const void* lt, const int64_t* labels, int64_t ignore_index,
                      const int* n_valid, int64_t n_all, float beta, float temperature, int64_t rows, int64_t cols,
                      int64_t ld, int write, int dtype, hipStream_t st, const int* rows_lim, int64_t rows_off) {
  if (rows == 0) return HK_OK;
  return dispatch_t(dtype, [&](auto tag) -> int {
    using T = typename decltype(tag)::type;
    constexpr int V = 16 / sizeof(T);
    const bool vec = rows_vec_ok<T>(ls, ld) && rows_vec_ok<T>(lt, ld);
    const int mode = beta == 0.f ? 0 : beta == 1.f ? 1 : 2;
    auto go = [&](auto vc, auto mc, auto wc) {
      hipLaunchKernelGGL((jsd_logits_kernel<T, decltype(vc)::value, decltype(mc)::value, decltype(wc)::value>),
                         dim3((unsigned)rows), dim3(kLogitLanes), 0, st, loss_rows, (T*)ls, (const T*)lt, labels,
                         ignore_index, n_valid, n_all, beta, 1.0f / temperature, cols, ld, rows_lim, rows_off);
    };
    auto by_mode = [&](auto vc, auto wc) {
      if (mode == 0) go(vc, std::integral_constant<int, 0>{}, wc);
      else if (mode == 1) go(vc, std::integral_constant<int, 1>{}, wc);
      else go(vc, std::integral_constant<int, 2>{}, wc);
    };
    auto by_write = [&](auto vc) {
      if (write) by_mode(vc, std::true_type{});
      else by_mode(vc, std::false_type{});
    };
    if (vec) by_write(std::integral_constant<int, V>{});
    else by_write(std::integral_constant<int, 1>{});
    return check_launch("jsd_logits_kernel");
  });
}

int scaled_sum_rows_launch(float* out, const float* v, int64_t n, float scale, hipStream_t st) {
  return scaled_sum_launch(out, v, n, scale, st);
}

}  // namespace hk

using namespace hk;

extern "C" {

int hk_kl_div_fwd(float* loss_out, float* loss_rows, const void* y_pred, const void* y_true, int64_t rows,
                  int64_t cols, int64_t ld_pred, int64_t ld_true, int log_target, float eps, int reduction, int dtype,
                  hk_stream_t stream) {
  HK_REQUIRE(rows >= 0 && cols >= 0 && ld_pred >= cols && ld_true >= cols, "invalid shape");
  HK_REQUIRE(rows < (1LL << 31), "too many rows");
  HK_REQUIRE(reduction >= HK_REDUCTION_NONE && reduction <= HK_REDUCTION_BATCHMEAN, "invalid reduction %d",
             reduction);
  HK_REQUIRE(rows == 0 || (loss_rows && y_pred && y_true), "null pointer argument");
  hipStream_t st = (hipStream_t)stream;
  return dispatch_t(dtype, [&](auto tag) -> int {
    using T = typename decltype(tag)::type;
    constexpr int V = 16 / sizeof(T);
    if (rows > 0) {
      const bool vec = rows_vec_ok<T>(y_pred, ld_pred) && rows_vec_ok<T>(y_true, ld_true);
      auto go = [&](auto vc, auto lc) {
        hipLaunchKernelGGL((kl_div_fwd_kernel<T, decltype(vc)::value, decltype(lc)::value>), dim3((unsigned)rows),
                           dim3(kThreads), 0, st, loss_rows, (const T*)y_pred, (const T*)y_true, cols, ld_pred,
                           ld_true, eps);
      };
      using VV = std::integral_constant<int, V>;
      using V1 = std::integral_constant<int, 1>;
      using LT = std::true_type;
      using LF = std::false_type;
      if (vec) log_target ? go(VV{}, LT{}) : go(VV{}, LF{});
      else log_target ? go(V1{}, LT{}) : go(V1{}, LF{});
      const int rc = check_launch("kl_div_fwd_kernel");
      if (rc) return rc;
    }
    if (loss_out == nullptr || reduction == HK_REDUCTION_NONE) return HK_OK;
    float scale = 1.0f;  // kl_div.py:130-138
    if (reduction == HK_REDUCTION_MEAN) scale = 1.0f / (float)((double)rows * (double)cols);
    if (reduction == HK_REDUCTION_BATCHMEAN) scale = 1.0f / (float)rows;
    return scaled_sum_launch(loss_out, loss_rows, rows, scale, st);
  });
}

int hk_kl_div_bwd(void* dy_pred, const void* y_true, const float* g, int per_row, float factor, int64_t rows,
                  int64_t cols, int64_t ld_true, int64_t ld_out, int log_target, int dtype, hk_stream_t stream) {
  HK_REQUIRE(rows >= 0 && cols >= 0 && ld_true >= cols && ld_out >= cols, "invalid shape");
  HK_REQUIRE(rows < (1LL << 31), "too many rows");
  HK_REQUIRE(rows == 0 || cols == 0 || (dy_pred && y_true && g), "null pointer argument");
  hipStream_t st = (hipStream_t)stream;
  return dispatch_t(dtype, [&](auto tag) -> int {
    using T = typename decltype(tag)::type;
    constexpr int V = 16 / sizeof(T);
    if (rows == 0 || cols == 0) return HK_OK;
    const bool vec = rows_vec_ok<T>(y_true, ld_true) && rows_vec_ok<T>(dy_pred, ld_out);
    if (vec && !per_row && ld_true == cols && ld_out == cols) {  // one contiguous stream, one scale
      const int dev = current_device();
      const int64_t cus = dev >= 0 && cu_count(dev) > 0 ? cu_count(dev) : 256;
      const int64_t n = rows * cols / V;
      const dim3 grid((unsigned)std::max<int64_t>(1, std::min<int64_t>(cus, (n + kThreads - 1) / kThreads)));
      if (log_target)
        hipLaunchKernelGGL((kl_div_bwd_flat_kernel<T, V, true>), grid, dim3(kThreads), 0, st, (T*)dy_pred,
                           (const T*)y_true, g, factor, n);
      else
        hipLaunchKernelGGL((kl_div_bwd_flat_kernel<T, V, false>), grid, dim3(kThreads), 0, st, (T*)dy_pred,
                           (const T*)y_true, g, factor, n);
      return check_launch("kl_div_bwd_flat_kernel");
    }
    auto go = [&](auto vc, auto lc) {
      hipLaunchKernelGGL((kl_div_bwd_kernel<T, decltype(vc)::value, decltype(lc)::value>), dim3((unsigned)rows),
                         dim3(kThreads), 0, st, (T*)dy_pred, (const T*)y_true, g, per_row, factor, cols, ld_true,
                         ld_out);
    };
    using VV = std::integral_constant<int, V>;
    using V1 = std::integral_constant<int, 1>;
    if (vec) log_target ? go(VV{}, std::true_type{}) : go(VV{}, std::false_type{});
    else log_target ? go(V1{}, std::true_type{}) : go(V1{}, std::false_type{});
    return check_launch("kl_div_bwd_kernel");
  });
}

size_t hk_jsd_workspace_size(void) { return 256; }

int hk_jsd_fwd(float* loss_out, float* loss_rows, void* dX, const void* X, const void* Y, const int64_t* labels,
               int64_t ignore_index, float beta, int64_t rows, int64_t cols, int64_t ldx, int64_t ldy, int64_t ld_dx,
               int dtype, void* workspace, size_t workspace_bytes, hk_stream_t stream) {
  HK_REQUIRE(rows >= 0 && cols >= 0 && ldx >= cols && ldy >= cols && ld_dx >= cols, "invalid shape");
  HK_REQUIRE(rows < (1LL << 31), "too many rows");
  HK_REQUIRE(beta >= 0.f && beta <= 1.f, "beta must lie in [0, 1] (got %g)", (double)beta);
  HK_REQUIRE(rows == 0 || (loss_rows && dX && X && Y), "null pointer argument");
  HK_REQUIRE(labels == nullptr || (workspace && workspace_bytes >= hk_jsd_workspace_size() &&
                                   aligned_to(workspace, 4)),
             "labels need a workspace of hk_jsd_workspace_size() bytes");
  hipStream_t st = (hipStream_t)stream;
  return dispatch_t(dtype, [&](auto tag) -> int {
    using T = typename decltype(tag)::type;
    constexpr int V = 16 / sizeof(T);
    int* n_valid = labels ? (int*)workspace : nullptr;
    if (rows > 0) {
      if (labels) {
        const int rc = count_valid_launch(n_valid, labels, rows, ignore_index, 1, st);
        if (rc) return rc;
      }
      const bool vec = rows_vec_ok<T>(X, ldx) && rows_vec_ok<T>(Y, ldy) && rows_vec_ok<T>(dX, ld_dx);
      const int mode = beta == 0.f ? 0 : beta == 1.f ? 1 : 2;  // the reference branches on these values (jsd.py:67-87)
      auto go = [&](auto vc, auto mc) {
        const int dev = current_device();
        const int64_t cus = dev >= 0 && cu_count(dev) > 0 ? cu_count(dev) : 256;
        hipLaunchKernelGGL((jsd_kernel<T, decltype(vc)::value, decltype(mc)::value>), dim3((unsigned)std::min(rows, cus)),
                           dim3(kThreads), 0, st, loss_rows, (T*)dX, (const T*)X, (const T*)Y, labels, ignore_index,
                           n_valid, rows, beta, cols, ldx, ldy, ld_dx);
      };
      using VV = std::integral_constant<int, V>;
      using V1 = std::integral_constant<int, 1>;
      using M0 = std::integral_constant<int, 0>;
      using M1 = std::integral_constant<int, 1>;
      using M2 = std::integral_constant<int, 2>;
      if (vec) mode == 0 ? go(VV{}, M0{}) : mode == 1 ? go(VV{}, M1{}) : go(VV{}, M2{});
      else mode == 0 ? go(V1{}, M0{}) : mode == 1 ? go(V1{}, M1{}) : go(V1{}, M2{});
      const int rc = check_launch("jsd_kernel");
      if (rc) return rc;
    }
    if (loss_out == nullptr) return HK_OK;
    return scaled_sum_launch(loss_out, loss_rows, rows, 1.0f, st);
  });
}

}  // extern "C"
