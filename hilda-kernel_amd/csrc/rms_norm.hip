// RMSNorm and FusedAddRMSNorm, forward and backward, for gfx950.
//
// Design: one row is owned by a "row group" of `wpr` wavefronts (64*wpr
// lanes). Each lane keeps NCH packed vectors of VEC elements of the row in
// registers, so a row crosses HBM exactly once per pass; the sum of squares
// (forward) or sum(dy*w*x) (backward) is a wave64 butterfly reduction plus an
// LDS exchange between the row group's waves when wpr > 1. Vector j of lane l
// covers elements [(j*64*wpr + l)*VEC, +VEC), so every load instruction of a
// wave touches one contiguous 64*VEC*sizeof(T)-byte span (1 KiB for 16-byte
// vectors).
//
// Backward saves only rstd (the forward's [rows] fp32 output) and recomputes
// the normalised row. dW is reduced either by atomics into one [cols]
// accumulator or by per-row-group partial rows plus a reduction pass; the
// choice follows the reference rule "atomic when rows <= 8 * CU count"
// (rms_norm.py:325-326). dW is accumulated in fp64 (registers, partial rows
// and atomics alike): a sum over thousands of rows in fp32 drifts by ~1e-4,
// more than the 1e-5 fp32 tolerance allows, and the fp64 VALU rate is far
// above what this HBM-bound kernel needs.
#include "hk_common.h"
#include "../../include/hilda_kernel_amd.h"

#include <type_traits>
#include <utility>

namespace hk {
namespace {

constexpr int kMaxWaves = 16;  // 1024-thread blocks at most

// ------------------------------------------------------------------------
// forward
// ------------------------------------------------------------------------
template <typename T, typename W, int VEC, int NCH, bool ADD>
__global__ __launch_bounds__(1024) void rmsnorm_fwd_kernel(
    T* __restrict__ y, T* __restrict__ s_out, float* __restrict__ rstd_out, const T* __restrict__ x,
    const T* __restrict__ r, const W* __restrict__ w, int64_t rows, int cols, int64_t ld_x, int64_t ld_r,
    int64_t ld_y, int64_t ld_s, int wpr, float eps) {
  __shared__ float red[kMaxWaves];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int rpb = blockDim.x / (kWave * wpr);
  const int rib = wave / wpr;
  const int lr = (wave % wpr) * kWave + lane;
  const int gl = wpr * kWave;
  const int64_t row = (int64_t)blockIdx.x * rpb + rib;
  const bool valid = row < rows;

  Pack<T, VEC> xv[NCH];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int col = (j * gl + lr) * VEC;
    if (valid && col < cols) {
      xv[j] = load_pack<T, VEC>(x + row * ld_x + col);
      if constexpr (ADD) {
        // s = x + r, rounded to T exactly like the stored residual
        Pack<T, VEC> rv = load_pack<T, VEC>(r + row * ld_r + col);
        float a[VEC], b[VEC];
        unpack(xv[j], a);
        unpack(rv, b);
#pragma unroll
        for (int i = 0; i < VEC; ++i) a[i] += b[i];
        xv[j] = pack<T, VEC>(a);
        store_pack<T, VEC>(s_out + row * ld_s + col, xv[j]);
      }
      float a[VEC];
      unpack(xv[j], a);
#pragma unroll
      for (int i = 0; i < VEC; ++i) ss = fmaf(a[i], a[i], ss);
    }
  }
  ss = wave_sum(ss);
  if (wpr > 1) {
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    ss = 0.f;
    for (int i = 0; i < wpr; ++i) ss += red[rib * wpr + i];
  }
  const float rstd = __builtin_amdgcn_rsqf(ss / (float)cols + eps);
  if (valid && lr == 0) rstd_out[row] = rstd;

#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int col = (j * gl + lr) * VEC;
    if (valid && col < cols) {
      float a[VEC];
      unpack(xv[j], a);
      float wf[VEC];
      unpack(load_pack<W, VEC>(w + col), wf);
#pragma unroll
      for (int i = 0; i < VEC; ++i) a[i] = round_through<T>(a[i] * rstd) * wf[i];
      store_pack<T, VEC>(y + row * ld_y + col, pack<T, VEC>(a));
    }
  }
}

// ------------------------------------------------------------------------
// backward: dx per row, dW accumulated per row group in registers
// ------------------------------------------------------------------------
template <typename T, typename W, int VEC, int NCH, bool HAS_DS, bool ATOMIC>
__global__ __launch_bounds__(1024) void rmsnorm_bwd_kernel(
    T* __restrict__ dx, double* __restrict__ dw_ws, const T* __restrict__ dy, const T* __restrict__ ds,
    const T* __restrict__ x, const W* __restrict__ w, const float* __restrict__ rstd, int64_t rows, int cols,
    int64_t ld_dy, int64_t ld_ds, int64_t ld_x, int64_t ld_dx, int wpr) {
  __shared__ float red[kMaxWaves];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int rpb = blockDim.x / (kWave * wpr);
  const int rib = wave / wpr;
  const int lr = (wave % wpr) * kWave + lane;
  const int gl = wpr * kWave;
  const int64_t groups = (int64_t)gridDim.x * rpb;
  const float n = (float)cols;

  float wf[NCH][VEC];
  double acc[NCH][VEC];
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int col = (j * gl + lr) * VEC;
    float wv[VEC];
    if (col < cols) unpack(load_pack<W, VEC>(w + col), wv);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      wf[j][i] = col < cols ? wv[i] : 0.f;
      acc[j][i] = 0.0;
    }
  }

  // The trip count is uniform over the block so every thread meets the barriers.
  for (int64_t base = (int64_t)blockIdx.x * rpb; base < rows; base += groups) {
    const int64_t row = base + rib;
    const bool valid = row < rows;
    Pack<T, VEC> dyv[NCH], xv[NCH];
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int col = (j * gl + lr) * VEC;
      if (valid && col < cols) {
        dyv[j] = load_pack<T, VEC>(dy + row * ld_dy + col);
        xv[j] = load_pack<T, VEC>(x + row * ld_x + col);
        float g[VEC], a[VEC];
        unpack(dyv[j], g);
        unpack(xv[j], a);
#pragma unroll
        for (int i = 0; i < VEC; ++i) dot = fmaf(g[i] * wf[j][i], a[i], dot);
      }
    }
    dot = wave_sum(dot);
    if (wpr > 1) {
      if (lane == 0) red[wave] = dot;
      __syncthreads();
      dot = 0.f;
      for (int i = 0; i < wpr; ++i) dot += red[rib * wpr + i];
      __syncthreads();
    }
    if (!valid) continue;
    const float rs = rstd[row];
    const float c = rs * rs * rs * (dot / n);
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int col = (j * gl + lr) * VEC;
      if (col < cols) {
        float g[VEC], a[VEC], o[VEC];
        unpack(dyv[j], g);
        unpack(xv[j], a);
        if constexpr (HAS_DS) {
          Pack<T, VEC> dsv = load_pack<T, VEC>(ds + row * ld_ds + col);
          unpack(dsv, o);
        }
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          float v = rs * (g[i] * wf[j][i]) - c * a[i];
          if constexpr (HAS_DS) v += o[i];
          o[i] = v;
          acc[j][i] += (double)g[i] * (double)(a[i] * rs);
        }
        store_pack<T, VEC>(dx + row * ld_dx + col, pack<T, VEC>(o));
      }
    }
  }

  const int64_t g = (int64_t)blockIdx.x * rpb + rib;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int col = (j * gl + lr) * VEC;
    if (col < cols) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        if constexpr (ATOMIC) {
          if (g < rows) unsafeAtomicAdd(dw_ws + col + i, acc[j][i]);
        } else {
          dw_ws[g * cols + col + i] = acc[j][i];
        }
      }
    }
  }
}

__global__ __launch_bounds__(256) void fill_zero_f64(double* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0.0;
}

template <typename W>
__global__ __launch_bounds__(256) void cast_f64_kernel(W* __restrict__ out, const double* __restrict__ in, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    out[i] = from_f32<W>((float)in[i]);
}

// out[c] = sum_g part[g*cols + c]; block = 64 columns x 16 group slices
template <typename W>
__global__ __launch_bounds__(1024) void reduce_partial_kernel(W* __restrict__ out, const double* __restrict__ part,
                                                              int64_t groups, int cols) {
  __shared__ double red[16][65];
  const int c = threadIdx.x % 64, s = threadIdx.x / 64;
  const int col = blockIdx.x * 64 + c;
  double t = 0.0;
  if (col < cols)
    for (int64_t g = s; g < groups; g += 16) t += part[g * cols + col];
  red[s][c] = t;
  __syncthreads();
  if (s == 0 && col < cols) {
    double u = 0.0;
#pragma unroll
    for (int i = 0; i < 16; ++i) u += red[i][c];
    out[col] = from_f32<W>((float)u);
  }
}

// ------------------------------------------------------------------------
// host dispatch
// ------------------------------------------------------------------------
template <typename T> struct Tag { using type = T; };

// Call f(Tag<T>, Tag<W>) for the supported (x dtype, w dtype) pairs:
// w has the dtype of x, or is fp32 (the module's default parameter dtype).
template <typename F>
int dispatch_xw(int dt_x, int dt_w, F&& f) {
  if (dt_x == kF32 && dt_w == kF32) return f(Tag<float>{}, Tag<float>{});
  if (dt_x == kBF16 && dt_w == kBF16) return f(Tag<__bf16>{}, Tag<__bf16>{});
  if (dt_x == kBF16 && dt_w == kF32) return f(Tag<__bf16>{}, Tag<float>{});
  if (dt_x == kF16 && dt_w == kF16) return f(Tag<_Float16>{}, Tag<_Float16>{});
  if (dt_x == kF16 && dt_w == kF32) return f(Tag<_Float16>{}, Tag<float>{});
  set_error("unsupported dtype pair (x=%d, w=%d): w must match x or be fp32", dt_x, dt_w);
  return HK_EINVAL;
}

template <typename F>
int dispatch_nch(int nch, F&& f) {
  switch (nch) {
    case 1: return f(std::integral_constant<int, 1>{});
    case 2: return f(std::integral_constant<int, 2>{});
    case 4: return f(std::integral_constant<int, 4>{});
    case 8: return f(std::integral_constant<int, 8>{});
  }
  set_error("internal: bad NCH %d", nch);
  return HK_EINVAL;
}

int dtype_size(int dt) { return dt == kF32 ? 4 : 2; }
bool valid_dtype(int dt) { return dt == kF32 || dt == kF16 || dt == kBF16; }

struct Geom {
  int vec;     // elements per vector (16 bytes, or 1)
  int nch;     // vectors per lane (1, 2, 4, 8)
  int wpr;     // waves per row
  int rpb;     // rows per block
  int block;   // threads per block
};

// Pick the row-group geometry: full 16-byte vectors when every row start and
// the weight are 16-byte aligned, and the fewest waves per row that keep at
// most `max_elems` elements of one tensor per lane.
bool choose_geom(int64_t cols, int esize, bool vec_ok, int max_elems, Geom* g) {
  g->vec = vec_ok ? 16 / esize : 1;
  const int64_t nv = cols / g->vec;
  for (int wpr = 1; wpr <= kMaxWaves; wpr *= 2) {
    int64_t nch = cdiv(nv, (int64_t)kWave * wpr);
    int n = nch <= 1 ? 1 : nch <= 2 ? 2 : nch <= 4 ? 4 : nch <= 8 ? 8 : 16;
    if (n <= 8 && (n * g->vec <= max_elems || wpr == kMaxWaves)) {
      g->nch = n;
      g->wpr = wpr;
      g->block = wpr >= 4 ? wpr * kWave : 256;
      g->rpb = g->block / (wpr * kWave);
      return true;
    }
  }
  return false;
}

bool rows_aligned(const void* p, int64_t ld, int esize) {
  return aligned_to(p, 16) && ((ld * esize) % 16 == 0);
}

int fwd_impl(void* y, void* s, float* rstd, const void* x, const void* r, const void* w, int64_t rows,
             int64_t cols, int64_t ld_x, int64_t ld_r, int64_t ld_y, int64_t ld_s, int dt_x, int dt_w, float eps,
             hk_stream_t stream, bool add) {
  HK_REQUIRE(valid_dtype(dt_x) && valid_dtype(dt_w), "invalid dtype code (x=%d, w=%d)", dt_x, dt_w);
  HK_REQUIRE(rows >= 0 && cols > 0, "invalid shape rows=%lld cols=%lld", (long long)rows, (long long)cols);
  HK_REQUIRE(cols <= (1 << 30), "cols=%lld too large", (long long)cols);
  HK_REQUIRE(ld_x >= cols && ld_y >= cols && (!add || (ld_r >= cols && ld_s >= cols)),
             "row stride smaller than cols");
  HK_REQUIRE(y && rstd && x && w && (!add || (r && s)), "null pointer argument");
  if (rows == 0) return HK_OK;
  const int es = dtype_size(dt_x), ws = dtype_size(dt_w);
  const int vec = 16 / es;
  bool vec_ok = cols % vec == 0 && rows_aligned(x, ld_x, es) && rows_aligned(y, ld_y, es) &&
                aligned_to(w, (size_t)ws * vec);
  if (add) vec_ok = vec_ok && rows_aligned(r, ld_r, es) && rows_aligned(s, ld_s, es);
  Geom g;
  HK_REQUIRE(choose_geom(cols, es, vec_ok, 32, &g), "cols=%lld exceeds the supported row length",
             (long long)cols);
  const int64_t grid = cdiv(rows, g.rpb);
  hipStream_t st = (hipStream_t)stream;
  int rc = dispatch_xw(dt_x, dt_w, [&](auto tx, auto tw) {
    using T = typename decltype(tx)::type;
    using W = typename decltype(tw)::type;
    return dispatch_nch(g.nch, [&](auto nch_c) {
      constexpr int NCH = decltype(nch_c)::value;
      auto launch = [&](auto vec_c) {
        constexpr int VEC = decltype(vec_c)::value;
        if (add)
          hipLaunchKernelGGL((rmsnorm_fwd_kernel<T, W, VEC, NCH, true>), dim3(grid), dim3(g.block), 0, st,
                             (T*)y, (T*)s, rstd, (const T*)x, (const T*)r, (const W*)w, rows, (int)cols, ld_x,
                             ld_r, ld_y, ld_s, g.wpr, eps);
        else
          hipLaunchKernelGGL((rmsnorm_fwd_kernel<T, W, VEC, NCH, false>), dim3(grid), dim3(g.block), 0, st,
                             (T*)y, (T*)nullptr, rstd, (const T*)x, (const T*)nullptr, (const W*)w, rows,
                             (int)cols, ld_x, ld_x, ld_y, ld_y, g.wpr, eps);
        return check_launch("rmsnorm_fwd_kernel");
      };
      if (g.vec == 1) return launch(std::integral_constant<int, 1>{});
      return launch(std::integral_constant<int, 16 / sizeof(T)>{});
    });
  });
  return rc;
}

// Geometry and grid of the backward launch, shared by the workspace query.
struct BwdPlan {
  Geom g;
  int64_t grid;
  bool atomic;
  int64_t ws_elems;  // fp64 accumulators
};

bool plan_bwd(int64_t rows, int64_t cols, int es, bool vec_ok, int dw_mode, int cu, BwdPlan* p) {
  if (!choose_geom(cols, es, vec_ok, 16, &p->g)) return false;
  const int64_t needed = cdiv(rows, p->g.rpb);
  // enough resident waves per CU to cover HBM latency, but few partial rows
  const int64_t target = (int64_t)(cu > 0 ? cu : 256) * (p->g.block >= 1024 ? 2 : p->g.block >= 512 ? 4 : 8) / 2;
  p->grid = needed < target ? needed : target;
  if (p->grid < 1) p->grid = 1;
  p->atomic = dw_mode == HK_DW_ATOMIC || (dw_mode == HK_DW_AUTO && rows <= 8LL * (cu > 0 ? cu : 256));
  p->ws_elems = p->atomic ? cols : p->grid * p->g.rpb * cols;
  return true;
}

int bwd_impl(void* dx, void* dw, const void* dy, const void* ds, const void* x, const void* w, const float* rstd,
             int64_t rows, int64_t cols, int64_t ld_dy, int64_t ld_ds, int64_t ld_x, int64_t ld_dx, int dt_x,
             int dt_w, int dw_mode, void* workspace, size_t ws_bytes, hk_stream_t stream) {
  HK_REQUIRE(valid_dtype(dt_x) && valid_dtype(dt_w), "invalid dtype code (x=%d, w=%d)", dt_x, dt_w);
  HK_REQUIRE(rows >= 0 && cols > 0, "invalid shape rows=%lld cols=%lld", (long long)rows, (long long)cols);
  HK_REQUIRE(cols <= (1 << 30), "cols=%lld too large", (long long)cols);
  HK_REQUIRE(ld_dy >= cols && ld_x >= cols && ld_dx >= cols && (!ds || ld_ds >= cols),
             "row stride smaller than cols");
  HK_REQUIRE(dw_mode == HK_DW_AUTO || dw_mode == HK_DW_ATOMIC || dw_mode == HK_DW_PARTIAL, "invalid dw_mode %d",
             dw_mode);
  HK_REQUIRE(dx && dw && dy && x && w && rstd, "null pointer argument");
  const int es = dtype_size(dt_x), wsz = dtype_size(dt_w);
  const int vec = 16 / es;
  bool vec_ok = cols % vec == 0 && rows_aligned(dy, ld_dy, es) && rows_aligned(x, ld_x, es) &&
                rows_aligned(dx, ld_dx, es) && aligned_to(w, (size_t)wsz * vec);
  if (ds) vec_ok = vec_ok && rows_aligned(ds, ld_ds, es);
  const int dev = current_device();
  if (dev < 0) return (int)hipErrorNoDevice;
  BwdPlan p;
  HK_REQUIRE(plan_bwd(rows, cols, es, vec_ok, dw_mode, cu_count(dev), &p),
             "cols=%lld exceeds the supported row length", (long long)cols);
  HK_REQUIRE(workspace != nullptr && ws_bytes >= (size_t)p.ws_elems * sizeof(double),
             "workspace too small: need %zu bytes, got %zu", (size_t)p.ws_elems * sizeof(double), ws_bytes);
  HK_REQUIRE(aligned_to(workspace, 16), "workspace must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  double* wsf = (double*)workspace;

  return dispatch_xw(dt_x, dt_w, [&](auto tx, auto tw) {
    using T = typename decltype(tx)::type;
    using W = typename decltype(tw)::type;
    if (p.atomic) {
      hipLaunchKernelGGL(fill_zero_f64, dim3((unsigned)cdiv(cols, 256)), dim3(256), 0, st, wsf, cols);
      int rc = check_launch("fill_zero_f64");
      if (rc) return rc;
    }
    if (rows > 0) {
      int rc = dispatch_nch(p.g.nch, [&](auto nch_c) {
        constexpr int NCH = decltype(nch_c)::value;
        auto launch = [&](auto vec_c) {
          constexpr int VEC = decltype(vec_c)::value;
#define HK_BWD_LAUNCH(HDS, AT)                                                                               \
  hipLaunchKernelGGL((rmsnorm_bwd_kernel<T, W, VEC, NCH, HDS, AT>), dim3(p.grid), dim3(p.g.block), 0, st,     \
                     (T*)dx, wsf, (const T*)dy, (const T*)ds, (const T*)x, (const W*)w, rstd, rows, (int)cols, \
                     ld_dy, ld_ds, ld_x, ld_dx, p.g.wpr)
          if (ds) {
            if (p.atomic) HK_BWD_LAUNCH(true, true); else HK_BWD_LAUNCH(true, false);
          } else {
            if (p.atomic) HK_BWD_LAUNCH(false, true); else HK_BWD_LAUNCH(false, false);
          }
#undef HK_BWD_LAUNCH
          return check_launch("rmsnorm_bwd_kernel");
        };
        if (p.g.vec == 1) return launch(std::integral_constant<int, 1>{});
        return launch(std::integral_constant<int, 16 / sizeof(T)>{});
      });
      if (rc) return rc;
    }
    if (p.atomic) {
      hipLaunchKernelGGL((cast_f64_kernel<W>), dim3((unsigned)cdiv(cols, 256)), dim3(256), 0, st, (W*)dw, wsf,
                         cols);
      return check_launch("cast_f64_kernel");
    }
    hipLaunchKernelGGL((reduce_partial_kernel<W>), dim3((unsigned)cdiv(cols, 64)), dim3(1024), 0, st, (W*)dw, wsf,
                       p.grid * p.g.rpb, (int)cols);
    return check_launch("reduce_partial_kernel");
  });
}

}  // namespace
}  // namespace hk

using namespace hk;

extern "C" {

int hk_rms_norm_fwd(void* y, float* rstd, const void* x, const void* w, int64_t rows, int64_t cols, int64_t ld_x,
                    int64_t ld_y, int dtype_x, int dtype_w, float eps, hk_stream_t stream) {
  return fwd_impl(y, nullptr, rstd, x, nullptr, w, rows, cols, ld_x, ld_x, ld_y, ld_y, dtype_x, dtype_w, eps, stream,
                  false);
}

int hk_fused_add_rms_norm_fwd(void* y, void* s, float* rstd, const void* x, const void* r, const void* w,
                              int64_t rows, int64_t cols, int64_t ld, int dtype_x, int dtype_w, float eps,
                              hk_stream_t stream) {
  return fwd_impl(y, s, rstd, x, r, w, rows, cols, ld, ld, ld, ld, dtype_x, dtype_w, eps, stream, true);
}

size_t hk_rms_norm_bwd_workspace_size(int64_t rows, int64_t cols, int dtype_x, int dtype_w, int dw_mode,
                                      int device) {
  (void)dtype_w;
  if (rows < 0 || cols <= 0 || !valid_dtype(dtype_x)) return 0;
  BwdPlan p;
  // The vector width can only shrink the geometry's group count, so plan
  // with full vectors and the widest alternative and take the larger.
  size_t best = 0;
  for (int v = 0; v < 2; ++v) {
    if (plan_bwd(rows, cols, dtype_size(dtype_x), v == 0, dw_mode, cu_count(device), &p)) {
      size_t b = (size_t)p.ws_elems * sizeof(double);
      if (b > best) best = b;
    }
  }
  return best;
}

int hk_rms_norm_bwd(void* dx, void* dw, const void* dy, const void* x, const void* w, const float* rstd, int64_t rows,
                    int64_t cols, int64_t ld_dy, int64_t ld_x, int64_t ld_dx, int dtype_x, int dtype_w, int dw_mode,
                    void* workspace, size_t workspace_bytes, hk_stream_t stream) {
  return bwd_impl(dx, dw, dy, nullptr, x, w, rstd, rows, cols, ld_dy, ld_dy, ld_x, ld_dx, dtype_x, dtype_w, dw_mode,
                  workspace, workspace_bytes, stream);
}

int hk_fused_add_rms_norm_bwd(void* dx, void* dw, const void* dy, const void* ds_out, const void* s, const void* w,
                              const float* rstd, int64_t rows, int64_t cols, int64_t ld, int dtype_x, int dtype_w,
                              int dw_mode, void* workspace, size_t workspace_bytes, hk_stream_t stream) {
  return bwd_impl(dx, dw, dy, ds_out, s, w, rstd, rows, cols, ld, ld, ld, ld, dtype_x, dtype_w, dw_mode, workspace,
                  workspace_bytes, stream);
}

}  // extern "C"
