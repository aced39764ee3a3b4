// RMSNorm and FusedAddRMSNorm, forward and backward, for gfx950.
//
// Design: one row is owned by a "row group" of `wpr` wavefronts (64*wpr
// lanes). Each lane keeps NCH packed vectors of VEC elements of the row in
// registers, so a row crosses HBM exactly once per pass; the sum of squares
// (forward) or sum(dy*w*x) (backward) is a wave64 butterfly reduction plus an
// LDS exchange between the row group's waves when wpr > 1. Vector j of lane l
// covers elements [(j*64*wpr + l)*VEC, +VEC), so every load instruction of a
// wave touches one contiguous 64*VEC*sizeof(T)-byte span (1 KiB for 16-byte
// vectors). The weight is loaded together with the row, so a row costs one
// memory latency, not two.
//
// Backward saves only rstd (the forward's [rows] fp32 output) and recomputes
// the normalised row. Each of the G row groups walks rows g, g + G, g + 2G, ...
// (so at any moment the whole GPU reads one contiguous window of G rows, as
// the forward's one-row-a-block grid does; runs of consecutive rows per group
// measured 10% slower at C2's bf16 [8192, 4096]), accumulating its dW
// contribution in registers: fp32 for 16-bit inputs, fp64 for fp32 inputs (a
// sum over thousands of rows in fp32 drifts by ~1e-4, more than the 1e-5 fp32
// tolerance allows). For 16-bit inputs a 1024-lane block holds several groups
// (4 at H = 4096), one block a CU, and their accumulators are summed in LDS in
// a fixed order; fp32 inputs run up to 512 lanes a block, two blocks a CU. Each
// block's sum goes either into one fp32 partial row (a group's rows round
// once), summed in fp64 by a separate pass, or into fp64 atomics on one [cols]
// accumulator. HK_DW_AUTO always takes the partial rows. The
// reference switches to atomics when rows <= 8 * CU count (rms_norm.py:325-326);
// here the groups' device-scope fp64 atomics on the one row measured 1.7-9x
// slower than the partial rows at every size tried (16 to 4096 rows, H 1024 to
// 8192), so atomics run only when HK_DW_ATOMIC asks for them.
#include "hk_common.h"
#include "colsum.h"
#include "../../include/hilda_kernel_amd.h"

#include <algorithm>
#include <mutex>
#include <type_traits>
#include <utility>

namespace hk {
namespace {

constexpr int kMaxWaves = 16;  // 1024-thread blocks at most

// ------------------------------------------------------------------------
// forward
// ------------------------------------------------------------------------
template <typename T, typename W, int VEC, int NCH, bool ADD, int LB>
__global__ __launch_bounds__(LB) void rmsnorm_fwd_kernel(
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
  Pack<W, VEC> wv[NCH];
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int col = (j * gl + lr) * VEC;
    if (col < cols) wv[j] = load_pack<W, VEC>(w + col);
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
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int col = (j * gl + lr) * VEC;
    if (valid && col < cols) {
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
      unpack(wv[j], wf);
#pragma unroll
      for (int i = 0; i < VEC; ++i) a[i] = round_through<T>(a[i] * rstd) * wf[i];
      store_pack<T, VEC>(y + row * ld_y + col, pack<T, VEC>(a));
    }
  }
}

// ------------------------------------------------------------------------
// backward: dx per row; dW accumulated per row group over rows g, g + G, ...
// ------------------------------------------------------------------------
template <typename T, typename W, typename A, int VEC, int NCH, bool HAS_DS, int LB>
__global__ __launch_bounds__(LB) void rmsnorm_bwd_kernel(
    T* __restrict__ dx, void* __restrict__ dw_ws, int atomic,
    const T* __restrict__ dy, const T* __restrict__ ds, const T* __restrict__ x, const W* __restrict__ w,
    const float* __restrict__ rstd, int64_t rows, int cols, int64_t ld_dy, int64_t ld_ds, int64_t ld_x,
    int64_t ld_dx, int wpr, int64_t rows_per_group) {
  __shared__ float red[2][kMaxWaves];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int rpb = blockDim.x / (kWave * wpr);
  const int rib = wave / wpr;
  const int lr = (wave % wpr) * kWave + lane;
  const int gl = wpr * kWave;
  const int64_t group = (int64_t)blockIdx.x * rpb + rib;
  const int64_t ngroups = (int64_t)gridDim.x * rpb;
  const float inv_n = 1.f / (float)cols;
  Pack<W, VEC> wv[NCH];
  A acc[NCH][VEC];
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int col = (j * gl + lr) * VEC;
    if (col < cols) wv[j] = load_pack<W, VEC>(w + col);
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[j][i] = A(0);
  }

  // The trip count is uniform over the block so every thread meets the barriers.
#pragma unroll 1
  for (int64_t t = 0; t < rows_per_group; ++t) {
    const int64_t row = group + t * ngroups;
    const bool valid = row < rows;
    const int64_t rr = valid ? row : rows - 1;  // loads stay unconditional
    const float rs = rstd[rr];
    Pack<T, VEC> gv[NCH], xv[NCH], dv[NCH];
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int col = (j * gl + lr) * VEC;
      if (col < cols) {
        gv[j] = load_pack<T, VEC>(dy + rr * ld_dy + col);
        xv[j] = load_pack<T, VEC>(x + rr * ld_x + col);
        if constexpr (HAS_DS) dv[j] = load_pack<T, VEC>(ds + rr * ld_ds + col);
      }
    }
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int col = (j * gl + lr) * VEC;
      if (col < cols) {
        float g[VEC], a[VEC], wf[VEC];
        unpack(gv[j], g);
        unpack(xv[j], a);
        unpack(wv[j], wf);
#pragma unroll
        for (int i = 0; i < VEC; ++i) dot = fmaf(g[i] * wf[i], a[i], dot);
      }
    }
    dot = wave_sum(dot);
    if (wpr > 1) {
      const int b = (int)(t & 1);  // two slots: no second barrier before the next row's write
      if (lane == 0) red[b][wave] = dot;
      __syncthreads();
      dot = 0.f;
      for (int i = 0; i < wpr; ++i) dot += red[b][rib * wpr + i];
    }
    // unpack again below rather than keep the floats live across the barrier
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      make_opaque(gv[j]);
      make_opaque(xv[j]);
      make_opaque(wv[j]);
    }
    const float c = rs * rs * rs * (dot * inv_n);
    const float vf = valid ? 1.f : 0.f;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int col = (j * gl + lr) * VEC;
      if (col < cols) {
        float g[VEC], a[VEC], wf[VEC], o[VEC];
        unpack(gv[j], g);
        unpack(xv[j], a);
        unpack(wv[j], wf);
        if constexpr (HAS_DS) unpack(dv[j], o);
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          float v = rs * (g[i] * wf[i]) - c * a[i];
          if constexpr (HAS_DS) v += o[i];
          o[i] = v;
          acc[j][i] += A(g[i] * vf) * A(a[i] * rs);
        }
        if (valid) store_pack<T, VEC>(dx + row * ld_dx + col, pack<T, VEC>(o));
      }
    }
  }

  if (rpb == 1) {
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int col = (j * gl + lr) * VEC;
      if (col < cols) {
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          if (atomic) {
            if (group < rows) unsafeAtomicAdd(static_cast<double*>(dw_ws) + col + i, (double)acc[j][i]);
          } else {
            static_cast<float*>(dw_ws)[group * cols + col + i] = (float)acc[j][i];
          }
        }
      }
    }
    return;
  }
  // Several row groups a block: their accumulators are summed in LDS, group by
  // group in a fixed order, and the block writes one partial row (or adds it
  // atomically), so the dW pass reads rpb times fewer rows.
  extern __shared__ __align__(16) unsigned char dyn_lds[];
  A* buf = reinterpret_cast<A*>(dyn_lds);
  for (int r = 0; r < rpb; ++r) {
    if (rib == r) {
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        const int col = (j * gl + lr) * VEC;
        if (col < cols) {
#pragma unroll
          for (int i = 0; i < VEC; ++i) buf[col + i] = r == 0 ? acc[j][i] : buf[col + i] + acc[j][i];
        }
      }
    }
    __syncthreads();
  }
  const bool any_row = (int64_t)blockIdx.x * rpb < rows;
  for (int c = threadIdx.x; c < cols; c += blockDim.x) {
    if (atomic) {
      if (any_row) unsafeAtomicAdd(static_cast<double*>(dw_ws) + c, (double)buf[c]);
    } else {
      static_cast<float*>(dw_ws)[(int64_t)blockIdx.x * cols + c] = (float)buf[c];
    }
  }
}

// ------------------------------------------------------------------------
// rows too long to hold in registers (more than 16 waves x 8 16-byte vectors:
// fp32 rows over 32768 columns, 16-bit over 65536)
// ------------------------------------------------------------------------
constexpr int kStreamLanes = 1024;

// Forward: one 1024-lane block per row, two passes over the row (the sum of
// squares, then the normalised row; with ADD the first pass stores s = x + r
// and the second reads s back). The arithmetic is the register form's.
template <typename T, typename W, int VEC, bool ADD>
__global__ __launch_bounds__(kStreamLanes) void rmsnorm_fwd_stream_kernel(
    T* __restrict__ y, T* s_out, float* __restrict__ rstd_out, const T* __restrict__ x, const T* __restrict__ r,
    const W* __restrict__ w, int cols, int64_t ld_x, int64_t ld_r, int64_t ld_y, int64_t ld_s, float eps) {
  __shared__ float red[kStreamLanes / kWave];
  const int64_t row = blockIdx.x;
  float ss = 0.f;
  for (int col = (int)threadIdx.x * VEC; col < cols; col += kStreamLanes * VEC) {
    Pack<T, VEC> xv = load_pack<T, VEC>(x + row * ld_x + col);
    float a[VEC];
    unpack(xv, a);
    if constexpr (ADD) {
      float b[VEC];
      unpack(load_pack<T, VEC>(r + row * ld_r + col), b);
#pragma unroll
      for (int i = 0; i < VEC; ++i) a[i] += b[i];
      xv = pack<T, VEC>(a);
      store_pack<T, VEC>(s_out + row * ld_s + col, xv);
      unpack(xv, a);  // s as stored
    }
#pragma unroll
    for (int i = 0; i < VEC; ++i) ss = fmaf(a[i], a[i], ss);
  }
  ss = block_sum<kStreamLanes / kWave>(ss, red);
  const float rstd = __builtin_amdgcn_rsqf(ss / (float)cols + eps);
  if (threadIdx.x == 0) rstd_out[row] = rstd;
  for (int col = (int)threadIdx.x * VEC; col < cols; col += kStreamLanes * VEC) {
    // with ADD: this thread's own stores of the first pass
    float a[VEC], wf[VEC];
    unpack(load_pack<T, VEC>(ADD ? s_out + row * ld_s + col : x + row * ld_x + col), a);
    unpack(load_pack<W, VEC>(w + col), wf);
#pragma unroll
    for (int i = 0; i < VEC; ++i) a[i] = round_through<T>(a[i] * rstd) * wf[i];
    store_pack<T, VEC>(y + row * ld_y + col, pack<T, VEC>(a));
  }
}

// Backward, first kernel: per row c = rstd^3 * <dy * w, x> / n (one
// 1024-lane block per row).
template <typename T, typename W, int VEC>
__global__ __launch_bounds__(kStreamLanes) void rmsnorm_bwd_dot_kernel(float* __restrict__ coef,
                                                                       const T* __restrict__ dy,
                                                                       const T* __restrict__ x,
                                                                       const W* __restrict__ w,
                                                                       const float* __restrict__ rstd, int cols,
                                                                       int64_t ld_dy, int64_t ld_x) {
  __shared__ float red[kStreamLanes / kWave];
  const int64_t row = blockIdx.x;
  float dot = 0.f;
  for (int col = (int)threadIdx.x * VEC; col < cols; col += kStreamLanes * VEC) {
    float g[VEC], a[VEC], wf[VEC];
    unpack(load_pack<T, VEC>(dy + row * ld_dy + col), g);
    unpack(load_pack<T, VEC>(x + row * ld_x + col), a);
    unpack(load_pack<W, VEC>(w + col), wf);
#pragma unroll
    for (int i = 0; i < VEC; ++i) dot = fmaf(g[i] * wf[i], a[i], dot);
  }
  dot = block_sum<kStreamLanes / kWave>(dot, red);
  if (threadIdx.x == 0) {
    const float rs = rstd[row];
    coef[row] = rs * rs * rs * (dot / (float)cols);
  }
}

// Backward, second kernel: block b takes column slice b % nslice (256 lanes x
// kSliceVecs vectors) of the rows of group b / nslice, writes dX there and
// sums its dW part over those rows in registers (A: fp64 for fp32 inputs),
// one fp32 partial row slice per group.
constexpr int kSliceLanes = 256, kSliceVecs = 4;
template <typename T, typename W, typename A, int VEC, bool HAS_DS>
__global__ __launch_bounds__(kSliceLanes) void rmsnorm_bwd_cols_kernel(
    T* __restrict__ dx, float* __restrict__ part, const T* __restrict__ dy, const T* __restrict__ ds,
    const T* __restrict__ x, const W* __restrict__ w, const float* __restrict__ rstd,
    const float* __restrict__ coef, int64_t rows, int cols, int64_t ld_dy, int64_t ld_ds, int64_t ld_x,
    int64_t ld_dx, int nslice, int64_t rows_per_group) {
  const int64_t group = blockIdx.x / nslice;
  const int c0 = (int)(blockIdx.x % nslice) * kSliceLanes * VEC * kSliceVecs;
  A acc[kSliceVecs][VEC];
  float wf[kSliceVecs][VEC];
#pragma unroll
  for (int j = 0; j < kSliceVecs; ++j) {
    const int col = c0 + (j * kSliceLanes + (int)threadIdx.x) * VEC;
    if (col < cols) unpack(load_pack<W, VEC>(w + col), wf[j]);
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[j][i] = A(0);
  }
  const int64_t r0 = group * rows_per_group, r1 = min(rows, r0 + rows_per_group);
  for (int64_t row = r0; row < r1; ++row) {
    const float rs = rstd[row], c = coef[row];
#pragma unroll
    for (int j = 0; j < kSliceVecs; ++j) {
      const int col = c0 + (j * kSliceLanes + (int)threadIdx.x) * VEC;
      if (col < cols) {
        float g[VEC], a[VEC], o[VEC];
        unpack(load_pack<T, VEC>(dy + row * ld_dy + col), g);
        unpack(load_pack<T, VEC>(x + row * ld_x + col), a);
        if constexpr (HAS_DS) unpack(load_pack<T, VEC>(ds + row * ld_ds + col), o);
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          float v = rs * (g[i] * wf[j][i]) - c * a[i];
          if constexpr (HAS_DS) v += o[i];
          o[i] = v;
          acc[j][i] += A(g[i]) * A(a[i] * rs);
        }
        store_pack<T, VEC>(dx + row * ld_dx + col, pack<T, VEC>(o));
      }
    }
  }
#pragma unroll
  for (int j = 0; j < kSliceVecs; ++j) {
    const int col = c0 + (j * kSliceLanes + (int)threadIdx.x) * VEC;
    if (col < cols) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) part[group * cols + col + i] = (float)acc[j][i];
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
// most 16 elements of one tensor per lane (4 waves of 2 vectors for a
// 4096-wide bf16 row: measured fastest for both passes).
bool choose_geom(int64_t cols, int esize, bool vec_ok, Geom* g) {
  constexpr int kMaxElems = 16;
  g->vec = vec_ok ? 16 / esize : 1;
  const int64_t nv = cdiv(cols, (int64_t)g->vec);
  for (int wpr = 1; wpr <= kMaxWaves; wpr *= 2) {
    int64_t nch = cdiv(nv, (int64_t)kWave * wpr);
    int n = nch <= 1 ? 1 : nch <= 2 ? 2 : nch <= 4 ? 4 : nch <= 8 ? 8 : 16;
    if (n <= 8 && (n * g->vec <= kMaxElems || wpr == kMaxWaves)) {
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

// f(integral_constant<LB>) with LB the launch bound matching the block size
template <typename F>
int dispatch_lb(int block, F&& f) {
  if (block <= 256) return f(std::integral_constant<int, 256>{});
  return f(std::integral_constant<int, 1024>{});
}
template <typename F>
int dispatch_lb_bwd(int block, F&& f) {
  if (block <= 256) return f(std::integral_constant<int, 256>{});
  if (block <= 512) return f(std::integral_constant<int, 512>{});
  return f(std::integral_constant<int, 1024>{});
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
  hipStream_t st = (hipStream_t)stream;
  if (!choose_geom(cols, es, vec_ok, &g)) {
    // rows too long for the register form: two streaming passes per row
    return dispatch_xw(dt_x, dt_w, [&](auto tx, auto tw) {
      using T = typename decltype(tx)::type;
      using W = typename decltype(tw)::type;
      auto launch = [&](auto vec_c) {
        constexpr int VEC = decltype(vec_c)::value;
        if (add)
          hipLaunchKernelGGL((rmsnorm_fwd_stream_kernel<T, W, VEC, true>), dim3((unsigned)rows), dim3(kStreamLanes),
                             0, st, (T*)y, (T*)s, rstd, (const T*)x, (const T*)r, (const W*)w, (int)cols, ld_x, ld_r,
                             ld_y, ld_s, eps);
        else
          hipLaunchKernelGGL((rmsnorm_fwd_stream_kernel<T, W, VEC, false>), dim3((unsigned)rows),
                             dim3(kStreamLanes), 0, st, (T*)y, (T*)nullptr, rstd, (const T*)x, (const T*)nullptr,
                             (const W*)w, (int)cols, ld_x, ld_x, ld_y, ld_y, eps);
        return check_launch("rmsnorm_fwd_stream_kernel");
      };
      if (vec_ok) return launch(std::integral_constant<int, 16 / sizeof(T)>{});
      return launch(std::integral_constant<int, 1>{});
    });
  }
  const int64_t grid = cdiv(rows, g.rpb);
  int rc = dispatch_xw(dt_x, dt_w, [&](auto tx, auto tw) {
    using T = typename decltype(tx)::type;
    using W = typename decltype(tw)::type;
    return dispatch_nch(g.nch, [&](auto nch_c) {
      constexpr int NCH = decltype(nch_c)::value;
      return dispatch_lb(g.block, [&](auto lb_c) {
        constexpr int LB = decltype(lb_c)::value;
        auto launch = [&](auto vec_c) {
          constexpr int VEC = decltype(vec_c)::value;
          if (add)
            hipLaunchKernelGGL((rmsnorm_fwd_kernel<T, W, VEC, NCH, true, LB>), dim3(grid), dim3(g.block), 0, st,
                               (T*)y, (T*)s, rstd, (const T*)x, (const T*)r, (const W*)w, rows, (int)cols, ld_x,
                               ld_r, ld_y, ld_s, g.wpr, eps);
          else
            hipLaunchKernelGGL((rmsnorm_fwd_kernel<T, W, VEC, NCH, false, LB>), dim3(grid), dim3(g.block), 0, st,
                               (T*)y, (T*)nullptr, rstd, (const T*)x, (const T*)nullptr, (const W*)w, rows,
                               (int)cols, ld_x, ld_x, ld_y, ld_y, g.wpr, eps);
          return check_launch("rmsnorm_fwd_kernel");
        };
        if (g.vec == 1) return launch(std::integral_constant<int, 1>{});
        return launch(std::integral_constant<int, 16 / sizeof(T)>{});
      });
    });
  });
  return rc;
}

// Geometry, grid and workspace layout of the backward launch, shared by the
// workspace query.
struct BwdPlan {
  Geom g;
  int block;          // threads a block: rpb row groups of g.wpr waves
  int rpb;            // row groups a block
  size_t lds;         // dynamic LDS for summing the groups of a block (rpb > 1)
  int64_t groups;     // row groups
  int64_t rpg;        // rows per group
  int64_t grid;       // blocks
  int64_t parts;      // partial rows: one per block (rpb > 1) or per group
  bool atomic;
  size_t total;
  // rows too long for the register form: rmsnorm_bwd_dot_kernel, then
  // rmsnorm_bwd_cols_kernel over groups x nslice column slices (partial rows,
  // whatever dw_mode asks), the per-row coefficients after the partial rows
  bool stream = false;
  int nslice = 0;
  int vec = 1;
  size_t coef_off = 0;
};

constexpr size_t kBwdLdsMax = 32 * 1024;

bool plan_bwd(int64_t rows, int64_t cols, int es, bool vec_ok, int dw_mode, int cu, BwdPlan* p, bool has_ds) {
  if (!choose_geom(cols, es, vec_ok, &p->g)) {
    p->stream = true;
    p->atomic = false;
    p->vec = vec_ok ? 16 / es : 1;
    const int64_t slice = (int64_t)kSliceLanes * kSliceVecs * p->vec;
    p->nslice = (int)cdiv(cols, slice);
    // about two blocks a CU in all; every group a run of whole rows
    const int64_t want = std::max<int64_t>(1, cdiv(2 * (int64_t)(cu > 0 ? cu : 256), p->nslice));
    p->groups = std::max<int64_t>(1, std::min<int64_t>(rows, want));
    p->rpg = rows > 0 ? cdiv(rows, p->groups) : 0;
    p->groups = rows > 0 ? cdiv(rows, p->rpg) : 1;
    p->parts = p->groups;
    p->grid = p->groups * p->nslice;
    p->coef_off = ((size_t)p->parts * cols * sizeof(float) + 255) / 256 * 256;
    p->total = p->coef_off + (size_t)std::max<int64_t>(rows, 1) * sizeof(float);
    return true;
  }
  const int64_t ncu = cu > 0 ? cu : 256;
  p->atomic = dw_mode == HK_DW_ATOMIC;
  // 1024-lane blocks of several row groups whose dW accumulators meet in LDS:
  // the partial rows (the dW pass's traffic) are one per block, not one per
  // group, and a CU holds 16 waves (256-lane single-group blocks, two a CU,
  // measured up to 1.5x slower below 4096 rows and within 5% above, with dS or
  // without). fp32 inputs: their fp64 accumulators make the 1024-lane form
  // spill, so groups of 64 or 128 lanes (H <= 2048) share 512-lane blocks, two
  // a CU (1.1-2x faster than a group a block); 256-lane groups run alone (two
  // groups a 512-lane block measured 3-6% slower at H = 4096, C1 among them).
  // The fused-add backward (a third input row, dS) of 256-lane 16-bit groups
  // at 32 rows a CU or more runs one group a block too: 1-3% faster there
  // (C2's [8192, 4096]: 46.4 -> 44.3 us), slower with 512-lane groups.
  const size_t acc_bytes = es == 4 ? sizeof(double) : sizeof(float);
  const bool alone = has_ds && p->g.wpr == 4 && rows >= 32 * ncu;
  const int rpb = es == 4 ? (p->g.wpr <= 2 ? 512 / (p->g.wpr * kWave) : 1)
                          : (alone ? 1 : std::max(1, 1024 / (p->g.wpr * kWave)));
  const bool combine = rpb > 1 && (size_t)cols * acc_bytes <= kBwdLdsMax;
  p->block = (combine ? rpb : 1) * p->g.wpr * kWave;  // without the LDS sum: one group a block
  p->rpb = p->block / (p->g.wpr * kWave);
  p->lds = combine ? (size_t)cols * acc_bytes : 0;
  // Many rows a group keep the partial rows few. One 1024-lane block a CU (the
  // 16-bit H = 4096 form needs ~100 VGPRs, so a second would not be resident);
  // two of 512 lanes or fewer.
  const int64_t blocks = (combine && p->block == 1024 ? 1 : 2) * ncu;
  const int64_t target = blocks * p->rpb;
  p->groups = std::max<int64_t>(1, std::min<int64_t>(rows, target));
  p->rpg = rows > 0 ? cdiv(rows, p->groups) : 0;
  p->groups = rows > 0 ? cdiv(rows, p->rpg) : 1;
  p->grid = cdiv(p->groups, (int64_t)p->rpb);
  p->groups = p->grid * p->rpb;  // every launched group walks rpg rows (past the end: masked)
  p->parts = p->rpb > 1 ? p->grid : p->groups;
  p->total = p->atomic ? (size_t)cols * 8 : (size_t)p->parts * cols * sizeof(float);
  return true;
}

// Argument checks of the backward entry points (no HIP call).
int bwd_check(void* dx, void* dw, const void* dy, const void* ds, const void* x, const void* w, const float* rstd,
              int64_t rows, int64_t cols, int64_t ld_dy, int64_t ld_ds, int64_t ld_x, int64_t ld_dx, int dt_x,
              int dt_w, int dw_mode) {
  HK_REQUIRE(valid_dtype(dt_x) && valid_dtype(dt_w), "invalid dtype code (x=%d, w=%d)", dt_x, dt_w);
  HK_REQUIRE(rows >= 0 && cols > 0, "invalid shape rows=%lld cols=%lld", (long long)rows, (long long)cols);
  HK_REQUIRE(cols <= (1 << 30), "cols=%lld too large", (long long)cols);
  HK_REQUIRE(ld_dy >= cols && ld_x >= cols && ld_dx >= cols && (!ds || ld_ds >= cols),
             "row stride smaller than cols");
  HK_REQUIRE(dw_mode == HK_DW_AUTO || dw_mode == HK_DW_ATOMIC || dw_mode == HK_DW_PARTIAL, "invalid dw_mode %d",
             dw_mode);
  HK_REQUIRE(dx && dw && dy && x && w && rstd, "null pointer argument");
  return HK_OK;
}

int bwd_impl(void* dx, void* dw, const void* dy, const void* ds, const void* x, const void* w, const float* rstd,
             int64_t rows, int64_t cols, int64_t ld_dy, int64_t ld_ds, int64_t ld_x, int64_t ld_dx, int dt_x,
             int dt_w, int dw_mode, void* workspace, size_t ws_bytes, hk_stream_t stream) {
  if (const int rc = bwd_check(dx, dw, dy, ds, x, w, rstd, rows, cols, ld_dy, ld_ds, ld_x, ld_dx, dt_x, dt_w,
                               dw_mode))
    return rc;
  const int es = dtype_size(dt_x), wsz = dtype_size(dt_w);
  const int vec = 16 / es;
  bool vec_ok = cols % vec == 0 && rows_aligned(dy, ld_dy, es) && rows_aligned(x, ld_x, es) &&
                rows_aligned(dx, ld_dx, es) && aligned_to(w, (size_t)wsz * vec);
  if (ds) vec_ok = vec_ok && rows_aligned(ds, ld_ds, es);
  const int dev = current_device();
  if (dev < 0) return (int)hipErrorNoDevice;
  BwdPlan p;
  plan_bwd(rows, cols, es, vec_ok, dw_mode, cu_count(dev), &p, ds != nullptr);
  HK_REQUIRE(workspace != nullptr && ws_bytes >= p.total, "workspace too small: need %zu bytes, got %zu", p.total,
             ws_bytes);
  HK_REQUIRE(aligned_to(workspace, 16), "workspace must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  void* part = workspace;

  return dispatch_xw(dt_x, dt_w, [&](auto tx, auto tw) {
    using T = typename decltype(tx)::type;
    using W = typename decltype(tw)::type;
    using A = typename std::conditional<std::is_same<T, float>::value, double, float>::type;
    if (p.stream) {
      float* coef = (float*)((char*)workspace + p.coef_off);
      if (rows > 0) {
        auto launch = [&](auto vec_c) {
          constexpr int VEC = decltype(vec_c)::value;
          hipLaunchKernelGGL((rmsnorm_bwd_dot_kernel<T, W, VEC>), dim3((unsigned)rows), dim3(kStreamLanes), 0, st,
                             coef, (const T*)dy, (const T*)x, (const W*)w, rstd, (int)cols, ld_dy, ld_x);
          int rc = check_launch("rmsnorm_bwd_dot_kernel");
          if (rc) return rc;
          auto go = [&](auto hds_c) {
            constexpr bool HDS = decltype(hds_c)::value;
            hipLaunchKernelGGL((rmsnorm_bwd_cols_kernel<T, W, A, VEC, HDS>), dim3((unsigned)p.grid),
                               dim3(kSliceLanes), 0, st, (T*)dx, (float*)part, (const T*)dy, (const T*)ds,
                               (const T*)x, (const W*)w, rstd, coef, rows, (int)cols, ld_dy, ld_ds, ld_x, ld_dx,
                               p.nslice, p.rpg);
            return check_launch("rmsnorm_bwd_cols_kernel");
          };
          if (ds) return go(std::true_type{});
          return go(std::false_type{});
        };
        const int rc = p.vec > 1 ? launch(std::integral_constant<int, 16 / sizeof(T)>{})
                                 : launch(std::integral_constant<int, 1>{});
        if (rc) return rc;
      }
      colsum_launch<W>((W*)dw, nullptr, (const float*)part, rows > 0 ? p.parts : 0, cols, cols, cols, st);
      return check_launch("colsum_kernel");
    }
    if (p.atomic) {
      hipLaunchKernelGGL(fill_zero_f64, dim3((unsigned)cdiv(cols, 256)), dim3(256), 0, st, (double*)part, cols);
      int rc = check_launch("fill_zero_f64");
      if (rc) return rc;
    }
    if (rows > 0) {
      int rc = dispatch_nch(p.g.nch, [&](auto nch_c) {
        constexpr int NCH = decltype(nch_c)::value;
        return dispatch_lb_bwd(p.block, [&](auto lb_c) {
          constexpr int LB = decltype(lb_c)::value;
          auto launch = [&](auto vec_c) {
            constexpr int VEC = decltype(vec_c)::value;
            auto go = [&](auto hds_c) {
              constexpr bool HDS = decltype(hds_c)::value;
              hipLaunchKernelGGL((rmsnorm_bwd_kernel<T, W, A, VEC, NCH, HDS, LB>), dim3((unsigned)p.grid),
                                 dim3(p.block), p.lds, st, (T*)dx, part, (int)p.atomic, (const T*)dy, (const T*)ds,
                                 (const T*)x, (const W*)w, rstd, rows, (int)cols, ld_dy, ld_ds, ld_x, ld_dx, p.g.wpr,
                                 p.rpg);
              return check_launch("rmsnorm_bwd_kernel");
            };
            if (ds) return go(std::true_type{});
            return go(std::false_type{});
          };
          if (p.g.vec == 1) return launch(std::integral_constant<int, 1>{});
          return launch(std::integral_constant<int, 16 / sizeof(T)>{});
        });
      });
      if (rc) return rc;
    }
    if (p.atomic) {
      hipLaunchKernelGGL((cast_f64_kernel<W>), dim3((unsigned)cdiv(cols, 256)), dim3(256), 0, st, (W*)dw,
                         (const double*)part, cols);
      return check_launch("cast_f64_kernel");
    }
    // (no rows: zero groups are summed and dW comes out zero)
    colsum_launch<W>((W*)dw, nullptr, (const float*)part, rows > 0 ? p.parts : 0, cols, cols, cols, st);
    return check_launch("colsum_kernel");
  });
}

// ------------------------------------------------------------------------
// allocation-free backward: the dW scratch in a file-scope device array
// ------------------------------------------------------------------------
// hk_rms_norm_bwd_noalloc keeps its dW partial rows (or fp64 accumulator) here
// instead of in caller workspace. Every GPU the library runs on holds its own
// copy, at its own address, until the process ends. Host code never uses the
// array's name as a device address: scratch_ptr() looks the address up once
// per device with hipGetSymbolAddress and kernels receive that pointer.
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxScratchDevices = 64;

// The device address of `scratch` on `device`, which must be the current
// device; looked up on the first call for that device. nullptr on failure
// (the error text is set).
void* scratch_ptr(int device) {
  static std::once_flag once[kMaxScratchDevices];
  static void* ptr[kMaxScratchDevices];
  static hipError_t err[kMaxScratchDevices];
  if (device < 0 || device >= kMaxScratchDevices) {
    set_error("device %d out of range for the scratch table", device);
    return nullptr;
  }
  std::call_once(once[device], [device] {
    void* p = nullptr;
    err[device] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    ptr[device] = err[device] == hipSuccess ? p : nullptr;
  });
  if (!ptr[device]) set_error("hipGetSymbolAddress(scratch) failed on device %d: %s", device,
                              hipGetErrorString(err[device]));
  return ptr[device];
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
  // The vector width and the dS input only change the geometry, so plan every
  // combination (this query serves both backwards) and take the largest.
  size_t best = 0;
  for (int v = 0; v < 2; ++v)
    for (int d = 0; d < 2; ++d)
      if (plan_bwd(rows, cols, dtype_size(dtype_x), v == 0, dw_mode, cu_count(device), &p, d == 1))
        best = std::max(best, p.total);
  return best;
}

int hk_rms_norm_bwd(void* dx, void* dw, const void* dy, const void* x, const void* w, const float* rstd, int64_t rows,
                    int64_t cols, int64_t ld_dy, int64_t ld_x, int64_t ld_dx, int dtype_x, int dtype_w, int dw_mode,
                    void* workspace, size_t workspace_bytes, hk_stream_t stream) {
  return bwd_impl(dx, dw, dy, nullptr, x, w, rstd, rows, cols, ld_dy, ld_dy, ld_x, ld_dx, dtype_x, dtype_w, dw_mode,
                  workspace, workspace_bytes, stream);
}

int hk_rms_norm_bwd_noalloc(void* dx, void* dw, const void* dy, const void* x, const void* w, const float* rstd,
                            int64_t rows, int64_t cols, int64_t ld_dy, int64_t ld_x, int64_t ld_dx, int dtype_x,
                            int dtype_w, int dw_mode, hk_stream_t stream) {
  if (const int rc = bwd_check(dx, dw, dy, nullptr, x, w, rstd, rows, cols, ld_dy, ld_dy, ld_x, ld_dx, dtype_x,
                               dtype_w, dw_mode))
    return rc;
  const int dev = current_device();
  if (dev < 0) return (int)hipErrorNoDevice;
  const size_t need = hk_rms_norm_bwd_workspace_size(rows, cols, dtype_x, dtype_w, dw_mode, dev);
  HK_REQUIRE(need <= kNoAllocScratchBytes,
             "rows=%lld cols=%lld need %zu bytes of dW scratch, more than the %zu this entry point holds "
             "(use hk_rms_norm_bwd with a workspace)",
             (long long)rows, (long long)cols, need, kNoAllocScratchBytes);
  void* ws = scratch_ptr(dev);
  if (!ws) return (int)hipErrorInvalidSymbol;
  return bwd_impl(dx, dw, dy, nullptr, x, w, rstd, rows, cols, ld_dy, ld_dy, ld_x, ld_dx, dtype_x, dtype_w, dw_mode,
                  ws, kNoAllocScratchBytes, stream);
}

int hk_fused_add_rms_norm_bwd(void* dx, void* dw, const void* dy, const void* ds_out, const void* s, const void* w,
                              const float* rstd, int64_t rows, int64_t cols, int64_t ld, int dtype_x, int dtype_w,
                              int dw_mode, void* workspace, size_t workspace_bytes, hk_stream_t stream) {
  return bwd_impl(dx, dw, dy, ds_out, s, w, rstd, rows, cols, ld, ld, ld, ld, dtype_x, dtype_w, dw_mode, workspace,
                  workspace_bytes, stream);
}

}  // extern "C"
