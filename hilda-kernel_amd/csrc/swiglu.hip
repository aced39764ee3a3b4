// SwiGLU forward/backward for gfx950: c = silu(a) * b, elementwise, HBM-bound.
//
// Each thread moves UNROLL 16-byte vectors per tensor, all loads issued
// before any arithmetic so a wave keeps UNROLL*1 KiB per tensor in flight.
// Rounding points follow kernels/swiglu.py:55-56 (silu computed in fp32 and
// rounded to the dtype of b before the product) and :99-105 (gradients in
// fp32, one rounding at the store). The backward writes fresh da/db buffers
// instead of overwriting the saved a/b; the HBM traffic is the same.
#include "hk_common.h"
#include "../../include/hilda_kernel_amd.h"

#include <type_traits>

namespace hk {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;

template <typename T, int VEC>
__global__ __launch_bounds__(kThreads) void swiglu_fwd_kernel(T* __restrict__ c, const T* __restrict__ a,
                                                              const T* __restrict__ b, int64_t nvec) {
  const int64_t base = (int64_t)blockIdx.x * (kThreads * kUnroll) + threadIdx.x;
  Pack<T, VEC> av[kUnroll], bv[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = base + (int64_t)u * kThreads;
    if (i < nvec) {
      av[u] = load_pack<T, VEC>(a + i * VEC);
      bv[u] = load_pack<T, VEC>(b + i * VEC);
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = base + (int64_t)u * kThreads;
    if (i < nvec) {
      float x[VEC], y[VEC];
      unpack(av[u], x);
      unpack(bv[u], y);
#pragma unroll
      for (int e = 0; e < VEC; ++e) x[e] = round_through<T>(x[e] * sigmoid_fast(x[e])) * y[e];
      store_pack<T, VEC>(c + i * VEC, pack<T, VEC>(x));
    }
  }
}

template <typename T, int VEC>
__global__ __launch_bounds__(kThreads) void swiglu_bwd_kernel(T* __restrict__ da, T* __restrict__ db,
                                                              const T* __restrict__ a, const T* __restrict__ b,
                                                              const T* __restrict__ dc, int64_t nvec) {
  const int64_t base = (int64_t)blockIdx.x * (kThreads * kUnroll) + threadIdx.x;
  Pack<T, VEC> av[kUnroll], bv[kUnroll], gv[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = base + (int64_t)u * kThreads;
    if (i < nvec) {
      av[u] = load_pack<T, VEC>(a + i * VEC);
      bv[u] = load_pack<T, VEC>(b + i * VEC);
      gv[u] = load_pack<T, VEC>(dc + i * VEC);
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = base + (int64_t)u * kThreads;
    if (i < nvec) {
      float x[VEC], y[VEC], g[VEC];
      unpack(av[u], x);
      unpack(bv[u], y);
      unpack(gv[u], g);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float s = sigmoid_fast(x[e]);
        const float silu = x[e] * s;
        const float d_b = g[e] * silu;
        const float d_a = g[e] * y[e] * (s + x[e] * s * (1.0f - s));
        x[e] = d_a;
        y[e] = d_b;
      }
      store_pack<T, VEC>(da + i * VEC, pack<T, VEC>(x));
      store_pack<T, VEC>(db + i * VEC, pack<T, VEC>(y));
    }
  }
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

template <typename T>
int launch_fwd(void* c, const void* a, const void* b, int64_t n, hipStream_t st) {
  constexpr int V = 16 / sizeof(T);
  const bool vec = aligned_to(a, 16) && aligned_to(b, 16) && aligned_to(c, 16);
  if (vec) {
    const int64_t nvec = n / V, tail = n - nvec * V;
    if (nvec > 0)
      hipLaunchKernelGGL((swiglu_fwd_kernel<T, V>), dim3((unsigned)cdiv(nvec, kThreads * kUnroll)), dim3(kThreads),
                         0, st, (T*)c, (const T*)a, (const T*)b, nvec);
    if (tail > 0)
      hipLaunchKernelGGL((swiglu_fwd_kernel<T, 1>), dim3(1), dim3(kThreads), 0, st, (T*)c + nvec * V,
                         (const T*)a + nvec * V, (const T*)b + nvec * V, tail);
  } else {
    hipLaunchKernelGGL((swiglu_fwd_kernel<T, 1>), dim3((unsigned)cdiv(n, kThreads * kUnroll)), dim3(kThreads), 0,
                       st, (T*)c, (const T*)a, (const T*)b, n);
  }
  return check_launch("swiglu_fwd_kernel");
}

template <typename T>
int launch_bwd(void* da, void* db, const void* a, const void* b, const void* dc, int64_t n, hipStream_t st) {
  constexpr int V = 16 / sizeof(T);
  const bool vec = aligned_to(a, 16) && aligned_to(b, 16) && aligned_to(dc, 16) && aligned_to(da, 16) &&
                   aligned_to(db, 16);
  if (vec) {
    const int64_t nvec = n / V, tail = n - nvec * V;
    if (nvec > 0)
      hipLaunchKernelGGL((swiglu_bwd_kernel<T, V>), dim3((unsigned)cdiv(nvec, kThreads * kUnroll)), dim3(kThreads),
                         0, st, (T*)da, (T*)db, (const T*)a, (const T*)b, (const T*)dc, nvec);
    if (tail > 0)
      hipLaunchKernelGGL((swiglu_bwd_kernel<T, 1>), dim3(1), dim3(kThreads), 0, st, (T*)da + nvec * V,
                         (T*)db + nvec * V, (const T*)a + nvec * V, (const T*)b + nvec * V, (const T*)dc + nvec * V,
                         tail);
  } else {
    hipLaunchKernelGGL((swiglu_bwd_kernel<T, 1>), dim3((unsigned)cdiv(n, kThreads * kUnroll)), dim3(kThreads), 0,
                       st, (T*)da, (T*)db, (const T*)a, (const T*)b, (const T*)dc, n);
  }
  return check_launch("swiglu_bwd_kernel");
}

}  // namespace
}  // namespace hk

using namespace hk;

extern "C" {

int hk_swiglu_fwd(void* c, const void* a, const void* b, int64_t n, int dtype, hk_stream_t stream) {
  HK_REQUIRE(n >= 0, "invalid element count %lld", (long long)n);
  HK_REQUIRE(n == 0 || (c && a && b), "null pointer argument");
  HK_REQUIRE(n <= (int64_t)UINT32_MAX * kThreads * kUnroll, "too many elements");
  return dispatch_t(dtype, [&](auto t) {
    using T = typename decltype(t)::type;
    if (n == 0) return HK_OK;
    return launch_fwd<T>(c, a, b, n, (hipStream_t)stream);
  });
}

int hk_swiglu_bwd(void* da, void* db, const void* a, const void* b, const void* dc, int64_t n, int dtype,
                  hk_stream_t stream) {
  HK_REQUIRE(n >= 0, "invalid element count %lld", (long long)n);
  HK_REQUIRE(n == 0 || (da && db && a && b && dc), "null pointer argument");
  HK_REQUIRE(n <= (int64_t)UINT32_MAX * kThreads * kUnroll, "too many elements");
  return dispatch_t(dtype, [&](auto t) {
    using T = typename decltype(t)::type;
    if (n == 0) return HK_OK;
    return launch_bwd<T>(da, db, a, b, dc, n, (hipStream_t)stream);
  });
}

}  // extern "C"
