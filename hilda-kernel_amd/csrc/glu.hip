// Gated activations for gfx950, elementwise and HBM-bound:
//   SwiGLU c = silu(a) * b            (kernels/swiglu.py)
//   GeGLU  c = gelu_tanh(a) * b       (kernels/geglu.py)
//
// Each thread moves UNROLL 16-byte vectors per tensor, all loads issued
// before any arithmetic so a wave keeps UNROLL*1 KiB per tensor in flight.
// Rounding points follow the reference: the activation is computed in fp32
// and rounded to the dtype of b before the product (swiglu.py:55-56,
// geglu.py:69-71); gradients are computed in fp32 with one rounding at the
// store (swiglu.py:99-105, geglu.py:110-124). The backward writes fresh da/db
// buffers instead of overwriting the saved a/b; the HBM traffic is the same.
#include "hk_common.h"
#include "../../include/hilda_kernel_amd.h"

#include <type_traits>

namespace hk {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;

// silu(x) = x * sigmoid(x); silu'(x) = s + x s (1 - s)
struct SiLU {
  __device__ __forceinline__ static float f(float x) { return x * sigmoid_fast(x); }
  __device__ __forceinline__ static void f_df(float x, float* f, float* df) {
    const float s = sigmoid_fast(x);
    *f = x * s;
    *df = s + x * s * (1.0f - s);
  }
};

// tanh-approximated GELU, 0.5 x (1 + tanh(u)) with u = sqrt(2/pi) (x + 0.044715 x^3)
// (geglu.py:69-70). Since 0.5 (1 + tanh(u)) = sigmoid(2u), gelu(x) = x sigmoid(2u):
// no tanh routine is needed, and the left tail keeps full relative precision
// instead of cancelling in 1 + tanh(u). With s = sigmoid(2u), 1 - tanh(u)^2 =
// 4 s (1 - s), so the derivative of geglu.py:115-116 becomes
// gelu'(x) = s + 2 x s (1 - s) sqrt(2/pi) (1 + 3 * 0.044715 x^2).
struct GeluTanh {
  static constexpr float kSqrt2OverPi = 0.7978845608028654f;
  static constexpr float kCoeff = 0.044715f;
  __device__ __forceinline__ static float sig2u(float x) {
    const float u = kSqrt2OverPi * (x + kCoeff * x * x * x);
    return sigmoid_fast(2.0f * u);
  }
  __device__ __forceinline__ static float f(float x) { return x * sig2u(x); }
  __device__ __forceinline__ static void f_df(float x, float* f, float* df) {
    const float s = sig2u(x);
    *f = x * s;
    *df = s + 2.0f * x * s * (1.0f - s) * kSqrt2OverPi * (1.0f + 3.0f * kCoeff * x * x);
  }
};

template <class Act, typename T, int VEC>
__device__ __forceinline__ void glu_fwd(T* __restrict__ c, const T* __restrict__ a, const T* __restrict__ b,
                                        int64_t nvec) {
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
      for (int e = 0; e < VEC; ++e) x[e] = round_through<T>(Act::f(x[e])) * y[e];
      store_pack<T, VEC>(c + i * VEC, pack<T, VEC>(x));
    }
  }
}

template <class Act, typename T, int VEC>
__device__ __forceinline__ void glu_bwd(T* __restrict__ da, T* __restrict__ db, const T* __restrict__ a,
                                        const T* __restrict__ b, const T* __restrict__ dc, int64_t nvec) {
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
        float f, df;
        Act::f_df(x[e], &f, &df);
        const float d_b = g[e] * f;
        const float d_a = g[e] * y[e] * df;
        x[e] = d_a;
        y[e] = d_b;
      }
      store_pack<T, VEC>(da + i * VEC, pack<T, VEC>(x));
      store_pack<T, VEC>(db + i * VEC, pack<T, VEC>(y));
    }
  }
}

// one named kernel per activation, so profiles tell them apart
template <typename T, int VEC>
__global__ __launch_bounds__(kThreads) void swiglu_fwd_kernel(T* __restrict__ c, const T* __restrict__ a,
                                                              const T* __restrict__ b, int64_t nvec) {
  glu_fwd<SiLU, T, VEC>(c, a, b, nvec);
}
template <typename T, int VEC>
__global__ __launch_bounds__(kThreads) void swiglu_bwd_kernel(T* __restrict__ da, T* __restrict__ db,
                                                              const T* __restrict__ a, const T* __restrict__ b,
                                                              const T* __restrict__ dc, int64_t nvec) {
  glu_bwd<SiLU, T, VEC>(da, db, a, b, dc, nvec);
}
template <typename T, int VEC>
__global__ __launch_bounds__(kThreads) void geglu_fwd_kernel(T* __restrict__ c, const T* __restrict__ a,
                                                             const T* __restrict__ b, int64_t nvec) {
  glu_fwd<GeluTanh, T, VEC>(c, a, b, nvec);
}
template <typename T, int VEC>
__global__ __launch_bounds__(kThreads) void geglu_bwd_kernel(T* __restrict__ da, T* __restrict__ db,
                                                             const T* __restrict__ a, const T* __restrict__ b,
                                                             const T* __restrict__ dc, int64_t nvec) {
  glu_bwd<GeluTanh, T, VEC>(da, db, a, b, dc, nvec);
}

template <class Act, typename T, int VEC> struct Kern;
template <typename T, int VEC> struct Kern<SiLU, T, VEC> {
  static constexpr auto fwd = swiglu_fwd_kernel<T, VEC>;
  static constexpr auto bwd = swiglu_bwd_kernel<T, VEC>;
  static constexpr const char* fwd_name = "swiglu_fwd_kernel";
  static constexpr const char* bwd_name = "swiglu_bwd_kernel";
};
template <typename T, int VEC> struct Kern<GeluTanh, T, VEC> {
  static constexpr auto fwd = geglu_fwd_kernel<T, VEC>;
  static constexpr auto bwd = geglu_bwd_kernel<T, VEC>;
  static constexpr const char* fwd_name = "geglu_fwd_kernel";
  static constexpr const char* bwd_name = "geglu_bwd_kernel";
};

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

template <class Act, typename T>
int launch_fwd(void* c, const void* a, const void* b, int64_t n, hipStream_t st) {
  constexpr int V = 16 / sizeof(T);
  using KV = Kern<Act, T, V>;
  using K1 = Kern<Act, T, 1>;
  const bool vec = aligned_to(a, 16) && aligned_to(b, 16) && aligned_to(c, 16);
  if (vec) {
    const int64_t nvec = n / V, tail = n - nvec * V;
    if (nvec > 0)
      hipLaunchKernelGGL(KV::fwd, dim3((unsigned)cdiv(nvec, kThreads * kUnroll)), dim3(kThreads), 0, st, (T*)c,
                         (const T*)a, (const T*)b, nvec);
    if (tail > 0)
      hipLaunchKernelGGL(K1::fwd, dim3(1), dim3(kThreads), 0, st, (T*)c + nvec * V, (const T*)a + nvec * V,
                         (const T*)b + nvec * V, tail);
  } else {
    hipLaunchKernelGGL(K1::fwd, dim3((unsigned)cdiv(n, kThreads * kUnroll)), dim3(kThreads), 0, st, (T*)c,
                       (const T*)a, (const T*)b, n);
  }
  return check_launch(KV::fwd_name);
}

template <class Act, typename T>
int launch_bwd(void* da, void* db, const void* a, const void* b, const void* dc, int64_t n, hipStream_t st) {
  constexpr int V = 16 / sizeof(T);
  using KV = Kern<Act, T, V>;
  using K1 = Kern<Act, T, 1>;
  const bool vec = aligned_to(a, 16) && aligned_to(b, 16) && aligned_to(dc, 16) && aligned_to(da, 16) &&
                   aligned_to(db, 16);
  if (vec) {
    const int64_t nvec = n / V, tail = n - nvec * V;
    if (nvec > 0)
      hipLaunchKernelGGL(KV::bwd, dim3((unsigned)cdiv(nvec, kThreads * kUnroll)), dim3(kThreads), 0, st, (T*)da,
                         (T*)db, (const T*)a, (const T*)b, (const T*)dc, nvec);
    if (tail > 0)
      hipLaunchKernelGGL(K1::bwd, dim3(1), dim3(kThreads), 0, st, (T*)da + nvec * V, (T*)db + nvec * V,
                         (const T*)a + nvec * V, (const T*)b + nvec * V, (const T*)dc + nvec * V, tail);
  } else {
    hipLaunchKernelGGL(K1::bwd, dim3((unsigned)cdiv(n, kThreads * kUnroll)), dim3(kThreads), 0, st, (T*)da,
                       (T*)db, (const T*)a, (const T*)b, (const T*)dc, n);
  }
  return check_launch(KV::bwd_name);
}

template <class Act>
int glu_fwd_entry(void* c, const void* a, const void* b, int64_t n, int dtype, hk_stream_t stream) {
  HK_REQUIRE(n >= 0, "invalid element count %lld", (long long)n);
  HK_REQUIRE(n == 0 || (c && a && b), "null pointer argument");
  HK_REQUIRE(n <= (int64_t)UINT32_MAX * kThreads * kUnroll, "too many elements");
  return dispatch_t(dtype, [&](auto t) {
    using T = typename decltype(t)::type;
    if (n == 0) return HK_OK;
    return launch_fwd<Act, T>(c, a, b, n, (hipStream_t)stream);
  });
}

template <class Act>
int glu_bwd_entry(void* da, void* db, const void* a, const void* b, const void* dc, int64_t n, int dtype,
                  hk_stream_t stream) {
  HK_REQUIRE(n >= 0, "invalid element count %lld", (long long)n);
  HK_REQUIRE(n == 0 || (da && db && a && b && dc), "null pointer argument");
  HK_REQUIRE(n <= (int64_t)UINT32_MAX * kThreads * kUnroll, "too many elements");
  return dispatch_t(dtype, [&](auto t) {
    using T = typename decltype(t)::type;
    if (n == 0) return HK_OK;
    return launch_bwd<Act, T>(da, db, a, b, dc, n, (hipStream_t)stream);
  });
}

}  // namespace
}  // namespace hk

using namespace hk;

extern "C" {

int hk_swiglu_fwd(void* c, const void* a, const void* b, int64_t n, int dtype, hk_stream_t stream) {
  return glu_fwd_entry<SiLU>(c, a, b, n, dtype, stream);
}

int hk_swiglu_bwd(void* da, void* db, const void* a, const void* b, const void* dc, int64_t n, int dtype,
                  hk_stream_t stream) {
  return glu_bwd_entry<SiLU>(da, db, a, b, dc, n, dtype, stream);
}

int hk_geglu_fwd(void* c, const void* a, const void* b, int64_t n, int dtype, hk_stream_t stream) {
  return glu_fwd_entry<GeluTanh>(c, a, b, n, dtype, stream);
}

int hk_geglu_bwd(void* da, void* db, const void* a, const void* b, const void* dc, int64_t n, int dtype,
                 hk_stream_t stream) {
  return glu_bwd_entry<GeluTanh>(da, db, a, b, dc, n, dtype, stream);
}

}  // extern "C"
