// Shared device/host helpers for the hilda-kernel_amd HIP kernels (gfx950, wave64).
//
// Everything here is written for CDNA4: 64-lane wavefronts, 128-bit global
// loads/stores, hardware transcendental instructions (v_exp_f32 = 2^x,
// v_log_f32 = log2 x, v_rsq_f32, v_rcp_f32) and LDS for cross-wave reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace hk {

// ---------------------------------------------------------------------------
// dtype codes shared with the C ABI (include/hilda_kernel_amd.h)
// ---------------------------------------------------------------------------
enum Dtype : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---------------------------------------------------------------------------
// scalar conversions
// ---------------------------------------------------------------------------
template <typename T> __device__ __forceinline__ float to_f32(T v);
template <> __device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_f32<_Float16>(_Float16 v) { return (float)v; }
template <> __device__ __forceinline__ float to_f32<__bf16>(__bf16 v) { return (float)v; }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ _Float16 from_f32<_Float16>(float v) { return (_Float16)v; }
// gfx950 lowers this to v_cvt_pk_bf16_f32 (round to nearest even, NaN kept)
template <> __device__ __forceinline__ __bf16 from_f32<__bf16>(float v) { return (__bf16)v; }

// Round a float through T and back (models "x.to(T)" followed by an fp32 op).
template <typename T> __device__ __forceinline__ float round_through(float v) {
  return to_f32<T>(from_f32<T>(v));
}

// ---------------------------------------------------------------------------
// packed vectors: VEC elements of T moved as one global transaction
// (16 bytes when VEC*sizeof(T) == 16).
// ---------------------------------------------------------------------------
template <typename T, int VEC>
struct alignas(sizeof(T) * VEC) Pack {
  T v[VEC];
};

template <typename T, int VEC>
__device__ __forceinline__ Pack<T, VEC> load_pack(const T* p) {
  return *reinterpret_cast<const Pack<T, VEC>*>(p);
}
template <typename T, int VEC>
__device__ __forceinline__ void store_pack(T* p, const Pack<T, VEC>& v) {
  *reinterpret_cast<Pack<T, VEC>*>(p) = v;
}
// Streaming store for outputs that are not re-read by this kernel.
template <typename T, int VEC>
__device__ __forceinline__ void store_pack_nt(T* p, const Pack<T, VEC>& v) {
  constexpr int B = sizeof(T) * VEC;
  if constexpr (B == 16) {
    __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(&v), reinterpret_cast<u32x4*>(p));
  } else if constexpr (B == 8) {
    __builtin_nontemporal_store(*reinterpret_cast<const u32x2*>(&v), reinterpret_cast<u32x2*>(p));
  } else if constexpr (B == 4) {
    __builtin_nontemporal_store(*reinterpret_cast<const uint32_t*>(&v), reinterpret_cast<uint32_t*>(p));
  } else {
    *reinterpret_cast<Pack<T, VEC>*>(p) = v;
  }
}

template <typename T, int VEC>
__device__ __forceinline__ void unpack(const Pack<T, VEC>& p, float (&out)[VEC]) {
#pragma unroll
  for (int i = 0; i < VEC; ++i) out[i] = to_f32<T>(p.v[i]);
}
template <typename T, int VEC>
__device__ __forceinline__ Pack<T, VEC> pack(const float (&in)[VEC]) {
  Pack<T, VEC> p;
#pragma unroll
  for (int i = 0; i < VEC; ++i) p.v[i] = from_f32<T>(in[i]);
  return p;
}

// ---------------------------------------------------------------------------
// transcendental helpers on the hardware units
// ---------------------------------------------------------------------------
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float log2_fast(float x) { return __builtin_amdgcn_logf(x); }
// e^x with a single rounding of x*log2(e)
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }
__device__ __forceinline__ float log_fast(float x) { return __builtin_amdgcn_logf(x) * kLn2; }
__device__ __forceinline__ float rcp_fast(float x) { return __builtin_amdgcn_rcpf(x); }
// logistic function 1 / (1 + e^-x)
__device__ __forceinline__ float sigmoid_fast(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * kLog2e));
}

// ---------------------------------------------------------------------------
// wave64 reductions (butterfly over all 64 lanes; every lane gets the result)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Sum over the NW waves of a block; `red` must hold NW floats of LDS.
// Every thread of the block receives the result. Contains two barriers.
template <int NW>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  if constexpr (NW == 1) return v;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < NW; ++i) t += red[i];
  __syncthreads();
  return t;
}
template <int NW>
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  if constexpr (NW == 1) return v;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) t = fmaxf(t, red[i]);
  __syncthreads();
  return t;
}

// ---------------------------------------------------------------------------
// host-side helpers (error reporting, device properties, launch checks)
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int cu_count(int device);            // cached per device
int current_device();                // -1 on failure (error recorded)
int check_launch(const char* what);  // 0 or hipError_t after a launch

inline bool aligned_to(const void* p, size_t bytes) {
  return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace hk

// Status codes returned by every C-ABI entry point.
#define HK_OK 0
#define HK_EINVAL (-1)

#define HK_REQUIRE(cond, ...)        \
  do {                               \
    if (!(cond)) {                   \
      ::hk::set_error(__VA_ARGS__);  \
      return HK_EINVAL;              \
    }                                \
  } while (0)

#define HK_HIP(call)                                                               \
  do {                                                                             \
    hipError_t _e = (call);                                                        \
    if (_e != hipSuccess) {                                                        \
      ::hk::set_error("%s failed: %s", #call, hipGetErrorString(_e));              \
      return (int)_e;                                                              \
    }                                                                              \
  } while (0)
