// Shared device/host helpers for the hilda-kernel_amd HIP kernels (gfx950, wave64).
//
// Everything here is written for CDNA4: 64-lane wavefronts, 128-bit global
// loads/stores, hardware transcendental instructions (v_exp_f32 = 2^x,
// v_log_f32 = log2 x, v_rsq_f32, v_rcp_f32) and LDS for cross-wave reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include <type_traits>

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
// (16 bytes when VEC*sizeof(T) == 16). The payload is kept as raw 32-bit
// words so two 16-bit values share one VGPR; elements are widened to fp32 by
// bit operations (bf16: shift/mask) or the hardware half->float convert.
// ---------------------------------------------------------------------------
template <typename T, int VEC, bool SUB_WORD = (sizeof(T) * VEC < 4)>
struct Pack;

template <typename T, int VEC>
struct Pack<T, VEC, false> {
  static constexpr int kWords = sizeof(T) * VEC / 4;
  uint32_t w[kWords];
};
// a single 16-bit element
template <typename T, int VEC>
struct Pack<T, VEC, true> {
  static_assert(sizeof(T) == 2 && VEC == 1, "sub-word packs hold one 16-bit element");
  uint16_t h;
};

template <typename T, int VEC>
__device__ __forceinline__ Pack<T, VEC> load_pack(const T* p) {
  Pack<T, VEC> r;
  constexpr int B = sizeof(T) * VEC;
  if constexpr (B == 16) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(p);
    r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
  } else if constexpr (B == 32) {
    const u32x4 a = reinterpret_cast<const u32x4*>(p)[0];
    const u32x4 b = reinterpret_cast<const u32x4*>(p)[1];
    r.w[0] = a.x; r.w[1] = a.y; r.w[2] = a.z; r.w[3] = a.w;
    r.w[4] = b.x; r.w[5] = b.y; r.w[6] = b.z; r.w[7] = b.w;
  } else if constexpr (B == 8) {
    const u32x2 v = *reinterpret_cast<const u32x2*>(p);
    r.w[0] = v.x; r.w[1] = v.y;
  } else if constexpr (B == 4) {
    r.w[0] = *reinterpret_cast<const uint32_t*>(p);
  } else {
    r.h = *reinterpret_cast<const uint16_t*>(p);
  }
  return r;
}

template <typename T, int VEC>
__device__ __forceinline__ void store_pack(T* p, const Pack<T, VEC>& r) {
  constexpr int B = sizeof(T) * VEC;
  if constexpr (B == 16) {
    *reinterpret_cast<u32x4*>(p) = u32x4{r.w[0], r.w[1], r.w[2], r.w[3]};
  } else if constexpr (B == 32) {
    reinterpret_cast<u32x4*>(p)[0] = u32x4{r.w[0], r.w[1], r.w[2], r.w[3]};
    reinterpret_cast<u32x4*>(p)[1] = u32x4{r.w[4], r.w[5], r.w[6], r.w[7]};
  } else if constexpr (B == 8) {
    *reinterpret_cast<u32x2*>(p) = u32x2{r.w[0], r.w[1]};
  } else if constexpr (B == 4) {
    *reinterpret_cast<uint32_t*>(p) = r.w[0];
  } else {
    *reinterpret_cast<uint16_t*>(p) = r.h;
  }
}

// Streaming store for outputs that are not re-read by this kernel.
template <typename T, int VEC>
__device__ __forceinline__ void store_pack_nt(T* p, const Pack<T, VEC>& r) {
  constexpr int B = sizeof(T) * VEC;
  if constexpr (B == 16) {
    __builtin_nontemporal_store(u32x4{r.w[0], r.w[1], r.w[2], r.w[3]}, reinterpret_cast<u32x4*>(p));
  } else if constexpr (B == 8) {
    __builtin_nontemporal_store(u32x2{r.w[0], r.w[1]}, reinterpret_cast<u32x2*>(p));
  } else if constexpr (B == 4) {
    __builtin_nontemporal_store(r.w[0], reinterpret_cast<uint32_t*>(p));
  } else {
    store_pack<T, VEC>(p, r);
  }
}

__device__ __forceinline__ float bits_f32(uint32_t u) { return __builtin_bit_cast(float, u); }
__device__ __forceinline__ uint32_t f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }

template <typename T, int VEC>
__device__ __forceinline__ void unpack(const Pack<T, VEC>& r, float (&out)[VEC]) {
  if constexpr (std::is_same<T, float>::value) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) out[i] = bits_f32(r.w[i]);
  } else if constexpr (sizeof(T) * VEC < 4) {
    out[0] = to_f32<T>(__builtin_bit_cast(T, r.h));
  } else if constexpr (std::is_same<T, __bf16>::value) {
#pragma unroll
    for (int k = 0; k < VEC / 2; ++k) {
      out[2 * k] = bits_f32(r.w[k] << 16);
      out[2 * k + 1] = bits_f32(r.w[k] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int k = 0; k < VEC / 2; ++k) {
      out[2 * k] = (float)__builtin_bit_cast(_Float16, (uint16_t)(r.w[k] & 0xffffu));
      out[2 * k + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(r.w[k] >> 16));
    }
  }
}

// Two fp32 values rounded to a 16-bit T (nearest even), lo in the low half of
// the word: one two-operand convert (v_cvt_pk_bf16_f32 for bf16) rather than
// two converts and a merge.
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  typedef T T2 __attribute__((ext_vector_type(2)));
  typedef float F2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((F2){lo, hi}, T2));
}

template <typename T, int VEC>
__device__ __forceinline__ Pack<T, VEC> pack(const float (&in)[VEC]) {
  Pack<T, VEC> r;
  if constexpr (std::is_same<T, float>::value) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) r.w[i] = f32_bits(in[i]);
  } else if constexpr (sizeof(T) * VEC < 4) {
    r.h = __builtin_bit_cast(uint16_t, from_f32<T>(in[0]));
  } else {
#pragma unroll
    for (int k = 0; k < VEC / 2; ++k) r.w[k] = pack2<T>(in[2 * k], in[2 * k + 1]);
  }
  return r;
}

// One element of a pack, widened to fp32.
template <typename T, int VEC>
__device__ __forceinline__ float pack_elem(const Pack<T, VEC>& r, int i) {
  float x[VEC];
  unpack(r, x);
  return x[i];
}

// A pack with every element equal to `value` (rounded to T).
template <typename T, int VEC>
__device__ __forceinline__ Pack<T, VEC> splat_pack(float value) {
  float x[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) x[i] = value;
  return pack<T, VEC>(x);
}

// A uniform load issued on the scalar unit (s_load, counted by lgkmcnt): the
// pointer is read as constant memory, so use it only on data that the kernel
// never writes. A vector load of the same value would be counted by vmcnt,
// and waiting for it would also wait for every older vector load or store.
template <typename T>
__device__ __forceinline__ T scalar_load(const T* p) {
  return *(const __attribute__((address_space(4))) T*)p;
}

// word 3 of a raw buffer descriptor on gfx9-family parts (32-bit data format, no swizzle)
constexpr int kRsrcWord3 = 0x00020000;

// Keep the optimiser from reusing values derived from the pack across this
// point (it re-derives them from the raw words instead of keeping copies live).
template <typename T, int VEC>
__device__ __forceinline__ void make_opaque(Pack<T, VEC>& r) {
  if constexpr (sizeof(T) * VEC >= 4) {
#pragma unroll
    for (int k = 0; k < Pack<T, VEC>::kWords; ++k) asm volatile("" : "+v"(r.w[k]));
  }
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
// wave64 reductions on DPP lane moves (no LDS round trips): within each quad
// (lane ^ 1, lane ^ 2), then the half-row and row mirrors, then lane 15 of
// rows 0 and 2 into rows 1 and 3 and lane 31 into rows 2 and 3, which leaves
// the total in lane 63; every lane receives it through a readlane.
// ---------------------------------------------------------------------------
namespace dpp {
constexpr int kXor1 = 0xb1;        // quad_perm [1, 0, 3, 2]
constexpr int kXor2 = 0x4e;        // quad_perm [2, 3, 0, 1]
constexpr int kHalfMirror = 0x141; // row_half_mirror
constexpr int kMirror = 0x140;     // row_mirror
constexpr int kBcast15 = 0x142;    // row_bcast:15
constexpr int kBcast31 = 0x143;    // row_bcast:31
}  // namespace dpp

// lane value moved by the DPP pattern CTRL; rows outside ROW_MASK receive `old`
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_move(float old, float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, v),
                                                               CTRL, ROW_MASK, 0xf, false));
}
__device__ __forceinline__ float lane63(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_move<dpp::kXor1>(0.f, v);
  v += dpp_move<dpp::kXor2>(0.f, v);
  v += dpp_move<dpp::kHalfMirror>(0.f, v);
  v += dpp_move<dpp::kMirror>(0.f, v);
  v += dpp_move<dpp::kBcast15, 0xa>(0.f, v);
  v += dpp_move<dpp::kBcast31, 0xc>(0.f, v);
  return lane63(v);
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_move<dpp::kXor1>(v, v));
  v = fmaxf(v, dpp_move<dpp::kXor2>(v, v));
  v = fmaxf(v, dpp_move<dpp::kHalfMirror>(v, v));
  v = fmaxf(v, dpp_move<dpp::kMirror>(v, v));
  v = fmaxf(v, dpp_move<dpp::kBcast15, 0xa>(v, v));
  v = fmaxf(v, dpp_move<dpp::kBcast31, 0xc>(v, v));
  return lane63(v);
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
int blocks_per_cu(const void* kernel, int block);  // resident blocks a CU (occupancy), cached per kernel
int current_device();                // -1 on failure (error recorded)
int check_launch(const char* what);  // 0 or hipError_t after a launch

// A second stream on `device` (which must be current) for HBM-bound work that
// runs beside an MFMA-bound kernel of the caller's stream: default priority,
// non-blocking (no implicit ordering with the null stream), one per host
// thread and device, created on first use and kept until the process ends.
// nullptr on failure (error recorded).
hipStream_t side_stream(int device);
// Order `to` after the work enqueued on `from` so far (an event recorded on
// `from`, waited on by `to`; a stream capture follows the edge).
int stream_after(hipStream_t to, hipStream_t from);

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
