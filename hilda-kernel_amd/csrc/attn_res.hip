// AttnRes (attention over depth) for gfx950, row-wise and HBM-bound
// (kernels/attn_res.py):
//   k_i = round(round(v_i * rstd_i) * w_norm), rstd_i = 1/sqrt(mean(v_i^2) + eps)
//   score_i = <w_query, k_i>,  alpha = softmax_i(score),  h = sum_i alpha_i v_i
// over the N stacked blocks v_i of one token (attn_res.py:31-98), and the
// analytic backward of attn_res.py:101-190: dV, with dW_query / dW_norm summed
// over tokens.
//
// 256 lanes per token. Each lane owns P 16-byte packs of the D columns. The
// N per-block sums of a pass (sum of squares, then the scores; in the
// backward <dh, v_i>, then <dk_i, v_i>) are reduced together and exchanged
// through LDS once for all N: the streaming forms with one wave butterfly per
// value, the register-resident forms with one transposed butterfly for all N.
// For 16-bit inputs the sums whose both factors are 16-bit (v_i . v_i,
// w_query . k_i, dh . v_i) use the hardware two-element dot product. With
// per-element unpacking and fmas the forward issued 18 VALU instructions per
// element at N = 8 and was bound by them (146 us at [8, 4, 2048, 4096] bf16);
// at about 10 it runs within 6% of a copy kernel of its own access order.
//
// When a token's N rows fit in registers (N <= 8 and D <= 512*VEC, or
// N <= 16 and D <= 256*VEC; VEC = 8 for bf16/fp16, 4 for fp32) the register-resident
// kernels read V once per direction. Otherwise the streaming kernels keep the
// per-block scalars in LDS, so the loops over blocks stay rolled, and re-read
// the token's rows per pass (three times forward, four times backward; the
// N*D*es bytes stay in L2 between passes).
//
// In the backward each workgroup walks a run of tokens and keeps its
// dW_query / dW_norm partials in registers (P*VEC columns per lane; the
// resident form keeps their common factor only), writes one fp32 partial row
// pair per workgroup, and a column reduction adds the rows in fp64 (the
// reference uses fp32 atomics per token, attn_res.py:189-190).
#include "hk_common.h"
#include "colsum.h"
#include "../../include/hilda_kernel_amd.h"

#include <algorithm>
#include <type_traits>

namespace hk {
namespace {

constexpr int kMaxBlocks = 32;  // the reference's largest MAX_BLOCKS (attn_res.py:201-206)
constexpr int kNT = 256;        // lanes per token
constexpr int kNW = kNT / kWave;

constexpr int kU = 4;           // blocks whose loads are in flight together

template <int VEC, int NT = kNT>
__device__ __forceinline__ int64_t col_of(int j) {  // column of pack j of this lane (NT lanes per token)
  return ((int64_t)j * NT + threadIdx.x) * VEC;
}

// Per-block sums over the token's lanes: each lane adds its part for block i
// with add(i, part) (a wave reduction, then one LDS slot per wave and block);
// finish(n, out) sums the waves into out[0..n) (LDS). Two barriers per pass,
// whatever the block count.
template <int NW>
struct BlockSumsT {
  float* red;  // NW * kMaxBlocks floats of LDS
  __device__ __forceinline__ void add(int i, float part) const {
    part = wave_sum(part);
    if ((threadIdx.x & (kWave - 1)) == 0) red[(threadIdx.x / kWave) * kMaxBlocks + i] = part;
  }
  // add(i, v[i]) for every i < NB at once (NB a power of two): a transposed
  // butterfly keeps, at the exchange with lane ^ 32, half of the values (the
  // lane's half of the rows, plus the partner's copy of them), then half of
  // those at lane ^ 16, and so on; after log2(NB) such steps v[0] holds the sum
  // of row lane / (64 / NB) over the lanes differing in the top bits, and plain
  // exchanges over the low bits finish it. NB - 1 + 6 - log2(NB) shuffles in
  // all (10 for 8 rows) where NB separate wave sums take 6 NB.
  template <int NB>
  __device__ __forceinline__ void add_all(float (&v)[NB]) const {
    static_assert(NB >= 1 && NB <= kWave && (NB & (NB - 1)) == 0, "NB must be a power of two <= 64");
    const int lane = threadIdx.x & (kWave - 1);
    int o = kWave / 2;
#pragma unroll
    for (int h = NB / 2; h >= 1; h /= 2, o /= 2) {
      // all ones in the upper lanes of each pair of halves; a bitwise blend,
      // as a select on the array would become indexing by a lane value
      const uint32_t up = (lane & o) ? 0xffffffffu : 0u;
#pragma unroll
      for (int i = 0; i < h; ++i) {
        const uint32_t lo = f32_bits(v[i]), hi = f32_bits(v[i + h]);
        const float keep = bits_f32((hi & up) | (lo & ~up));
        const float give = bits_f32((lo & up) | (hi & ~up));
        v[i] = keep + __shfl_xor(give, o, kWave);
      }
    }
#pragma unroll
    for (; o >= 1; o /= 2) v[0] += __shfl_xor(v[0], o, kWave);
    constexpr int kSpan = kWave / NB;  // lanes that hold one row's sum
    if (lane % kSpan == 0) red[(threadIdx.x / kWave) * kMaxBlocks + lane / kSpan] = v[0];
  }
  __device__ __forceinline__ void finish(int n, float* out) const {
    __syncthreads();
    if ((int)threadIdx.x < n) {
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) t += red[w * kMaxBlocks + threadIdx.x];
      out[threadIdx.x] = t;
    }
    __syncthreads();
  }
};
using BlockSums = BlockSumsT<kNW>;

// Two 16-bit elements (the low and high halves of a word) at once: the
// hardware two-element dot product into fp32 (the products of 16-bit values
// are exact in fp32).
template <typename T>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (std::is_same<T, __bf16>::value) {
    typedef __bf16 T2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(T2, a), __builtin_bit_cast(T2, b), c, false);
  } else {
    typedef _Float16 T2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(T2, a), __builtin_bit_cast(T2, b), c, false);
  }
}

// acc + sum of the squares of a pack's elements
template <typename T, int VEC>
__device__ __forceinline__ float sumsq_pack(const Pack<T, VEC>& x, float acc) {
  if constexpr (sizeof(T) == 2 && VEC % 2 == 0) {
#pragma unroll
    for (int k = 0; k < VEC / 2; ++k) acc = dot2<T>(x.w[k], x.w[k], acc);
  } else {
    float f[VEC];
    unpack(x, f);
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc = fmaf(f[e], f[e], acc);
  }
  return acc;
}

// acc + <w_query, round(round(x * r) * w_norm)> over a pack (attn_res.py:70-73),
// w_norm already widened to fp32
template <typename T, int VEC>
__device__ __forceinline__ float score_pack(const Pack<T, VEC>& x, float r, const float (&wn)[VEC],
                                            const Pack<T, VEC>& q, float acc) {
  float f[VEC];
  unpack(x, f);
  if constexpr (sizeof(T) == 2 && VEC % 2 == 0) {
#pragma unroll
    for (int k = 0; k < VEC / 2; ++k) {
      Pack<T, 2> k1;
      k1.w[0] = pack2<T>(f[2 * k] * r, f[2 * k + 1] * r);
      float g[2];
      unpack(k1, g);
      acc = dot2<T>(pack2<T>(g[0] * wn[2 * k], g[1] * wn[2 * k + 1]), q.w[k], acc);
    }
  } else {
    float qf[VEC];
    unpack(q, qf);
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc = fmaf(qf[e], round_through<T>(round_through<T>(f[e] * r) * wn[e]), acc);
  }
  return acc;
}

template <typename T, int VEC>
__global__ __launch_bounds__(kNT) void attn_res_fwd_kernel(T* __restrict__ out, float* __restrict__ alpha_out,
                                                           float* __restrict__ rstd_out, const T* __restrict__ V,
                                                           const T* __restrict__ wq, const T* __restrict__ wn, int N,
                                                           int P, int64_t ntok, int64_t D, float eps) {
  __shared__ float red[kNW * kMaxBlocks];
  __shared__ float rs[kMaxBlocks], al[kMaxBlocks];
  const BlockSums bs{red};
  const int64_t tok = blockIdx.x;
  const int64_t bstride = ntok * D;  // elements between blocks i and i+1
  const T* v0 = V + tok * D;
  // pass 1: sums of squares -> rstd_i (kU blocks at a time, all their loads first)
  for (int i0 = 0; i0 < N; i0 += kU) {
    float part[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) part[u] = 0.f;
    for (int j = 0; j < P; ++j) {
      const int64_t c = col_of<VEC>(j);
      if (c < D) {
        Pack<T, VEC> pv[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u)
          if (i0 + u < N) pv[u] = load_pack<T, VEC>(v0 + (i0 + u) * bstride + c);
#pragma unroll
        for (int u = 0; u < kU; ++u)
          if (i0 + u < N) part[u] = sumsq_pack(pv[u], part[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u)
      if (i0 + u < N) bs.add(i0 + u, part[u]);
  }
  bs.finish(N, rs);
  if ((int)threadIdx.x < N) rs[threadIdx.x] = rsqrtf(rs[threadIdx.x] / (float)D + eps);
  __syncthreads();
  // pass 2: score_i = <w_query, round(round(v_i * rstd_i) * w_norm)>
  for (int i0 = 0; i0 < N; i0 += kU) {
    float part[kU], r[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      part[u] = 0.f;
      r[u] = i0 + u < N ? rs[i0 + u] : 0.f;
    }
    for (int j = 0; j < P; ++j) {
      const int64_t c = col_of<VEC>(j);
      if (c < D) {
        Pack<T, VEC> pv[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u)
          if (i0 + u < N) pv[u] = load_pack<T, VEC>(v0 + (i0 + u) * bstride + c);
        const Pack<T, VEC> q = load_pack<T, VEC>(wq + c);
        float w[VEC];
        unpack(load_pack<T, VEC>(wn + c), w);
#pragma unroll
        for (int u = 0; u < kU; ++u)
          if (i0 + u < N) part[u] = score_pack(pv[u], r[u], w, q, part[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u)
      if (i0 + u < N) bs.add(i0 + u, part[u]);
  }
  bs.finish(N, al);
  // softmax over the blocks (every lane; the N scores are in LDS)
  float m = -INFINITY;
  for (int i = 0; i < N; ++i) m = fmaxf(m, al[i]);
  float z = 0.f;
  for (int i = 0; i < N; ++i) z += exp_fast(al[i] - m);
  const float iz = 1.0f / z;
  __syncthreads();  // every lane has read the scores
  if ((int)threadIdx.x < N) {
    const float a = exp_fast(al[threadIdx.x] - m) * iz;
    al[threadIdx.x] = a;
    alpha_out[threadIdx.x * ntok + tok] = a;
    rstd_out[threadIdx.x * ntok + tok] = rs[threadIdx.x];
  }
  __syncthreads();
  // pass 3: h = sum_i alpha_i v_i
  for (int j = 0; j < P; ++j) {
    const int64_t c = col_of<VEC>(j);
    if (c < D) {
      float h[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) h[e] = 0.f;
      for (int i0 = 0; i0 < N; i0 += kU) {
        Pack<T, VEC> pv[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u)
          if (i0 + u < N) pv[u] = load_pack<T, VEC>(v0 + (i0 + u) * bstride + c);
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          if (i0 + u < N) {
            const float a = al[i0 + u];
            float x[VEC];
            unpack(pv[u], x);
#pragma unroll
            for (int e = 0; e < VEC; ++e) h[e] = fmaf(a, x[e], h[e]);
          }
        }
      }
      store_pack<T, VEC>(out + tok * D + c, pack<T, VEC>(h));
    }
  }
}

// Backward for tokens [blockIdx.x * tpb, +tpb): dV written, dW partial rows
// part[blockIdx.x][2][D] (query, norm) in fp32. P: packs per lane (template,
// as the dW partials of P*VEC columns stay in registers).
template <typename T, int VEC, int P>
__global__ __launch_bounds__(kNT) void attn_res_bwd_kernel(T* __restrict__ dV, float* __restrict__ part,
                                                           const T* __restrict__ dh, const T* __restrict__ V,
                                                           const T* __restrict__ wq, const T* __restrict__ wn,
                                                           const float* __restrict__ alpha,
                                                           const float* __restrict__ rstd, int N, int64_t ntok,
                                                           int64_t D, int64_t tpb) {
  __shared__ float red[kNW * kMaxBlocks];
  __shared__ float da[kMaxBlocks], kv[kMaxBlocks], ds[kMaxBlocks], al[kMaxBlocks], rs[kMaxBlocks];
  const BlockSums bs{red};
  const int64_t bstride = ntok * D;
  float dwq[P][VEC], dwn[P][VEC];
#pragma unroll
  for (int j = 0; j < P; ++j)
#pragma unroll
    for (int e = 0; e < VEC; ++e) dwq[j][e] = dwn[j][e] = 0.f;
  const int64_t t0 = (int64_t)blockIdx.x * tpb, t1 = min(t0 + tpb, ntok);
  for (int64_t tok = t0; tok < t1; ++tok) {
    const T* v0 = V + tok * D;
    const T* g = dh + tok * D;
    if ((int)threadIdx.x < N) {
      al[threadIdx.x] = alpha[threadIdx.x * ntok + tok];
      rs[threadIdx.x] = rstd[threadIdx.x * ntok + tok];
    }
    // d_alpha_i = <dh, v_i>
    for (int i0 = 0; i0 < N; i0 += kU) {
      float p[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) p[u] = 0.f;
#pragma unroll
      for (int j = 0; j < P; ++j) {
        const int64_t c = col_of<VEC>(j);
        if (c < D) {
          Pack<T, VEC> pv[kU];
#pragma unroll
          for (int u = 0; u < kU; ++u)
            if (i0 + u < N) pv[u] = load_pack<T, VEC>(v0 + (i0 + u) * bstride + c);
          float y[VEC];
          unpack(load_pack<T, VEC>(g + c), y);
#pragma unroll
          for (int u = 0; u < kU; ++u) {
            if (i0 + u < N) {
              float x[VEC];
              unpack(pv[u], x);
#pragma unroll
              for (int e = 0; e < VEC; ++e) p[u] = fmaf(x[e], y[e], p[u]);
            }
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kU; ++u)
        if (i0 + u < N) bs.add(i0 + u, p[u]);
    }
    bs.finish(N, da);
    // softmax backward: ds_i = alpha_i (da_i - sum_j alpha_j da_j)  (attn_res.py:148-149)
    if ((int)threadIdx.x < N) {
      float sa = 0.f;
      for (int i = 0; i < N; ++i) sa = fmaf(al[i], da[i], sa);
      ds[threadIdx.x] = al[threadIdx.x] * (da[threadIdx.x] - sa);
    }
    __syncthreads();
    // <dk_i, v_i> with dk_i = ds_i * w_query * w_norm
    for (int i0 = 0; i0 < N; i0 += kU) {
      float p[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) p[u] = 0.f;
#pragma unroll
      for (int j = 0; j < P; ++j) {
        const int64_t c = col_of<VEC>(j);
        if (c < D) {
          Pack<T, VEC> pv[kU];
#pragma unroll
          for (int u = 0; u < kU; ++u)
            if (i0 + u < N) pv[u] = load_pack<T, VEC>(v0 + (i0 + u) * bstride + c);
          float q[VEC], w[VEC];
          unpack(load_pack<T, VEC>(wq + c), q);
          unpack(load_pack<T, VEC>(wn + c), w);
#pragma unroll
          for (int u = 0; u < kU; ++u) {
            if (i0 + u < N) {
              float x[VEC];
              unpack(pv[u], x);
#pragma unroll
              for (int e = 0; e < VEC; ++e) p[u] = fmaf(q[e] * w[e], x[e], p[u]);
            }
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kU; ++u)
        if (i0 + u < N) bs.add(i0 + u, p[u] * ds[i0 + u]);
    }
    bs.finish(N, kv);
    // dv_i = alpha_i dh + rstd dk - rstd^3 <dk, v>/D v; dW sums (attn_res.py:151-190)
#pragma unroll
    for (int j = 0; j < P; ++j) {
      const int64_t c = col_of<VEC>(j);
      if (c < D) {
        float y[VEC], q[VEC], w[VEC];
        unpack(load_pack<T, VEC>(g + c), y);
        unpack(load_pack<T, VEC>(wq + c), q);
        unpack(load_pack<T, VEC>(wn + c), w);
        for (int i0 = 0; i0 < N; i0 += kU) {
          Pack<T, VEC> pv[kU];
#pragma unroll
          for (int u = 0; u < kU; ++u)
            if (i0 + u < N) pv[u] = load_pack<T, VEC>(v0 + (i0 + u) * bstride + c);
#pragma unroll
          for (int u = 0; u < kU; ++u) {
            const int i = i0 + u;
            if (i < N) {
              const float a = al[i], d = ds[i], r = rs[i];
              const float coef = r * r * r * (kv[i] / (float)D);
              float x[VEC];
              unpack(pv[u], x);
#pragma unroll
              for (int e = 0; e < VEC; ++e) {
                const float dk = d * q[e] * w[e];
                const float vn = x[e] * r;
                dwq[j][e] = fmaf(d, vn * w[e], dwq[j][e]);
                dwn[j][e] = fmaf(d * q[e], vn, dwn[j][e]);
                x[e] = a * y[e] + r * dk - coef * x[e];
              }
              store_pack<T, VEC>(dV + i * bstride + tok * D + c, pack<T, VEC>(x));
            }
          }
        }
      }
    }
    __syncthreads();  // the token's LDS scalars are read before the next token overwrites them
  }
  float* pq = part + (int64_t)blockIdx.x * 2 * D;
#pragma unroll
  for (int j = 0; j < P; ++j) {
    const int64_t c = col_of<VEC>(j);
    if (c < D) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        pq[c + e] = dwq[j][e];
        pq[D + c + e] = dwn[j][e];
      }
    }
  }
}

// Register-resident forms, used when a token's N rows fit in NB*P packs per
// lane (64 VGPRs at most): V is read once per direction, the passes work on
// the registers. The per-element arithmetic is the streaming forms'; the
// cross-lane sums run in another order (all N blocks in one butterfly).
template <typename T, int VEC, int NB, int P, int NT>
__global__ __launch_bounds__(NT) void attn_res_fwd_res_kernel(T* __restrict__ out, float* __restrict__ alpha_out,
                                                               float* __restrict__ rstd_out, const T* __restrict__ V,
                                                               const T* __restrict__ wq, const T* __restrict__ wn,
                                                               int N, int64_t ntok, int64_t D, float eps) {
  // one token per workgroup: the workgroups resident on a CU overlap one
  // token's loads with another's reductions (measured faster than a run of
  // tokens per workgroup with the next token's rows prefetched). The weights
  // are loaded with the rows, so the token costs one memory round trip.
  __shared__ float red[NT / kWave * kMaxBlocks];
  __shared__ float rs[kMaxBlocks], al[kMaxBlocks];
  const BlockSumsT<NT / kWave> bs{red};
  const int64_t tok = blockIdx.x;
  const int64_t bstride = ntok * D;
  const T* v0 = V + tok * D;
  Pack<T, VEC> pv[NB][P], qv[P], wv[P];
#pragma unroll
  for (int j = 0; j < P; ++j) {
    const int64_t c = col_of<VEC, NT>(j) < D ? col_of<VEC, NT>(j) : 0;
    qv[j] = load_pack<T, VEC>(wq + c);
    wv[j] = load_pack<T, VEC>(wn + c);
  }
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int j = 0; j < P; ++j)
      if (i < N && col_of<VEC, NT>(j) < D) pv[i][j] = load_pack<T, VEC>(v0 + i * bstride + col_of<VEC, NT>(j));
  float part[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    float acc = 0.f;
    if (i < N) {
#pragma unroll
      for (int j = 0; j < P; ++j)
        if (col_of<VEC, NT>(j) < D) acc = sumsq_pack(pv[i][j], acc);
    }
    part[i] = acc;
  }
  bs.add_all(part);
  bs.finish(N, rs);
  if ((int)threadIdx.x < N) rs[threadIdx.x] = rsqrtf(rs[threadIdx.x] / (float)D + eps);
  __syncthreads();
  float wf[P][VEC];  // w_norm widened once for every block
#pragma unroll
  for (int j = 0; j < P; ++j) unpack(wv[j], wf[j]);
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    float acc = 0.f;
    if (i < N) {
      const float r = rs[i];
#pragma unroll
      for (int j = 0; j < P; ++j)
        if (col_of<VEC, NT>(j) < D) acc = score_pack(pv[i][j], r, wf[j], qv[j], acc);
    }
    part[i] = acc;
  }
  bs.add_all(part);
  bs.finish(N, al);
  float m = -INFINITY;
  for (int i = 0; i < N; ++i) m = fmaxf(m, al[i]);
  float z = 0.f;
  for (int i = 0; i < N; ++i) z += exp_fast(al[i] - m);
  const float iz = 1.0f / z;
  __syncthreads();
  if ((int)threadIdx.x < N) {
    const float a = exp_fast(al[threadIdx.x] - m) * iz;
    al[threadIdx.x] = a;
    alpha_out[threadIdx.x * ntok + tok] = a;
    rstd_out[threadIdx.x * ntok + tok] = rs[threadIdx.x];
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < P; ++j) {
    const int64_t c = col_of<VEC, NT>(j);
    if (c < D) {
      float h[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) h[e] = 0.f;
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        if (i < N) {
          const float a = al[i];
          float x[VEC];
          unpack(pv[i][j], x);
#pragma unroll
          for (int e = 0; e < VEC; ++e) h[e] = fmaf(a, x[e], h[e]);
        }
      }
      store_pack<T, VEC>(out + tok * D + c, pack<T, VEC>(h));
    }
  }
}

// acc + <a, b> over two packs
template <typename T, int VEC>
__device__ __forceinline__ float dot_pack(const Pack<T, VEC>& a, const Pack<T, VEC>& b, float acc) {
  if constexpr (sizeof(T) == 2 && VEC % 2 == 0) {
#pragma unroll
    for (int k = 0; k < VEC / 2; ++k) acc = dot2<T>(a.w[k], b.w[k], acc);
  } else {
    float x[VEC], y[VEC];
    unpack(a, x);
    unpack(b, y);
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc = fmaf(x[e], y[e], acc);
  }
  return acc;
}

// The two weight gradients share one factor (attn_res.py:181-187):
//   dW_query += ds_i * (v_i * rstd_i) * w_norm,  dW_norm += ds_i * w_query * (v_i * rstd_i)
// so each lane accumulates S = sum over its tokens and blocks of ds_i * rstd_i * v_i
// and the workgroup's partial rows are S * w_norm and S * w_query. dk_i =
// ds_i * w_query * w_norm enters dV and <dk_i, v_i> through the per-lane
// product w_query * w_norm, formed once.
template <typename T, int VEC, int NB, int P, int NT>
__global__ __launch_bounds__(NT) void attn_res_bwd_res_kernel(T* __restrict__ dV, float* __restrict__ part,
                                                               const T* __restrict__ dh, const T* __restrict__ V,
                                                               const T* __restrict__ wq, const T* __restrict__ wn,
                                                               const float* __restrict__ alpha,
                                                               const float* __restrict__ rstd, int N, int64_t ntok,
                                                               int64_t D, int64_t tpb) {
  __shared__ float red[NT / kWave * kMaxBlocks];
  __shared__ float da[kMaxBlocks], kv[kMaxBlocks], ds[kMaxBlocks], al[kMaxBlocks], rs[kMaxBlocks];
  const BlockSumsT<NT / kWave> bs{red};
  const int64_t bstride = ntok * D;
  const float inv_d = 1.0f / (float)D;
  float qw[P][VEC], S[P][VEC];
#pragma unroll
  for (int j = 0; j < P; ++j) {
    const int64_t c = col_of<VEC, NT>(j) < D ? col_of<VEC, NT>(j) : 0;
    float q[VEC], w[VEC];
    unpack(load_pack<T, VEC>(wq + c), q);
    unpack(load_pack<T, VEC>(wn + c), w);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      qw[j][e] = q[e] * w[e];
      S[j][e] = 0.f;
    }
  }
  const int64_t t0 = (int64_t)blockIdx.x * tpb, t1 = min(t0 + tpb, ntok);
  // the token's rows live in pv/gv; the next token's are loaded into them as the
  // current token's dV is stored (the last token reloads itself), so loads of
  // one token overlap the stores and reductions of the previous one
  Pack<T, VEC> pv[NB][P], gv[P];
  auto load_token = [&](int64_t t, int i, int j) {
    const int64_t c = col_of<VEC, NT>(j) < D ? col_of<VEC, NT>(j) : 0;  // in-bounds address; unused when >= D
    if (i < 0) gv[j] = load_pack<T, VEC>(dh + t * D + c);
    else pv[i][j] = load_pack<T, VEC>(V + i * bstride + t * D + c);
  };
  if (t0 < t1) {
#pragma unroll
    for (int j = 0; j < P; ++j) {
      load_token(t0, -1, j);
#pragma unroll
      for (int i = 0; i < NB; ++i)
        if (i < N) load_token(t0, i, j);
    }
  }
  float sums[NB];
  for (int64_t tok = t0; tok < t1; ++tok) {
    const int64_t nxt = tok + 1 < t1 ? tok + 1 : tok;
    if ((int)threadIdx.x < N) {
      al[threadIdx.x] = alpha[threadIdx.x * ntok + tok];
      rs[threadIdx.x] = rstd[threadIdx.x * ntok + tok];
    }
    // d_alpha_i = <dh, v_i>
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      float acc = 0.f;
      if (i < N) {
#pragma unroll
        for (int j = 0; j < P; ++j)
          if (col_of<VEC, NT>(j) < D) acc = dot_pack(pv[i][j], gv[j], acc);
      }
      sums[i] = acc;
    }
    bs.add_all(sums);
    bs.finish(N, da);
    if ((int)threadIdx.x < N) {
      float sa = 0.f;
      for (int i = 0; i < N; ++i) sa = fmaf(al[i], da[i], sa);
      ds[threadIdx.x] = al[threadIdx.x] * (da[threadIdx.x] - sa);
    }
    __syncthreads();
    // <dk_i, v_i> = ds_i <w_query * w_norm, v_i>
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      float acc = 0.f;
      if (i < N) {
#pragma unroll
        for (int j = 0; j < P; ++j) {
          if (col_of<VEC, NT>(j) < D) {
            float x[VEC];
            unpack(pv[i][j], x);
#pragma unroll
            for (int e = 0; e < VEC; ++e) acc = fmaf(qw[j][e], x[e], acc);
          }
        }
        acc *= ds[i];
      }
      sums[i] = acc;
    }
    bs.add_all(sums);
    bs.finish(N, kv);
#pragma unroll
    for (int j = 0; j < P; ++j) {
      const int64_t c = col_of<VEC, NT>(j);
      float y[VEC];
      unpack(gv[j], y);
      load_token(nxt, -1, j);
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        if (i < N) {
          const float a = al[i], r = rs[i], dr = ds[i] * r;
          const float coef = r * r * r * (kv[i] * inv_d);  // rstd_i^3 <dk_i, v_i> / D
          float x[VEC];
          unpack(pv[i][j], x);
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            S[j][e] = fmaf(dr, x[e], S[j][e]);
            // alpha_i dh + rstd_i dk_i - rstd_i^3 <dk_i, v_i> / D v_i
            x[e] = fmaf(a, y[e], fmaf(dr, qw[j][e], -coef * x[e]));
          }
          if (c < D) store_pack<T, VEC>(dV + i * bstride + tok * D + c, pack<T, VEC>(x));
          load_token(nxt, i, j);
        }
      }
    }
    __syncthreads();
  }
  float* pq = part + (int64_t)blockIdx.x * 2 * D;
#pragma unroll
  for (int j = 0; j < P; ++j) {
    const int64_t c = col_of<VEC, NT>(j);
    if (c < D) {
      float q[VEC], w[VEC];
      unpack(load_pack<T, VEC>(wq + c), q);
      unpack(load_pack<T, VEC>(wn + c), w);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        pq[c + e] = S[j][e] * w[e];
        pq[D + c + e] = S[j][e] * q[e];
      }
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

// packs per lane for D columns of T
template <typename T>
int packs_per_lane(int64_t D) {
  constexpr int VEC = 16 / sizeof(T);
  return (int)cdiv(D / VEC, kNT);
}

// f(P) with P rounded up to 2, 4 or 8 (the backward keeps P*VEC dW columns per lane)
template <class F>
int dispatch_p(int P, F&& f) {
  if (P <= 2) return f(std::integral_constant<int, 2>{});
  if (P <= 4) return f(std::integral_constant<int, 4>{});
  return f(std::integral_constant<int, 8>{});
}

// The register-resident kernels hold NB x P 16-byte packs per lane; a token
// spreads over NT lanes. f(NT, NB, P) for the first form that fits N blocks of
// D columns, or -2 when none does (the streaming kernels then run).
template <typename T, class F>
int dispatch_resident(int N, int64_t D, F&& f) {
  using std::integral_constant;
  constexpr int VEC = 16 / sizeof(T);
  const int64_t P256 = cdiv(D / VEC, 256), P512 = cdiv(D / VEC, 512);
  if (N <= 8 && P256 <= 2)
    return f(integral_constant<int, 256>{}, integral_constant<int, 8>{}, integral_constant<int, 2>{});
  if (N <= 16 && P256 <= 1)
    return f(integral_constant<int, 256>{}, integral_constant<int, 16>{}, integral_constant<int, 1>{});
  if (N <= 8 && P512 <= 2)
    return f(integral_constant<int, 512>{}, integral_constant<int, 8>{}, integral_constant<int, 2>{});
  if (N <= 16 && P512 <= 1)
    return f(integral_constant<int, 512>{}, integral_constant<int, 16>{}, integral_constant<int, 1>{});
  return -2;
}

// workgroups walking runs of tokens: per_cu per CU (what the register use lets run at once)
int64_t token_groups(int64_t ntok, int per_cu) {
  const int dev = current_device();
  const int cu = dev >= 0 ? cu_count(dev) : 256;
  return std::max<int64_t>(1, std::min<int64_t>(ntok, (int64_t)cu * per_cu));
}
int64_t bwd_groups(int64_t ntok) { return token_groups(ntok, 2); }

}  // namespace
}  // namespace hk

using namespace hk;

extern "C" {

int hk_attn_res_fwd(void* out, float* alpha, float* rstd, const void* V, const void* w_query, const void* w_norm,
                    int64_t n_blocks, int64_t n_tokens, int64_t D, float eps, int dtype, hk_stream_t stream) {
  HK_REQUIRE(n_blocks >= 1 && n_blocks <= kMaxBlocks, "AttnRes supports 1..%d blocks (got %lld)", kMaxBlocks,
             (long long)n_blocks);
  HK_REQUIRE(n_tokens >= 0 && D > 0 && n_tokens < (1LL << 31), "invalid shape");
  HK_REQUIRE(n_tokens == 0 || (out && alpha && rstd && V && w_query && w_norm), "null pointer argument");
  hipStream_t st = (hipStream_t)stream;
  return dispatch_t(dtype, [&](auto tag) -> int {
    using T = typename decltype(tag)::type;
    constexpr int VEC = 16 / sizeof(T);
    HK_REQUIRE(D % VEC == 0 && D <= 8 * kNT * VEC, "D must be a multiple of %d and at most %d", VEC, 8 * kNT * VEC);
    HK_REQUIRE(aligned_to(V, 16) && aligned_to(out, 16) && aligned_to(w_query, 16) && aligned_to(w_norm, 16),
               "16-byte aligned tensors expected");
    if (n_tokens == 0) return HK_OK;
    const int P = packs_per_lane<T>(D);
    const int N = (int)n_blocks;
    const int rc = dispatch_resident<T>(N, D, [&](auto ntc, auto nbc, auto pc) {
      constexpr int NT = decltype(ntc)::value, NB = decltype(nbc)::value, PP = decltype(pc)::value;
      hipLaunchKernelGGL((attn_res_fwd_res_kernel<T, VEC, NB, PP, NT>), dim3((unsigned)n_tokens), dim3(NT), 0, st,
                         (T*)out, alpha, rstd, (const T*)V, (const T*)w_query, (const T*)w_norm, N, n_tokens, D, eps);
      return check_launch("attn_res_fwd_res_kernel");
    });
    if (rc != -2) return rc;
    hipLaunchKernelGGL((attn_res_fwd_kernel<T, VEC>), dim3((unsigned)n_tokens), dim3(kNT), 0, st, (T*)out, alpha,
                       rstd, (const T*)V, (const T*)w_query, (const T*)w_norm, N, P, n_tokens, D, eps);
    return check_launch("attn_res_fwd_kernel");
  });
}

size_t hk_attn_res_bwd_workspace_size(int64_t n_tokens, int64_t D) {
  return (size_t)bwd_groups(n_tokens) * 2 * (size_t)D * 4;
}

int hk_attn_res_bwd(void* dV, void* dw_query, void* dw_norm, const void* dh, const void* V, const void* w_query,
                    const void* w_norm, const float* alpha, const float* rstd, int64_t n_blocks, int64_t n_tokens,
                    int64_t D, int dtype, void* workspace, size_t workspace_bytes, hk_stream_t stream) {
  HK_REQUIRE(n_blocks >= 1 && n_blocks <= kMaxBlocks, "AttnRes supports 1..%d blocks (got %lld)", kMaxBlocks,
             (long long)n_blocks);
  HK_REQUIRE(n_tokens >= 0 && D > 0 && n_tokens < (1LL << 31), "invalid shape");
  HK_REQUIRE(dw_query && dw_norm && w_query && w_norm, "null pointer argument");
  HK_REQUIRE(n_tokens == 0 || (dV && dh && V && alpha && rstd), "null pointer argument");
  const size_t need = hk_attn_res_bwd_workspace_size(n_tokens, D);
  HK_REQUIRE(workspace && workspace_bytes >= need && aligned_to(workspace, 16),
             "workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
  hipStream_t st = (hipStream_t)stream;
  return dispatch_t(dtype, [&](auto tag) -> int {
    using T = typename decltype(tag)::type;
    constexpr int VEC = 16 / sizeof(T);
    HK_REQUIRE(D % VEC == 0 && D <= 8 * kNT * VEC, "D must be a multiple of %d and at most %d", VEC, 8 * kNT * VEC);
    HK_REQUIRE(aligned_to(V, 16) && aligned_to(dV, 16) && aligned_to(dh, 16) && aligned_to(w_query, 16) &&
                   aligned_to(w_norm, 16),
               "16-byte aligned tensors expected");
    float* part = (float*)workspace;
    const int N = (int)n_blocks;
    int64_t used = 0;  // partial dW rows written
    if (n_tokens > 0) {
      int rc = dispatch_resident<T>(N, D, [&](auto ntc, auto nbc, auto pc) {
        constexpr int NT = decltype(ntc)::value, NB = decltype(nbc)::value, PP = decltype(pc)::value;
        // the register use lets two 256-lane workgroups, or one 512-lane one, run per CU
        const int64_t groups = token_groups(n_tokens, NT == 256 ? 2 : 1);
        const int64_t tpb = cdiv(n_tokens, groups);
        used = cdiv(n_tokens, tpb);
        hipLaunchKernelGGL((attn_res_bwd_res_kernel<T, VEC, NB, PP, NT>), dim3((unsigned)used), dim3(NT), 0, st,
                           (T*)dV, part, (const T*)dh, (const T*)V, (const T*)w_query, (const T*)w_norm, alpha, rstd,
                           N, n_tokens, D, tpb);
        return check_launch("attn_res_bwd_res_kernel");
      });
      if (rc == -2) {
        const int64_t groups = bwd_groups(n_tokens);
        const int64_t tpb = cdiv(n_tokens, groups);
        used = cdiv(n_tokens, tpb);
        rc = dispatch_p(packs_per_lane<T>(D), [&](auto pc) {
          constexpr int PP = decltype(pc)::value;
          hipLaunchKernelGGL((attn_res_bwd_kernel<T, VEC, PP>), dim3((unsigned)used), dim3(kNT), 0, st, (T*)dV, part,
                             (const T*)dh, (const T*)V, (const T*)w_query, (const T*)w_norm, alpha, rstd, N, n_tokens,
                             D, tpb);
          return check_launch("attn_res_bwd_kernel");
        });
      }
      if (rc) return rc;
    }
    // partial row pairs [query | norm] of 2D columns
    colsum_launch<T>((T*)dw_query, (T*)dw_norm, (const float*)part, used, 2 * D, 2 * D, D, st);
    return check_launch("colsum_kernel");
  });
}

}  // extern "C"
