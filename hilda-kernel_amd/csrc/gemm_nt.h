// bf16/fp16 "NT" GEMM on gfx950 MFMA: C[M,N] = A[M,K] * B[N,K]^T, both operands
// K-contiguous, fp32 accumulation, result handed to an epilogue functor.
//
// One workgroup computes a BM x BN tile with WGM x WGN waves; each wave owns a
// (BM/WGM) x (BN/WGN) sub-tile made of 32x32 v_mfma_f32_32x32x16 tiles. K
// advances BK per stage through two LDS buffers (A and B stage tiles side by
// side). Stage tiles are [rows][BK] with the 16-byte chunk index XOR-swizzled
// by the row, so a half-wave reading 32 consecutive rows at one k-chunk hits
// distinct bank groups. The next stage's global loads are issued into
// registers before the current stage's MFMAs and written to the other LDS
// buffer after them (one barrier per stage). With FRAG_PIPE the MFMA operands
// of sub-step ks+1 are read from LDS while sub-step ks computes.
//
// Workgroups are renumbered so each of the 8 XCDs walks a contiguous band of
// output tiles (grouped by GROUP_M rows of tiles), keeping the shared A/B
// panels in that XCD's L2.
#pragma once

#include "hk_common.h"

#include <type_traits>

namespace hk {
namespace gemm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

template <int BM_, int BN_, int BK_, int WGM_, int WGN_, bool FRAG_PIPE_ = false, int GROUP_M_ = 16>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WGM = WGM_, WGN = WGN_;
  static constexpr bool FRAG_PIPE = FRAG_PIPE_;
  static constexpr int GROUP_M = GROUP_M_;
  static constexpr int NT = WGM * WGN * 64;       // threads per workgroup
  static constexpr int WTM = BM / WGM, WTN = BN / WGN;  // wave tile
  static constexpr int TM = WTM / 32, TN = WTN / 32;    // MFMA tiles per wave
  static constexpr int CPR = BK / 8;              // 16-byte chunks per stage row
  static constexpr int LA = BM * CPR / NT, LB = BN * CPR / NT;  // chunks per thread per stage
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32x32");
  static_assert(BK % 16 == 0 && (CPR == 2 || CPR == 4 || CPR == 8), "BK must be 16, 32 or 64");
  static_assert(BM * CPR % NT == 0 && BN * CPR % NT == 0, "stage tile must split evenly over the threads");
  static constexpr int STAGE = (BM + BN) * BK;    // elements per LDS stage
};

struct Shape {
  int M, N, K;
  int64_t lda, ldb;
};

template <typename T>
__device__ __forceinline__ f32x16_t mfma32(const u32x4& a, const u32x4& b, const f32x16_t& c) {
  if constexpr (std::is_same<T, __bf16>::value)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
}

// element offset of (row, 16-byte chunk kc) in a swizzled [rows][BK] stage tile
template <int BK>
__device__ __forceinline__ int swz(int row, int kc) {
  constexpr int CPR = BK / 8;
  int s;
  if constexpr (CPR == 8) s = row & 7;
  else if constexpr (CPR == 4) s = (row >> 1) & 3;
  else s = (row >> 2) & 1;
  return row * BK + ((kc ^ s) << 3);
}

template <int GROUP_M>
__device__ __forceinline__ void tile_of_block(int nbm, int nbn, int* tm, int* tn) {
  constexpr int kXcds = 8;
  const int total = nbm * nbn;
  const int pid = blockIdx.x;
  const int q = total / kXcds, r = total % kXcds;
  const int xcd = pid % kXcds, local = pid / kXcds;
  const int logical = xcd < r ? xcd * (q + 1) + local : r * (q + 1) + (xcd - r) * q + local;
  const int per_group = GROUP_M * nbn;
  const int group = logical / per_group;
  const int first_m = group * GROUP_M;
  const int gsize = min(nbm - first_m, GROUP_M);
  const int in_group = logical - group * per_group;
  *tm = first_m + in_group % gsize;
  *tn = in_group / gsize;
}

// Epilogue contract: epi(row, col, value) for every in-range element. Element
// e of 32x32 tile (i, j) of a wave sits at row i*32 + (e/4)*8 + (lane/32)*4 + e%4
// and column j*32 + lane%32 of the wave tile (the CDNA 32x32 accumulator layout).
template <typename T, class C, class Epi>
__global__ __launch_bounds__(C::NT) void gemm_nt_kernel(const T* __restrict__ A, const T* __restrict__ B, Shape g,
                                                        Epi epi) {
  __shared__ __attribute__((aligned(16))) T lds[2][C::STAGE];

  const int nbm = (g.M + C::BM - 1) / C::BM, nbn = (g.N + C::BN - 1) / C::BN;
  int tm, tn;
  tile_of_block<C::GROUP_M>(nbm, nbn, &tm, &tn);
  const int m0 = tm * C::BM, n0 = tn * C::BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / C::WGN, wn = wave % C::WGN;

  f32x16_t acc[C::TM][C::TN];
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // global -> LDS: chunk c = tid + i*NT covers row c / CPR, k-chunk c % CPR
  u32x4 ra[C::LA], rb[C::LB];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < C::LA; ++i) {
      const int c = tid + i * C::NT, r = c / C::CPR, kc = c % C::CPR;
      const int gm = m0 + r, gk = k0 + kc * 8;
      ra[i] = (gm < g.M && gk < g.K) ? *reinterpret_cast<const u32x4*>(A + (int64_t)gm * g.lda + gk)
                                     : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < C::LB; ++i) {
      const int c = tid + i * C::NT, r = c / C::CPR, kc = c % C::CPR;
      const int gn = n0 + r, gk = k0 + kc * 8;
      rb[i] = (gn < g.N && gk < g.K) ? *reinterpret_cast<const u32x4*>(B + (int64_t)gn * g.ldb + gk)
                                     : u32x4{0, 0, 0, 0};
    }
  };
  auto lstore = [&](int s) {
#pragma unroll
    for (int i = 0; i < C::LA; ++i) {
      const int c = tid + i * C::NT, r = c / C::CPR, kc = c % C::CPR;
      *reinterpret_cast<u32x4*>(&lds[s][swz<C::BK>(r, kc)]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < C::LB; ++i) {
      const int c = tid + i * C::NT, r = c / C::CPR, kc = c % C::CPR;
      *reinterpret_cast<u32x4*>(&lds[s][C::BM * C::BK + swz<C::BK>(r, kc)]) = rb[i];
    }
  };

  const int fr = lane & 31, fk = lane >> 5;  // operand lane -> (row in tile, 8-wide k half)
  auto frag = [&](int s, int ks, u32x4 (&af)[C::TM], u32x4 (&bf)[C::TN]) {
#pragma unroll
    for (int i = 0; i < C::TM; ++i) {
      const int r = wm * C::WTM + i * 32 + fr;
      af[i] = *reinterpret_cast<const u32x4*>(&lds[s][swz<C::BK>(r, ks * 2 + fk)]);
    }
#pragma unroll
    for (int j = 0; j < C::TN; ++j) {
      const int r = wn * C::WTN + j * 32 + fr;
      bf[j] = *reinterpret_cast<const u32x4*>(&lds[s][C::BM * C::BK + swz<C::BK>(r, ks * 2 + fk)]);
    }
  };
  auto mma = [&](const u32x4 (&af)[C::TM], const u32x4 (&bf)[C::TN]) {
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int j = 0; j < C::TN; ++j) acc[i][j] = mfma32<T>(af[i], bf[j], acc[i][j]);
  };

  const int KT = (g.K + C::BK - 1) / C::BK;
  gload(0);
  lstore(0);
  __syncthreads();

  for (int kt = 0; kt < KT; ++kt) {
    const int s = kt & 1;
    if (kt + 1 < KT) gload((kt + 1) * C::BK);
    if constexpr (C::FRAG_PIPE) {
      u32x4 af[2][C::TM], bf[2][C::TN];
      frag(s, 0, af[0], bf[0]);
#pragma unroll
      for (int ks = 0; ks < C::BK / 16; ++ks) {
        if (ks + 1 < C::BK / 16) frag(s, ks + 1, af[(ks + 1) & 1], bf[(ks + 1) & 1]);
        mma(af[ks & 1], bf[ks & 1]);
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < C::BK / 16; ++ks) {
        u32x4 af[C::TM], bf[C::TN];
        frag(s, ks, af, bf);
        mma(af, bf);
      }
    }
    if (kt + 1 < KT) lstore(s ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = m0 + wm * C::WTM + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
        const int col = n0 + wn * C::WTN + j * 32 + (lane & 31);
        if (row < g.M && col < g.N) epi(row, col, acc[i][j][e]);
      }
}

template <typename T, class C, class Epi>
int launch(const T* A, const T* B, int M, int N, int K, int64_t lda, int64_t ldb, Epi epi, hipStream_t st) {
  if (M == 0 || N == 0) return 0;
  Shape g{M, N, K, lda, ldb};
  const int64_t blocks = (int64_t)((M + C::BM - 1) / C::BM) * ((N + C::BN - 1) / C::BN);
  hipLaunchKernelGGL((gemm_nt_kernel<T, C, Epi>), dim3((unsigned)blocks), dim3(C::NT), 0, st, A, B, g, epi);
  return check_launch("gemm_nt_kernel");
}

}  // namespace gemm
}  // namespace hk
