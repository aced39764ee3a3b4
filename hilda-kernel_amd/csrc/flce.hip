// FusedLinearCrossEntropy for gfx950: lm_head GEMMs on bf16/fp16 MFMA with the
// cross-entropy gradient produced chunk by chunk, so the full (BT, V) logits
// never exist.
//
// Every contraction is one "NT" GEMM, C[M,N] = A[M,K] * B[N,K]^T with both
// operands K-contiguous, the layout the MFMA operand fetch wants:
//   logits_c = X_c  * W^T          A = X_c  [C,H],  B = W   [V,H]
//   dX_c     = D_c  * (W^T)^T      A = D_c  [C,V],  B = W^T [H,V]
//   dW      += D_c^T * X_c          A = D_c^T[V,C],  B = X^T [H,C] (columns of X^T)
// W^T and X^T are transposed once per call, D_c^T once per chunk (tiled LDS
// transposes, HBM-bound and small next to the GEMMs). dW accumulates in fp32
// across chunks; the last chunk's epilogue writes the bf16 result.
//
// GEMM kernel: 256x256 output tile per workgroup of 4 waves (2x2), each wave a
// 128x128 sub-tile of 4x4 v_mfma_f32_32x32x16 tiles (256 fp32 accumulators per
// lane). K advances 64 per stage; A and B stage tiles (2 x 32 KiB) are
// double-buffered in LDS with a 16-byte-chunk XOR swizzle so the MFMA operand
// reads (32 rows x 16 bytes per half-wave) are bank-conflict free. The next
// stage's global loads are issued before the current stage's MFMAs. Workgroups
// are renumbered so each XCD walks a contiguous band of output tiles (its L2
// keeps the shared A/B panels), grouped by M within the band.
#include "hk_common.h"
#include "hk_internal.h"
#include "../../include/hilda_kernel_amd.h"

#include <algorithm>
#include <type_traits>

namespace hk {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kThreads = 256;
constexpr int kTM = 4, kTN = 4;     // 32x32 MFMA tiles per wave in M and N
constexpr int kStageElems = kBM * kBK;  // one operand tile (A or B) per stage
constexpr int kXcds = 8;
constexpr int kGroupM = 16;

template <typename T>
__device__ __forceinline__ f32x16_t mfma32(const u32x4& a, const u32x4& b, const f32x16_t& c) {
  if constexpr (std::is_same<T, __bf16>::value)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
}

// element offset of (row, 8-element chunk kc) in a swizzled [rows][64] stage tile
__device__ __forceinline__ int swz(int row, int kc) { return row * kBK + ((kc ^ (row & 7)) << 3); }

struct GemmShape {
  int M, N, K;
  int64_t lda, ldb;
};

// Output tile (tm, tn) of this workgroup: XCD-banded, then grouped by kGroupM.
__device__ __forceinline__ void tile_of_block(int nbm, int nbn, int* tm, int* tn) {
  const int total = nbm * nbn;
  const int pid = blockIdx.x;
  const int q = total / kXcds, r = total % kXcds;
  const int xcd = pid % kXcds, local = pid / kXcds;
  const int logical = xcd < r ? xcd * (q + 1) + local : r * (q + 1) + (xcd - r) * q + local;
  const int per_group = kGroupM * nbn;
  const int group = logical / per_group;
  const int first_m = group * kGroupM;
  const int gsize = min(nbm - first_m, kGroupM);
  const int in_group = logical - group * per_group;
  *tm = first_m + in_group % gsize;
  *tn = in_group / gsize;
}

// Epilogues receive each lane's 32x32 accumulator tile: element e of tile (i, j)
// sits at row i*32 + (e/4)*8 + (lane/32)*4 + e%4 and column j*32 + lane%32 of
// the wave's 128x128 sub-tile (the CDNA 32x32 accumulator layout).
template <typename T>
struct EpiStore {  // C (T) = acc
  T* C;
  int64_t ldc;
  __device__ __forceinline__ void operator()(int row, int col, float v) const { C[row * ldc + col] = from_f32<T>(v); }
};

// fp32 accumulator across calls; the last call writes T.
// MODE 0: acc = v; 1: acc += v; 2: out = acc + v; 3: out = v
template <typename T, int MODE>
struct EpiAccum {
  float* acc;
  T* out;
  int64_t ld;
  __device__ __forceinline__ void operator()(int row, int col, float v) const {
    const int64_t o = row * ld + col;
    if constexpr (MODE == 0) acc[o] = v;
    else if constexpr (MODE == 1) acc[o] += v;
    else if constexpr (MODE == 2) out[o] = from_f32<T>(acc[o] + v);
    else out[o] = from_f32<T>(v);
  }
};

template <typename T, class Epi>
__global__ __launch_bounds__(kThreads) void gemm_nt_kernel(const T* __restrict__ A, const T* __restrict__ B,
                                                           GemmShape g, Epi epi) {
  __shared__ __attribute__((aligned(16))) T lds[2][2][kStageElems];  // [stage][A|B]: 128 KiB

  const int nbm = (g.M + kBM - 1) / kBM, nbn = (g.N + kBN - 1) / kBN;
  int tm, tn;
  tile_of_block(nbm, nbn, &tm, &tn);
  const int m0 = tm * kBM, n0 = tn * kBN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // global -> LDS mapping: 8 chunks of 16 bytes per thread and operand,
  // chunk c = tid + i*256 covers row c/8 (= tid/8 + 32i), k-chunk c%8 (= tid%8)
  const int lrow = tid >> 3, lkc = tid & 7;

  f32x16_t acc[kTM][kTN];
#pragma unroll
  for (int i = 0; i < kTM; ++i)
#pragma unroll
    for (int j = 0; j < kTN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  u32x4 ra[8], rb[8];
  auto gload = [&](int k0) {
    const int gk = k0 + lkc * 8;
    const bool kok = gk < g.K;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = lrow + i * 32;
      const int gm = m0 + r, gn = n0 + r;
      ra[i] = (kok && gm < g.M) ? *reinterpret_cast<const u32x4*>(A + (int64_t)gm * g.lda + gk) : u32x4{0, 0, 0, 0};
      rb[i] = (kok && gn < g.N) ? *reinterpret_cast<const u32x4*>(B + (int64_t)gn * g.ldb + gk) : u32x4{0, 0, 0, 0};
    }
  };
  auto lstore = [&](int s) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = lrow + i * 32;
      *reinterpret_cast<u32x4*>(&lds[s][0][swz(r, lkc)]) = ra[i];
      *reinterpret_cast<u32x4*>(&lds[s][1][swz(r, lkc)]) = rb[i];
    }
  };

  const int KT = (g.K + kBK - 1) / kBK;
  gload(0);
  lstore(0);
  __syncthreads();

  const int fr = lane & 31, fk = lane >> 5;  // MFMA operand lane -> (row, 8-wide k half)
  for (int kt = 0; kt < KT; ++kt) {
    const int s = kt & 1;
    if (kt + 1 < KT) gload((kt + 1) * kBK);
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      u32x4 af[kTM], bfr[kTN];
#pragma unroll
      for (int i = 0; i < kTM; ++i) {
        const int r = wm * 128 + i * 32 + fr;
        af[i] = *reinterpret_cast<const u32x4*>(&lds[s][0][swz(r, ks * 2 + fk)]);
      }
#pragma unroll
      for (int j = 0; j < kTN; ++j) {
        const int r = wn * 128 + j * 32 + fr;
        bfr[j] = *reinterpret_cast<const u32x4*>(&lds[s][1][swz(r, ks * 2 + fk)]);
      }
#pragma unroll
      for (int i = 0; i < kTM; ++i)
#pragma unroll
        for (int j = 0; j < kTN; ++j) acc[i][j] = mfma32<T>(af[i], bfr[j], acc[i][j]);
    }
    if (kt + 1 < KT) lstore(s ^ 1);
    __syncthreads();
  }

  // epilogue
#pragma unroll
  for (int i = 0; i < kTM; ++i)
#pragma unroll
    for (int j = 0; j < kTN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = m0 + wm * 128 + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
        const int col = n0 + wn * 128 + j * 32 + (lane & 31);
        if (row < g.M && col < g.N) epi(row, col, acc[i][j][e]);
      }
}

// out[c, r] = in[r, c] for a rows x cols matrix (row strides ld_in, ld_out);
// output columns r in [rows, rows_pad) are written as zeros. 64x64 tiles through LDS.
template <typename T>
__global__ __launch_bounds__(256) void transpose_kernel(T* __restrict__ out, const T* __restrict__ in, int64_t rows,
                                                        int64_t rows_pad, int64_t cols, int64_t ld_in,
                                                        int64_t ld_out) {
  __shared__ T tile[64][65];
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int y = ty + i * 4;
    const int64_t r = r0 + y, c = c0 + tx;
    tile[y][tx] = (r < rows && c < cols) ? in[r * ld_in + c] : from_f32<T>(0.f);
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int y = ty + i * 4;
    const int64_t c = c0 + y, r = r0 + tx;
    if (r < rows_pad && c < cols) out[c * ld_out + r] = tile[tx][y];
  }
}

template <typename T> struct Tag { using type = T; };

template <typename T, class Epi>
int launch_gemm(const T* A, const T* B, int M, int N, int K, int64_t lda, int64_t ldb, Epi epi, hipStream_t st) {
  if (M == 0 || N == 0) return HK_OK;
  GemmShape g{M, N, K, lda, ldb};
  const int64_t blocks = (int64_t)((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN);
  hipLaunchKernelGGL((gemm_nt_kernel<T, Epi>), dim3((unsigned)blocks), dim3(kThreads), 0, st, A, B, g, epi);
  return check_launch("gemm_nt_kernel");
}

template <typename T>
int launch_transpose(T* out, const T* in, int64_t rows, int64_t rows_pad, int64_t cols, int64_t ld_in,
                     int64_t ld_out, hipStream_t st) {
  if (rows_pad == 0 || cols == 0) return HK_OK;
  const dim3 grid((unsigned)cdiv(cols, 64), (unsigned)cdiv(rows_pad, 64));
  hipLaunchKernelGGL((transpose_kernel<T>), grid, dim3(256), 0, st, out, in, rows, rows_pad, cols, ld_in, ld_out);
  return check_launch("transpose_kernel");
}

int64_t pad8(int64_t x) { return (x + 7) & ~(int64_t)7; }

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct FlceLayout {
  size_t wt, xt, lg, dt, dwacc, nvalid, total;
};

FlceLayout flce_layout(int64_t BT, int64_t H, int64_t V, int64_t chunk, int es, bool grad) {
  FlceLayout L{};
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += align256(bytes);
    return o;
  };
  L.nvalid = take(256);
  L.lg = take((size_t)chunk * V * es);
  if (grad) {
    L.wt = take((size_t)H * V * es);
    L.xt = take((size_t)H * pad8(BT) * es);
    L.dt = take((size_t)V * pad8(chunk) * es);
    L.dwacc = BT > chunk ? take((size_t)V * H * 4) : 0;
  }
  L.total = off;
  return L;
}

// Rows per chunk: a multiple of 8 (chunk starts stay 16-byte aligned in X^T), at most BT.
int64_t flce_chunk(int64_t BT, int64_t chunk) {
  if (chunk <= 0) chunk = 4096;
  chunk = std::max<int64_t>(8, chunk & ~(int64_t)7);
  return std::min<int64_t>(chunk, BT > 0 ? BT : 1);
}

}  // namespace
}  // namespace hk

using namespace hk;

extern "C" {

size_t hk_fused_linear_cross_entropy_workspace_size(int64_t BT, int64_t H, int64_t V, int64_t chunk, int dtype,
                                                    int with_grad) {
  if (BT < 0 || H <= 0 || V <= 0 || (dtype != HK_BF16 && dtype != HK_F16)) return 0;
  return flce_layout(BT, H, V, flce_chunk(BT, chunk), 2, with_grad != 0).total;
}

int hk_fused_linear_cross_entropy(float* loss_out, float* loss_rows, void* dhidden, void* dweight, const void* hidden,
                                  const void* weight, const int64_t* targets, const float* row_scale, int64_t BT,
                                  int64_t H, int64_t V, int64_t ignore_index, int reduction, int dtype, int64_t chunk,
                                  void* workspace, size_t workspace_bytes, hk_stream_t stream) {
  HK_REQUIRE(dtype == HK_BF16 || dtype == HK_F16, "fused linear cross entropy supports bf16 and fp16 (got %d)",
             dtype);
  HK_REQUIRE(BT >= 0 && H > 0 && V > 0, "invalid shape BT=%lld H=%lld V=%lld", (long long)BT, (long long)H,
             (long long)V);
  HK_REQUIRE(H % 8 == 0 && V % 8 == 0, "H and V must be multiples of 8 (16-byte rows)");
  HK_REQUIRE(BT < (1LL << 31) && H < (1LL << 31) && V < (1LL << 31) - 4096, "dimension too large");
  HK_REQUIRE(reduction >= HK_REDUCTION_NONE && reduction <= HK_REDUCTION_SUM, "invalid reduction %d", reduction);
  const bool grad = dhidden != nullptr || dweight != nullptr;
  HK_REQUIRE(!grad || (dhidden && dweight), "dhidden and dweight are computed together");
  HK_REQUIRE(loss_rows && hidden && weight && targets, "null pointer argument");
  HK_REQUIRE(aligned_to(hidden, 16) && aligned_to(weight, 16) && (!grad || (aligned_to(dhidden, 16) &&
                                                                             aligned_to(dweight, 16))),
             "hidden, weight and gradients must be 16-byte aligned");
  const int64_t C = flce_chunk(BT, chunk);
  const FlceLayout lay = flce_layout(BT, H, V, C, 2, grad);
  HK_REQUIRE(workspace && workspace_bytes >= lay.total, "workspace too small: need %zu bytes, got %zu", lay.total,
             workspace_bytes);
  HK_REQUIRE(aligned_to(workspace, 256), "workspace must be 256-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  int* n_valid = (int*)(ws + lay.nvalid);
  // every target equal to ignore_index is ignored (fused_linear_cross_entropy.py:121,62-65);
  // unlike the CrossEntropy op, -1 is not a "no ignore" sentinel here
  const int has_ignore = 1;
  const int64_t BTp = pad8(BT);

  auto run = [&](auto tag) -> int {
    using T = typename decltype(tag)::type;
    const int dt = dtype;
    const T* X = (const T*)hidden;
    const T* W = (const T*)weight;
    T* Lg = (T*)(ws + lay.lg);
    int rc = HK_OK;
    if (BT > 0) rc = count_valid_launch(n_valid, targets, BT, ignore_index, has_ignore, st);
    if (rc) return rc;
    T* Wt = grad ? (T*)(ws + lay.wt) : nullptr;
    T* Xt = grad ? (T*)(ws + lay.xt) : nullptr;
    T* Dt = grad ? (T*)(ws + lay.dt) : nullptr;
    float* dwacc = (grad && lay.dwacc) ? (float*)(ws + lay.dwacc) : nullptr;
    if (grad) {
      rc = launch_transpose<T>(Wt, W, V, V, H, H, V, st);  // W^T [H, V]
      if (rc) return rc;
      rc = launch_transpose<T>(Xt, X, BT, BTp, H, H, BTp, st);  // X^T [H, BTp], zero padded
      if (rc) return rc;
    }
    const int64_t nchunks = BT > 0 ? cdiv(BT, C) : 0;
    for (int64_t ci = 0; ci < nchunks; ++ci) {
      const int64_t r0 = ci * C;
      const int64_t cs = std::min<int64_t>(C, BT - r0);
      // logits_c = X_c W^T
      rc = launch_gemm<T>(X + r0 * H, W, (int)cs, (int)V, (int)H, H, H, EpiStore<T>{Lg, V}, st);
      if (rc) return rc;
      // per-row loss; with gradients, D_c = (softmax - onehot) * s * row_scale written over the logits
      rc = ce_rows_launch(grad ? (void*)Lg : nullptr, loss_rows + r0, Lg, targets + r0, cs, V, V, V, ignore_index,
                          has_ignore, n_valid, grad && reduction == HK_REDUCTION_MEAN,
                          row_scale ? row_scale + r0 : nullptr, dt, st);
      if (rc) return rc;
      if (!grad) continue;
      // dX_c = D_c W
      rc = launch_gemm<T>(Lg, Wt, (int)cs, (int)H, (int)V, V, V, EpiStore<T>{(T*)dhidden + r0 * H, H}, st);
      if (rc) return rc;
      // dW += D_c^T X_c; K = cs is padded to a multiple of 8 with zeros on both operands
      const int64_t csp = pad8(cs);
      rc = launch_transpose<T>(Dt, Lg, cs, csp, V, V, csp, st);
      if (rc) return rc;
      const int mode = nchunks == 1 ? 3 : ci == 0 ? 0 : ci + 1 == nchunks ? 2 : 1;
      auto dw_gemm = [&](auto epi) {
        return launch_gemm<T>(Dt, Xt + r0, (int)V, (int)H, (int)csp, csp, BTp, epi, st);
      };
      T* dWo = (T*)dweight;
      if (mode == 0) rc = dw_gemm(EpiAccum<T, 0>{dwacc, dWo, H});
      else if (mode == 1) rc = dw_gemm(EpiAccum<T, 1>{dwacc, dWo, H});
      else if (mode == 2) rc = dw_gemm(EpiAccum<T, 2>{dwacc, dWo, H});
      else rc = dw_gemm(EpiAccum<T, 3>{dwacc, dWo, H});
      if (rc) return rc;
    }
    if (grad && nchunks == 0) {
      // no rows: zero gradients
      rc = launch_gemm<T>(Dt, Xt, (int)V, (int)H, 0, 0, 0, EpiAccum<T, 3>{dwacc, (T*)dweight, H}, st);
      if (rc) return rc;
    }
    if (loss_out) {
      // with gradients the rows already carry 1/max(n_valid,1) for 'mean'; without, divide here
      const bool divide = !grad && reduction == HK_REDUCTION_MEAN && BT > 0;
      return sum_rows_launch(loss_out, loss_rows, BT, divide ? n_valid : nullptr, divide, st);
    }
    return HK_OK;
  };
  if (dtype == HK_BF16) return run(Tag<__bf16>{});
  return run(Tag<_Float16>{});
}

}  // extern "C"
