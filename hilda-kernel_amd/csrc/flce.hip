// FusedLinearCrossEntropy, FusedLinearJSD and FusedLinear-GRPO for gfx950:
// lm_head GEMMs on MFMA (bf16/fp16, or fp32 for fp32 inputs) with the loss
// gradient produced chunk by chunk, so the full (BT, V) logits never exist.
//
// Every contraction is one "NT" GEMM (gemm_nt.h), C[M,N] = A[M,K] * B[N,K]^T
// with both operands K-contiguous, the layout the MFMA operand fetch wants:
//   logits_c = X_c  * W^T          A = X_c  [C,H],  B = W   [V,H]
//   dX_c     = D_c  * (W^T)^T      A = D_c  [C,V],  B = W^T [H,V]
//   dW      += D_c^T * X_c          A = D_c^T[V,C],  B = X^T [H,C] (columns of X^T)
// W^T and X^T are transposed once per call, D_c^T once per chunk (tiled LDS
// transposes, HBM-bound and small next to the GEMMs). dW is either one GEMM
// over all rows after the chunk loop (every chunk's D_c^T kept side by side,
// when that needs no more memory than the alternative) or accumulated in fp32
// across chunks (the GEMM epilogue reads and writes the accumulator in
// coalesced 16-byte chunks; the last chunk's epilogue writes the input dtype).
//
// Rows that need no logits (ignored targets or labels, masked GRPO positions)
// are compacted away on the device first; the GEMMs, transposes and row
// kernels read the live count from device memory, so the host never waits.
#include "hk_common.h"
#include "hk_internal.h"
#include "gemm_nt.h"
#include "../../include/hilda_kernel_amd.h"

#include <algorithm>
#include <type_traits>

namespace hk {
namespace {

using gemm::f32x4_t;
struct NoPrior {};

// Stores n (<= 4) fp32 values at p in T, one 8- or 16-byte store when n == 4.
template <typename T>
__device__ __forceinline__ void store4(T* p, const float* v, int n) {
  if (n == 4) {
    if constexpr (sizeof(T) == 4) *reinterpret_cast<f32x4_t*>(p) = f32x4_t{v[0], v[1], v[2], v[3]};
    else *reinterpret_cast<u32x2*>(p) = u32x2{gemm::pack2<T>(v[0], v[1]), gemm::pack2<T>(v[2], v[3])};
  } else {
    for (int e = 0; e < n; ++e) p[e] = from_f32<T>(v[e]);
  }
}

// C (T) = acc, in 16-byte chunks (8 columns of a 16-bit type, 4 of fp32).
template <typename T>
struct EpiStore {
  using Stage = T;
  using Prior = NoPrior;
  static constexpr bool kReads = false;
  T* C;
  int64_t ldc;  // a multiple of 8, so full chunks are 16-byte aligned
  __device__ __forceinline__ Prior load(int, int, int) const { return {}; }
  __device__ __forceinline__ void store(int row, int col, const T* v, int n, const Prior&) const {
    T* p = C + (int64_t)row * ldc + col;
    if (n == 16 / (int)sizeof(T)) {
      *reinterpret_cast<u32x4*>(p) = *reinterpret_cast<const u32x4*>(v);
    } else {
      for (int e = 0; e < n; ++e) p[e] = v[e];
    }
  }
};

// C (T) = acc with GEMM row r stored at row rows[r] of C (the live rows of a
// compacted operand back in place), in 16-byte chunks.
template <typename T>
struct EpiScatter {
  using Stage = T;
  using Prior = NoPrior;
  static constexpr bool kReads = false;
  T* C;
  int64_t ldc;  // a multiple of 8
  const int* rows;
  __device__ __forceinline__ Prior load(int, int, int) const { return {}; }
  __device__ __forceinline__ void store(int row, int col, const T* v, int n, const Prior&) const {
    T* p = C + (int64_t)rows[row] * ldc + col;
    if (n == 16 / (int)sizeof(T)) {
      *reinterpret_cast<u32x4*>(p) = *reinterpret_cast<const u32x4*>(v);
    } else {
      for (int e = 0; e < n; ++e) p[e] = v[e];
    }
  }
};

// fp32 accumulator across calls, 4 columns per chunk; the last call writes T.
// MODE 0: acc = v; 1: acc += v; 2: out = acc + v
template <typename T, int MODE>
struct EpiAccum {
  using Stage = float;
  using Prior = f32x4_t;
  static constexpr bool kReads = MODE != 0;
  float* acc;
  T* out;
  int64_t ld;  // a multiple of 8
  __device__ __forceinline__ Prior load(int row, int col, int n) const {
    const float* p = acc + (int64_t)row * ld + col;
    if (n == 4) return *reinterpret_cast<const f32x4_t*>(p);
    Prior x = {0.f, 0.f, 0.f, 0.f};
    for (int e = 0; e < n; ++e) x[e] = p[e];
    return x;
  }
  __device__ __forceinline__ void store(int row, int col, const float* v, int n, const Prior& x) const {
    const int64_t o = (int64_t)row * ld + col;
    float r[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = MODE == 0 ? v[e] : x[e] + v[e];
    if constexpr (MODE == 2) {
      store4<T>(out + o, r, n);
    } else {
      if (n == 4) {
        *reinterpret_cast<f32x4_t*>(acc + o) = f32x4_t{r[0], r[1], r[2], r[3]};
      } else {
        for (int e = 0; e < n; ++e) acc[o + e] = r[e];
      }
    }
  }
};

// n16 16-byte words of zeros
__global__ __launch_bounds__(256) void zero16_kernel(u32x4* __restrict__ p, int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride) p[i] = u32x4{0, 0, 0, 0};
}

// Compacted rows (rows of n16 16-byte words): out[i] = in[rowmap[i]] for
// i < *n_live, zero rows for i in [*n_live, rows).
__global__ __launch_bounds__(256) void gather_rows_kernel(u32x4* __restrict__ out, const u32x4* __restrict__ in,
                                                          const int* __restrict__ rowmap,
                                                          const int* __restrict__ n_live, int64_t rows, int64_t n16) {
  const int64_t n = *n_live;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    u32x4* o = out + r * n16;
    if (r < n) {
      const u32x4* src = in + (int64_t)rowmap[r] * n16;
      for (int64_t w = threadIdx.x; w < n16; w += 256) o[w] = src[w];
    } else {
      for (int64_t w = threadIdx.x; w < n16; w += 256) o[w] = u32x4{0, 0, 0, 0};
    }
  }
}

// Per-row CE inputs of the compacted rows: targets and the optional row scale.
__global__ __launch_bounds__(256) void gather_ce_kernel(int64_t* __restrict__ t_out, float* __restrict__ s_out,
                                                        const int64_t* __restrict__ t_in,
                                                        const float* __restrict__ s_in, const int* __restrict__ rowmap,
                                                        const int* __restrict__ n_live) {
  const int64_t n = *n_live;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int r = rowmap[i];
    t_out[i] = t_in[r];
    if (s_in) s_out[i] = s_in[r];
  }
}

// Rows of the original order after a compacted pass: dead rows (inv[r] < 0)
// get a zero dX row (when dX) and loss 0; live rows take their loss from the
// compacted losses (when loss_rows).
__global__ __launch_bounds__(256) void finish_rows_kernel(u32x4* __restrict__ dX, int64_t n16,
                                                          float* __restrict__ loss_rows,
                                                          const float* __restrict__ loss_c,
                                                          const int* __restrict__ inv, int64_t rows) {
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const int k = inv[r];
    if (loss_rows && threadIdx.x == 0) loss_rows[r] = k >= 0 ? loss_c[k] : 0.f;
    if (dX && k < 0)
      for (int64_t w = threadIdx.x; w < n16; w += 256) dX[r * n16 + w] = u32x4{0, 0, 0, 0};
  }
}

// out[c, r] = in[r, c] for a rows x cols matrix of a 16-bit type (row strides
// ld_in, ld_out, both multiples of 8; cols a multiple of 8); output columns r
// in [rows, rows_pad) are written as zeros (rows_pad a multiple of 8).
// 16-byte global loads and stores, the tile staged in LDS (layout below).
// With lim (a compacted input whose first *lim - lim_off rows are live), rows
// past that are read as zeros and zeros are written up to the next multiple
// of 64 of the bound, both relative to lim_off and absolute: what a GEMM
// whose K is cut by the same bound reads (at least 64 columns).
template <typename T>
__global__ __launch_bounds__(512) void transpose_kernel(T* __restrict__ out, const T* __restrict__ in, int64_t rows,
                                                        int64_t rows_pad, int64_t cols, int64_t ld_in,
                                                        int64_t ld_out, const int* __restrict__ lim,
                                                        int64_t lim_off) {
  static_assert(sizeof(T) == 2, "16-bit elements");
  // 128 x 128 tiles: 256-byte runs on both sides (a 64 x 64 tile's 128-byte
  // input runs from 256 KB rows ran at 2.3 TB/s). Lane (q, k) of unit i loads
  // input rows 2q and 2q+1 at 16-byte column chunk k; each column's pair of
  // elements becomes one 32-bit word (v_perm), stored column-major: word
  // (column j, pair q) at j*64 + (((q >> 2) ^ (j >> 3)) << 2 | (q & 3)). The XOR
  // of 4-word groups keeps the word writes (16 chunks of a wave, 16 groups) and
  // the 16-byte reads (16 lanes of one column, 16 groups) free of bank conflicts.
  __shared__ __attribute__((aligned(16))) uint32_t tile[128 * 64];
  const int t = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.y * 128, c0 = (int64_t)blockIdx.x * 128;
  if (lim) {
    const int64_t n = *lim, v = n - lim_off;
    rows = std::max<int64_t>(0, std::min<int64_t>(rows, v));
    const int64_t z = std::max<int64_t>(64, std::max<int64_t>((v + 63) / 64 * 64, (n + 63) / 64 * 64 - lim_off));
    rows_pad = std::min<int64_t>(rows_pad, z);
    if (r0 >= rows_pad) return;  // uniform
  }
  const int k = t & 15;
  u32x4 va[2], vb[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int q = (t >> 4) + 32 * i;
    const int64_t r = r0 + 2 * q, c = c0 + 8 * k;
    va[i] = u32x4{0u, 0u, 0u, 0u};
    vb[i] = u32x4{0u, 0u, 0u, 0u};
    if (c < cols) {
      if (r < rows) va[i] = *reinterpret_cast<const u32x4*>(in + r * ld_in + c);
      if (r + 1 < rows) vb[i] = *reinterpret_cast<const u32x4*>(in + (r + 1) * ld_in + c);
    }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int q = (t >> 4) + 32 * i;
    const int slot = (((q >> 2) ^ k) << 2) | (q & 3);  // j >> 3 == k for the 8 columns of chunk k
    const uint32_t a[4] = {va[i].x, va[i].y, va[i].z, va[i].w};
    const uint32_t b[4] = {vb[i].x, vb[i].y, vb[i].z, vb[i].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      // low half: row 2q's element of column 8k + e, high half: row 2q+1's
      const uint32_t w = __builtin_amdgcn_perm(b[e >> 1], a[e >> 1], (e & 1) ? 0x07060302u : 0x05040100u);
      tile[(8 * k + e) * 64 + slot] = w;
    }
  }
  __syncthreads();
  const int m = t & 15;  // output chunk: rows 8m .. 8m+7 of the tile, words 4m .. 4m+3
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int j = (t >> 4) + 32 * i;
    const int64_t c = c0 + j, r = r0 + 8 * m;
    const u32x4 v = *reinterpret_cast<const u32x4*>(tile + j * 64 + ((m ^ (j >> 3)) << 2));
    if (c < cols && r < rows_pad) *reinterpret_cast<u32x4*>(out + c * ld_out + r) = v;
  }
}

// The fp32 form of transpose_kernel (same arguments and zero padding): 64x64
// tiles of 16-byte (4-element) loads and stores, staged in LDS with a pitch of
// 65 floats so the column reads of a wave fall in distinct banks.
__global__ __launch_bounds__(256) void transpose32_kernel(float* __restrict__ out, const float* __restrict__ in,
                                                          int64_t rows, int64_t rows_pad, int64_t cols, int64_t ld_in,
                                                          int64_t ld_out, const int* __restrict__ lim,
                                                          int64_t lim_off) {
  constexpr int P = 65;
  __shared__ float tile[64 * P];
  const int t = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  if (lim) {
    const int64_t n = *lim, v = n - lim_off;
    rows = std::max<int64_t>(0, std::min<int64_t>(rows, v));
    const int64_t z = std::max<int64_t>(64, std::max<int64_t>((v + 63) / 64 * 64, (n + 63) / 64 * 64 - lim_off));
    rows_pad = std::min<int64_t>(rows_pad, z);
    if (r0 >= rows_pad) return;  // uniform
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int rr = t / 16 + 16 * k, cc = (t % 16) * 4;
    const int64_t r = r0 + rr, c = c0 + cc;
    f32x4_t v = {0.f, 0.f, 0.f, 0.f};
    if (r < rows && c < cols) v = *reinterpret_cast<const f32x4_t*>(in + r * ld_in + c);
#pragma unroll
    for (int e = 0; e < 4; ++e) tile[rr * P + cc + e] = v[e];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int oc = t / 16 + 16 * k, oq = (t % 16) * 4;
    const int64_t c = c0 + oc, r = r0 + oq;
    if (c < cols && r < rows_pad)
      *reinterpret_cast<f32x4_t*>(out + c * ld_out + r) =
          f32x4_t{tile[oq * P + oc], tile[(oq + 1) * P + oc], tile[(oq + 2) * P + oc], tile[(oq + 3) * P + oc]};
  }
}

// The dX GEMM's epilogue when it may split K. Unsplit (the GEMM's split count
// is 1), it stores the tile like EpiScatter / EpiStore, 4 columns a chunk; split,
// split s stores fp32 partial sums at part + (s * m + row) * ld, m the GEMM's
// bounded row count, and splitk_sum_kernel adds them up.
template <typename T>
struct EpiDx {
  using Stage = float;
  using Prior = NoPrior;
  static constexpr bool kReads = false;
  T* C;
  int64_t ldc;       // a multiple of 8
  const int* rows;   // nullable: GEMM row r goes to row rows[r] of C
  float* part;
  int64_t ld;        // a multiple of 4
  int split = 0, nsplit = 1, m = 0;
  __device__ __forceinline__ void set_split(int s, int ns, int bounded_m) {
    split = s;
    nsplit = ns;
    m = bounded_m;
  }
  __device__ __forceinline__ Prior load(int, int, int) const { return {}; }
  __device__ __forceinline__ void store(int row, int col, const float* v, int n, const Prior&) const {
    if (nsplit == 1) {
      store4<T>(C + (int64_t)(rows ? rows[row] : row) * ldc + col, v, n);
      return;
    }
    float* p = part + ((int64_t)split * m + row) * ld + col;
    if (n == 4) {
      *reinterpret_cast<f32x4_t*>(p) = f32x4_t{v[0], v[1], v[2], v[3]};
    } else {
      for (int e = 0; e < n; ++e) p[e] = v[e];
    }
  }
};

// C[rows ? rows[r] : r] = sum over the splits of the partials (rounded once to
// T), 8 columns a thread, for r below the device-bounded M. The split count is
// the GEMM's own (auto_splits of its bounded tiles); unsplit, the GEMM stored
// C itself and this returns at once.
template <typename T>
__global__ __launch_bounds__(256) void splitk_sum_kernel(T* __restrict__ C, int64_t ldc, const int* __restrict__ rows,
                                                         const float* __restrict__ part, int M, int N, int KT,
                                                         int max_s, const int* lim, int lim_off) {
  if (lim) M = min(M, max(0, *lim - lim_off));
  const int S = gemm::auto_splits(((M + 255) / 256) * ((N + 255) / 256), KT, max_s);
  if (S == 1) return;
  const int n8 = N / 8;
  const int64_t total = (int64_t)M * n8, stride = (int64_t)M * N;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int r = (int)(i / n8), c = (int)(i - (int64_t)r * n8) * 8;
    const float* p = part + (int64_t)r * N + c;
    f32x4_t a = *reinterpret_cast<const f32x4_t*>(p), b = *reinterpret_cast<const f32x4_t*>(p + 4);
    for (int s = 1; s < S; ++s) {
      a += *reinterpret_cast<const f32x4_t*>(p + s * stride);
      b += *reinterpret_cast<const f32x4_t*>(p + s * stride + 4);
    }
    T* o = C + (int64_t)(rows ? rows[r] : r) * ldc + c;
    const float va[4] = {a[0], a[1], a[2], a[3]}, vb[4] = {b[0], b[1], b[2], b[3]};
    store4<T>(o, va, 4);
    store4<T>(o + 4, vb, 4);
  }
}

// lim (nullable): a device-side bound on M (or K with lim_k), see gemm::Shape
template <typename T, class Epi>
int launch_gemm(const T* A, const T* B, int M, int N, int K, int64_t lda, int64_t ldb, Epi epi, hipStream_t st,
                const int* lim = nullptr, int lim_off = 0, bool lim_k = false, int ksplit = 1) {
  return gemm::launch<T>(A, B, M, N, K, lda, ldb, epi, st, lim, lim_off, lim_k, ksplit);
}

// Most K splits the dX GEMM (M = chunk rows, N = H, K = V) may take; the
// kernel picks auto_splits() of the tiles left after the live-row bound, so a
// short or mostly ignored chunk (a 2048-row chunk at H = 4096 is 128 output
// tiles) still fills the chip. 1: never split.
// bk: the GEMM's stage depth (K elements per K tile) for the input type.
int dx_max_splits(int64_t H, int64_t V, int bk) {
  if (V % bk != 0 || H % 8 != 0) return 1;
  return (int)std::min<int64_t>(8, V / bk / 16);
}

// fp32 partial-sum bytes the dX GEMM of a chunk of up to C rows can need: the
// largest splits x rows over the row counts it may be cut to.
size_t dx_part_bytes(int64_t C, int64_t H, int64_t V, int bk) {
  const int smax = dx_max_splits(H, V, bk);
  if (smax <= 1) return 0;
  size_t best = 0;
  const int64_t ntn = cdiv(H, 256), kt = V / bk;
  for (int64_t mt = 1; mt <= cdiv(C, 256); ++mt) {
    const int s = gemm::auto_splits((int)(mt * ntn), (int)kt, smax);
    if (s > 1) best = std::max(best, (size_t)s * (size_t)std::min<int64_t>(C, mt * 256) * H * 4);
  }
  return best;
}

template <typename T>
int launch_transpose(T* out, const T* in, int64_t rows, int64_t rows_pad, int64_t cols, int64_t ld_in,
                     int64_t ld_out, hipStream_t st, const int* lim = nullptr, int64_t lim_off = 0) {
  if (rows_pad == 0 || cols == 0) return HK_OK;
  HK_REQUIRE(cols % 8 == 0 && rows_pad % 8 == 0 && ld_in % 8 == 0 && ld_out % 8 == 0 && aligned_to(in, 16) &&
                 aligned_to(out, 16),
             "transpose: 16-byte rows and chunks expected");
  if constexpr (sizeof(T) == 4) {
    const dim3 grid((unsigned)cdiv(cols, 64), (unsigned)cdiv(rows_pad, 64));
    hipLaunchKernelGGL(transpose32_kernel, grid, dim3(256), 0, st, out, in, rows, rows_pad, cols, ld_in, ld_out, lim,
                       lim_off);
    return check_launch("transpose32_kernel");
  } else {
    const dim3 grid((unsigned)cdiv(cols, 128), (unsigned)cdiv(rows_pad, 128));
    hipLaunchKernelGGL((transpose_kernel<T>), grid, dim3(512), 0, st, out, in, rows, rows_pad, cols, ld_in, ld_out,
                       lim, lim_off);
    return check_launch("transpose_kernel");
  }
}

int64_t pad8(int64_t x) { return (x + 7) & ~(int64_t)7; }

// Input dtypes of the fused-linear ops: bf16 and fp16 (16-bit MFMA) and fp32 (fp32 MFMA).
bool fl_dtype_ok(int dt) { return dt == HK_BF16 || dt == HK_F16 || dt == HK_F32; }
int fl_esize(int dt) { return dt == HK_F32 ? 4 : 2; }

// f(Tag<T>) for the dtype (checked by fl_dtype_ok)
template <typename T> struct Tag { using type = T; };
template <typename F>
int fl_dispatch(int dt, F&& f) {
  if (dt == HK_BF16) return f(Tag<__bf16>{});
  if (dt == HK_F16) return f(Tag<_Float16>{});
  return f(Tag<float>{});
}

// Leading dimension of the transposed GEMM operands (X^T, D^T): 128 bytes past
// the K extent, so the rows of a tile's panel do not all start at the same
// large power-of-two offset.
int64_t ld_t(int64_t k) { return pad8(k) + 64; }

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct FlceLayout {
  size_t wt, xt, lg, dt, dwacc, nvalid, extra, total;
  int ksplit;   // most K splits of the dX GEMM (dx_max_splits), their fp32 partial sums at `part`
  size_t part;
  bool defer;  // the whole D^T [V, BTp] is kept and dW is one GEMM after the chunk loop
  // the compaction of the live rows: row map, inverse map, live count, compacted hidden rows;
  // for CrossEntropy also the compacted targets, row scales and losses
  size_t rowmap, inv, nlive, xc, tc, sc, lc;
};

// extra: bytes for the row step's own scratch (16-byte aligned); ce: room for the
// compacted CrossEntropy row inputs and outputs
FlceLayout flce_layout(int64_t BT, int64_t H, int64_t V, int64_t chunk, int es, bool grad, size_t extra = 0,
                       bool ce = false) {
  FlceLayout L{};
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += align256(bytes);
    return o;
  };
  L.nvalid = take(256);
  const size_t bt = (size_t)std::max<int64_t>(BT, 1);
  L.nlive = take(256);
  L.rowmap = take(bt * 4);
  L.inv = take(bt * 4);
  L.xc = take((size_t)pad8(BT) * H * es);
  if (ce) {
    L.tc = take(bt * 8);
    L.sc = take(bt * 4);
    L.lc = take(bt * 4);
  }
  L.lg = take((size_t)chunk * V * es);
  if (grad) {
    L.wt = take((size_t)H * V * es);
    L.xt = take((size_t)H * ld_t(BT) * es);
    // Several chunks: keep every chunk's D^T and run dW as one GEMM over K = BT
    // (no fp32 accumulator round trips) when that takes no more memory than
    // one chunk's D^T plus the fp32 accumulator; otherwise accumulate per chunk.
    L.defer = BT > chunk && pad8(BT) <= pad8(chunk) + 2 * H;
    if (L.defer) {
      L.dt = take((size_t)V * ld_t(BT) * es);
    } else {
      L.dt = take((size_t)V * ld_t(chunk) * es);
      L.dwacc = BT > chunk ? take((size_t)V * H * 4) : 0;
    }
    const int bk = es == 4 ? gemm::F32Cfg::BK : gemm::DefaultCfg::BK;
    const size_t pb = dx_part_bytes(chunk, H, V, bk);
    L.ksplit = pb ? dx_max_splits(H, V, bk) : 1;
    L.part = pb ? take(pb) : 0;
  }
  L.extra = extra ? take(extra) : 0;
  L.total = off;
  return L;
}

// FusedLinearJSD: the shared chunk engine's workspace, then the JSD pieces:
// per-row losses (compacted order with labels), the teacher logits chunk, and
// with labels the compacted teacher rows and labels.
struct FljsdLayout {
  FlceLayout base;
  size_t lc, lt, xtc, labc, total;
};

FljsdLayout fljsd_layout(int64_t BT, int64_t H, int64_t Ht, int64_t V, int64_t chunk, int es, bool grad) {
  FljsdLayout L{};
  L.base = flce_layout(BT, H, V, chunk, es, grad);
  size_t off = L.base.total;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += align256(bytes);
    return o;
  };
  const size_t bt = (size_t)std::max<int64_t>(BT, 1);
  L.lc = take(bt * 4);
  L.lt = take((size_t)chunk * V * es);
  L.xtc = take((size_t)pad8(BT) * Ht * es);
  L.labc = take(bt * 8);
  L.total = off;
  return L;
}

// The compacted hidden rows (live rows in order, zero rows after them).
template <typename T>
int gather_rows(T* Xc, const T* X, const int* rowmap, const int* n_live, int64_t BT, int64_t H, hipStream_t st) {
  if (BT == 0) return HK_OK;
  hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)std::min<int64_t>(BT, 4096)), dim3(256), 0, st, (u32x4*)Xc,
                     (const u32x4*)X, rowmap, n_live, BT, H * (int64_t)sizeof(T) / 16);
  return check_launch("gather_rows_kernel");
}

// Zero dX rows of the dead rows and, with loss_rows, the losses back in the original order.
template <typename T>
int finish_rows(T* dX, float* loss_rows, const float* loss_c, const int* inv, int64_t BT, int64_t H,
                hipStream_t st) {
  if (BT == 0 || (!dX && !loss_rows)) return HK_OK;
  hipLaunchKernelGGL(finish_rows_kernel, dim3((unsigned)std::min<int64_t>(BT, 4096)), dim3(256), 0, st, (u32x4*)dX,
                     H * (int64_t)sizeof(T) / 16, loss_rows, loss_c, inv, BT);
  return check_launch("finish_rows_kernel");
}

// Rows per chunk: a multiple of 8 (chunk starts stay 16-byte aligned in X^T), at most BT.
int64_t flce_chunk(int64_t BT, int64_t chunk) {
  if (chunk <= 0) chunk = 8192;
  chunk = std::max<int64_t>(8, chunk & ~(int64_t)7);
  return std::min<int64_t>(chunk, BT > 0 ? BT : 1);
}

// The chunked lm_head shared by the fused-linear losses. Per chunk of C rows:
// logits_c = X_c W^T into the chunk buffer; row_step(Lg, r0, cs) produces the
// row losses and, with gradients, the dlogits D_c written over the logits;
// then dX_c = D_c W, and dW = sum_c D_c^T X_c either as one GEMM over all rows
// after the loop (the chunks' D_c^T side by side, lay.defer) or per chunk into
// an fp32 accumulator, the result rounded once into dWo. X [BT, H] and W [V, H]
// are K-contiguous.
//
// With rowmap, the rows are compacted first: X holds the live rows of the
// caller's hidden states in order (rowmap[i] is row i's original row), zero
// rows after them, and *n_live (device memory) is their count. Every GEMM is
// cut to the live rows on the device (tiles past them exit, the dW GEMM's K
// stops at them), and dX_c is stored straight into the original rows; the
// caller zeroes the dead rows of dX. Without rowmap (n_live null too) every
// row of X is processed in place.
template <typename T, class RowStep>
int chunked_lm_head(const T* X, const T* W, int64_t BT, int64_t H, int64_t V, int64_t C, char* ws,
                    const FlceLayout& lay, bool grad, T* dX, T* dWo, const int* n_live, const int* rowmap,
                    RowStep&& row_step, hipStream_t st) {
  const int64_t BTp = pad8(BT), ldx = ld_t(BT);
  T* Lg = (T*)(ws + lay.lg);
  T* Wt = grad ? (T*)(ws + lay.wt) : nullptr;
  T* Xt = grad ? (T*)(ws + lay.xt) : nullptr;
  T* Dt = grad ? (T*)(ws + lay.dt) : nullptr;
  float* dwacc = (grad && lay.dwacc) ? (float*)(ws + lay.dwacc) : nullptr;
  int rc = HK_OK;
  if (grad) {
    rc = launch_transpose<T>(Wt, W, V, V, H, H, V, st);  // W^T [H, V]
    if (rc) return rc;
    rc = launch_transpose<T>(Xt, X, BT, BTp, H, H, ldx, st);  // X^T [H, BTp] (row stride ldx), zero padded
    if (rc) return rc;
  }
  const int64_t nchunks = BT > 0 ? cdiv(BT, C) : 0;
  for (int64_t ci = 0; ci < nchunks; ++ci) {
    const int64_t r0 = ci * C;
    const int64_t cs = std::min<int64_t>(C, BT - r0);
    // logits_c = X_c W^T (live rows only)
    rc = launch_gemm<T>(X + r0 * H, W, (int)cs, (int)V, (int)H, H, H, EpiStore<T>{Lg, V}, st, n_live, (int)r0);
    if (rc) return rc;
    rc = row_step(Lg, r0, cs);
    if (rc) return rc;
    if (!grad) continue;
    // dX_c = D_c W, stored into the live rows' original places; a short chunk
    // splits K (= V) and sums the splits' fp32 partials in a second pass
    if (lay.ksplit > 1) {
      float* part = (float*)(ws + lay.part);
      T* dst = rowmap ? dX : dX + r0 * H;
      const int* map = rowmap ? rowmap + r0 : nullptr;
      rc = launch_gemm<T>(Lg, Wt, (int)cs, (int)H, (int)V, V, V, EpiDx<T>{dst, H, map, part, H}, st, n_live,
                          (int)r0, false, lay.ksplit);
      if (rc) return rc;
      const int64_t work = cs * (H / 8);
      hipLaunchKernelGGL((splitk_sum_kernel<T>), dim3((unsigned)std::min<int64_t>(cdiv(work, 256), 8192)), dim3(256),
                         0, st, dst, H, map, part, (int)cs, (int)H, (int)(V / gemm::CfgFor<T>::BK), lay.ksplit,
                         n_live, (int)r0);
      rc = check_launch("splitk_sum_kernel");
    } else if (rowmap) {
      rc = launch_gemm<T>(Lg, Wt, (int)cs, (int)H, (int)V, V, V, EpiScatter<T>{dX, H, rowmap + r0}, st, n_live,
                          (int)r0);
    } else {
      rc = launch_gemm<T>(Lg, Wt, (int)cs, (int)H, (int)V, V, V, EpiStore<T>{dX + r0 * H, H}, st);
    }
    if (rc) return rc;
    if (lay.defer) {
      // D_c^T into columns [r0, r0 + cs) of D^T [V, BTp]; zeros past the live rows
      rc = launch_transpose<T>(Dt + r0, Lg, cs, ci + 1 < nchunks ? cs : BTp - r0, V, V, ldx, st, n_live, r0);
      if (rc) return rc;
      continue;
    }
    // dW += D_c^T X_c; K = cs is padded to a multiple of 8 with zeros on both operands, and cut
    // on the device to the live rows
    const int64_t csp = pad8(cs), ldd = ld_t(cs);
    rc = launch_transpose<T>(Dt, Lg, cs, csp, V, V, ldd, st, n_live, r0);
    if (rc) return rc;
    auto dw_gemm = [&](auto epi) {
      return launch_gemm<T>(Dt, Xt + r0, (int)V, (int)H, (int)csp, ldd, ldx, epi, st, n_live, (int)r0, true);
    };
    if (nchunks == 1) rc = dw_gemm(EpiStore<T>{dWo, H});
    else if (ci == 0) rc = dw_gemm(EpiAccum<T, 0>{dwacc, dWo, H});
    else if (ci + 1 < nchunks) rc = dw_gemm(EpiAccum<T, 1>{dwacc, dWo, H});
    else rc = dw_gemm(EpiAccum<T, 2>{dwacc, dWo, H});
    if (rc) return rc;
  }
  if (grad && lay.defer && nchunks > 0) {
    rc = launch_gemm<T>(Dt, Xt, (int)V, (int)H, (int)BTp, ldx, ldx, EpiStore<T>{dWo, H}, st, n_live, 0, true);
    if (rc) return rc;
  }
  if (grad && nchunks == 0) {
    // no rows: the weight gradient is zero (dX is empty)
    const int64_t n16 = V * H * (int64_t)sizeof(T) / 16;
    hipLaunchKernelGGL(zero16_kernel, dim3((unsigned)std::min<int64_t>(cdiv(n16, 256), 4096)), dim3(256), 0, st,
                       (u32x4*)dWo, n16);
    rc = check_launch("zero16_kernel");
  }
  return rc;
}

}  // namespace
}  // namespace hk

using namespace hk;

extern "C" {

size_t hk_fused_linear_cross_entropy_workspace_size(int64_t BT, int64_t H, int64_t V, int64_t chunk, int dtype,
                                                    int with_grad) {
  if (BT < 0 || H <= 0 || V <= 0 || !fl_dtype_ok(dtype)) return 0;
  return flce_layout(BT, H, V, flce_chunk(BT, chunk), fl_esize(dtype), with_grad != 0, 0, true).total;
}

int hk_fused_linear_cross_entropy(float* loss_out, float* loss_rows, void* dhidden, void* dweight, const void* hidden,
                                  const void* weight, const int64_t* targets, const float* row_scale, int64_t BT,
                                  int64_t H, int64_t V, int64_t ignore_index, int reduction, int dtype, int64_t chunk,
                                  void* workspace, size_t workspace_bytes, hk_stream_t stream) {
  HK_REQUIRE(fl_dtype_ok(dtype), "fused linear cross entropy supports fp32, bf16 and fp16 (got %d)", dtype);
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
  const FlceLayout lay = flce_layout(BT, H, V, C, fl_esize(dtype), grad, 0, true);
  HK_REQUIRE(workspace && workspace_bytes >= lay.total, "workspace too small: need %zu bytes, got %zu", lay.total,
             workspace_bytes);
  HK_REQUIRE(aligned_to(workspace, 256), "workspace must be 256-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  int* n_valid = (int*)(ws + lay.nvalid);
  int* n_live = (int*)(ws + lay.nlive);
  int* rowmap = (int*)(ws + lay.rowmap);
  int* inv = (int*)(ws + lay.inv);
  int64_t* tc = (int64_t*)(ws + lay.tc);
  float* sc = (float*)(ws + lay.sc);
  float* lc = (float*)(ws + lay.lc);
  // every target equal to ignore_index is ignored (fused_linear_cross_entropy.py:121,62-65);
  // unlike the CrossEntropy op, -1 is not a "no ignore" sentinel here
  const int has_ignore = 1;

  auto run = [&](auto tag) -> int {
    using T = typename decltype(tag)::type;
    T* Xc = (T*)(ws + lay.xc);
    int rc = HK_OK;
    if (BT > 0) {
      rc = count_valid_launch(n_valid, targets, BT, ignore_index, has_ignore, st);
      if (rc) return rc;
      // the non-ignored rows, compacted: their hidden rows, targets and row scales
      rc = ce_compact_launch(rowmap, inv, n_live, targets, BT, ignore_index, st);
      if (rc) return rc;
      rc = gather_rows<T>(Xc, (const T*)hidden, rowmap, n_live, BT, H, st);
      if (rc) return rc;
      hipLaunchKernelGGL(gather_ce_kernel, dim3((unsigned)std::min<int64_t>(cdiv(BT, 256), 1024)), dim3(256), 0, st,
                         tc, sc, targets, row_scale, rowmap, n_live);
      rc = check_launch("gather_ce_kernel");
      if (rc) return rc;
    }
    // per-row loss of the compacted rows; with gradients, D_c = (softmax - onehot) * s * row_scale
    // written over the logits
    auto ce_step = [&](T* Lg, int64_t r0, int64_t cs) {
      return ce_rows_launch(grad ? (void*)Lg : nullptr, lc + r0, Lg, tc + r0, cs, V, V, V, ignore_index, has_ignore,
                            n_valid, grad && reduction == HK_REDUCTION_MEAN, row_scale ? sc + r0 : nullptr, dtype, st,
                            n_live, r0);
    };
    rc = chunked_lm_head<T>(Xc, (const T*)weight, BT, H, V, C, ws, lay, grad, (T*)dhidden, (T*)dweight, n_live,
                            rowmap, ce_step, st);
    if (rc) return rc;
    // losses back in row order (ignored rows 0); ignored rows of dhidden are zero
    rc = finish_rows<T>(grad ? (T*)dhidden : nullptr, loss_rows, lc, inv, BT, H, st);
    if (rc) return rc;
    if (loss_out) {
      // with gradients the rows already carry 1/max(n_valid,1) for 'mean'; without, divide here
      const bool divide = !grad && reduction == HK_REDUCTION_MEAN && BT > 0;
      return sum_rows_launch(loss_out, loss_rows, BT, divide ? n_valid : nullptr, divide, st);
    }
    return HK_OK;
  };
  return fl_dispatch(dtype, run);
}


size_t hk_fused_linear_jsd_workspace_size(int64_t BT, int64_t H, int64_t Ht, int64_t V, int64_t chunk, int dtype,
                                          int with_grad) {
  if (BT < 0 || H <= 0 || Ht <= 0 || V <= 0 || !fl_dtype_ok(dtype)) return 0;
  return fljsd_layout(BT, H, Ht, V, flce_chunk(BT, chunk), fl_esize(dtype), with_grad != 0).total;
}

int hk_fused_linear_jsd(float* loss_out, void* dinput, void* dweight, const void* s_input, const void* s_weight,
                        const void* t_input, const void* t_weight, const int64_t* labels, int64_t BT, int64_t H,
                        int64_t Ht, int64_t V, int64_t ignore_index, float beta, float temperature, int dtype,
                        int64_t chunk, void* workspace, size_t workspace_bytes, hk_stream_t stream) {
  HK_REQUIRE(fl_dtype_ok(dtype), "fused linear JSD supports fp32, bf16 and fp16 (got %d)", dtype);
  HK_REQUIRE(BT >= 0 && H > 0 && Ht > 0 && V > 0, "invalid shape BT=%lld H=%lld Ht=%lld V=%lld", (long long)BT,
             (long long)H, (long long)Ht, (long long)V);
  HK_REQUIRE(H % 8 == 0 && Ht % 8 == 0 && V % 8 == 0, "H, Ht and V must be multiples of 8 (16-byte rows)");
  HK_REQUIRE(BT < (1LL << 31) && H < (1LL << 31) && Ht < (1LL << 31) && V < (1LL << 31) - 4096,
             "dimension too large");
  HK_REQUIRE(beta >= 0.f && beta <= 1.f, "beta must lie in [0, 1] (got %g)", (double)beta);
  HK_REQUIRE(temperature > 0.f, "temperature must be positive (got %g)", (double)temperature);
  const bool grad = dinput != nullptr || dweight != nullptr;
  HK_REQUIRE(!grad || (dinput && dweight), "dinput and dweight are computed together");
  HK_REQUIRE(loss_out && s_input && s_weight && t_input && t_weight, "null pointer argument");
  HK_REQUIRE(aligned_to(s_input, 16) && aligned_to(s_weight, 16) && aligned_to(t_input, 16) &&
                 aligned_to(t_weight, 16) && (!grad || (aligned_to(dinput, 16) && aligned_to(dweight, 16))),
             "inputs, weights and gradients must be 16-byte aligned");
  const int64_t C = flce_chunk(BT, chunk);
  const FljsdLayout lay = fljsd_layout(BT, H, Ht, V, C, fl_esize(dtype), grad);
  HK_REQUIRE(workspace && workspace_bytes >= lay.total, "workspace too small: need %zu bytes, got %zu", lay.total,
             workspace_bytes);
  HK_REQUIRE(aligned_to(workspace, 256), "workspace must be 256-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  const FlceLayout& lb = lay.base;
  int* n_valid = (int*)(ws + lb.nvalid);
  // with labels the ignored rows are compacted away (the engine's row map and live count)
  int* n_live = labels ? (int*)(ws + lb.nlive) : nullptr;
  int* rowmap = labels ? (int*)(ws + lb.rowmap) : nullptr;
  int* inv = (int*)(ws + lb.inv);
  float* lc = (float*)(ws + lay.lc);
  int64_t* labc = (int64_t*)(ws + lay.labc);

  auto run = [&](auto tag) -> int {
    using T = typename decltype(tag)::type;
    const T* Xs = (const T*)s_input;
    const T* Xt_in = (const T*)t_input;
    const T* Wt_in = (const T*)t_weight;
    T* Lt = (T*)(ws + lay.lt);
    T* Xtc = (T*)(ws + lay.xtc);
    T* Xsc = (T*)(ws + lb.xc);
    int rc = HK_OK;
    if (labels && BT > 0) {
      // n counts the labels that are not ignore_index over all BT rows (fused_linear_jsd.py:137-141)
      rc = count_valid_launch(n_valid, labels, BT, ignore_index, 1, st);
      if (rc) return rc;
      rc = ce_compact_launch(rowmap, inv, n_live, labels, BT, ignore_index, st);
      if (rc) return rc;
      rc = gather_rows<T>(Xsc, Xs, rowmap, n_live, BT, H, st);
      if (rc) return rc;
      rc = gather_rows<T>(Xtc, Xt_in, rowmap, n_live, BT, Ht, st);
      if (rc) return rc;
      hipLaunchKernelGGL(gather_ce_kernel, dim3((unsigned)std::min<int64_t>(cdiv(BT, 256), 1024)), dim3(256), 0, st,
                         labc, nullptr, labels, nullptr, rowmap, n_live);
      rc = check_launch("gather_ce_kernel");
      if (rc) return rc;
    }
    float* lrows = labels ? lc : (float*)(ws + lay.lc);
    // row step: the teacher logits of the chunk's rows (fused_linear_jsd.py:159-160), then the log-softmaxes,
    // JSD and, with gradients, the student dlogits over the student logits (:163-199)
    auto jsd_step = [&](T* Ls, int64_t r0, int64_t cs) {
      const T* xt = (labels ? Xtc : Xt_in) + r0 * Ht;
      int r = launch_gemm<T>(xt, Wt_in, (int)cs, (int)V, (int)Ht, Ht, Ht, EpiStore<T>{Lt, V}, st, n_live, (int)r0);
      if (r) return r;
      return jsd_logits_launch(lrows + r0, Ls, Lt, labels ? labc + r0 : nullptr, ignore_index, n_valid, BT, beta,
                               temperature, cs, V, V, grad ? 1 : 0, dtype, st, n_live, r0);
    };
    rc = chunked_lm_head<T>(labels ? Xsc : Xs, (const T*)s_weight, BT, H, V, C, ws, lb, grad, (T*)dinput,
                            (T*)dweight, n_live, rowmap, jsd_step, st);
    if (rc) return rc;
    if (labels) {
      // losses back in row order (ignored rows 0); ignored rows of dinput are zero
      float* rows_out = (float*)(ws + lay.labc);  // the compacted labels are no longer needed
      rc = finish_rows<T>(grad ? (T*)dinput : nullptr, rows_out, lc, inv, BT, H, st);
      if (rc) return rc;
      lrows = rows_out;
    }
    // the rows already carry 1/n (:190)
    return scaled_sum_rows_launch(loss_out, lrows, BT, 1.0f, st);
  };
  return fl_dispatch(dtype, run);
}

size_t hk_fused_linear_grpo_workspace_size(int64_t B, int64_t L, int64_t H, int64_t V, int64_t chunk, int dtype,
                                           int with_grad) {
  if (B <= 0 || L < 0 || H <= 0 || V <= 0 || !fl_dtype_ok(dtype)) return 0;
  const int64_t BT = B * (L + 1);
  return flce_layout(BT, H, V, flce_chunk(BT, chunk), fl_esize(dtype), with_grad != 0, grpo_scratch_bytes(B, L))
      .total;
}

int hk_fused_linear_grpo(float* loss_out, float* kl_out, float* clip_out, float* lse_rows, float* loss_rows,
                         float* kl_rows, float* clip_rows, void* dhidden, void* dweight, const void* hidden,
                         const void* weight, const int64_t* ids, int64_t ids_sB, int64_t ids_sL,
                         const float* advantages, const float* old_logp, int64_t old_sB, int64_t old_sL,
                         const float* ref_logp, int64_t ref_sB, int64_t ref_sL, const void* mask, int mask_dtype,
                         int64_t mask_sB, int64_t mask_sL, int64_t B, int64_t L, int64_t H, int64_t V,
                         float temperature, float beta, float eps_low, float eps_high, int dtype, int64_t chunk,
                         void* workspace, size_t workspace_bytes, hk_stream_t stream) {
  HK_REQUIRE(fl_dtype_ok(dtype), "fused linear GRPO supports fp32, bf16 and fp16 (got %d)", dtype);
  const GrpoInputs in{ids,    ids_sB, ids_sL, advantages, old_logp, old_sB,      old_sL, ref_logp,
                      ref_sB, ref_sL, mask,   mask_dtype, mask_sB,  mask_sL,     B,      L,
                      V,      temperature,    beta,       eps_low,  eps_high};
  if (const int rc = grpo_check(in)) return rc;
  HK_REQUIRE(H > 0 && H % 8 == 0 && V % 8 == 0, "H and V must be positive multiples of 8 (16-byte rows)");
  HK_REQUIRE(B * (L + 1) < (1LL << 31) && H < (1LL << 31), "dimension too large");
  const bool grad = dhidden != nullptr || dweight != nullptr;
  HK_REQUIRE(!grad || (dhidden && dweight), "dhidden and dweight are computed together");
  HK_REQUIRE(loss_out && clip_out && hidden && weight && (L == 0 || (lse_rows && loss_rows && kl_rows && clip_rows)),
             "null pointer argument");
  HK_REQUIRE(aligned_to(hidden, 16) && aligned_to(weight, 16) && (!grad || (aligned_to(dhidden, 16) &&
                                                                             aligned_to(dweight, 16))),
             "hidden, weight and gradients must be 16-byte aligned");
  const int64_t BT = B * (L + 1);
  const int64_t C = flce_chunk(BT, chunk);
  const FlceLayout lay = flce_layout(BT, H, V, C, fl_esize(dtype), grad, grpo_scratch_bytes(B, L));
  HK_REQUIRE(workspace && workspace_bytes >= lay.total, "workspace too small: need %zu bytes, got %zu", lay.total,
             workspace_bytes);
  HK_REQUIRE(aligned_to(workspace, 256), "workspace must be 256-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  void* scratch = ws + lay.extra;
  int* n_live = (int*)(ws + lay.nlive);
  int* rowmap = (int*)(ws + lay.rowmap);
  int* inv = (int*)(ws + lay.inv);
  auto run = [&](auto tag) -> int {
    using T = typename decltype(tag)::type;
    T* Xc = (T*)(ws + lay.xc);
    int rc = grpo_prep_launch(in, scratch, st);
    if (rc) return rc;
    // the live positions (l < L, mask != 0), compacted: only their logits are computed
    rc = grpo_compact_launch(rowmap, inv, n_live, in, st);
    if (rc) return rc;
    rc = gather_rows<T>(Xc, (const T*)hidden, rowmap, n_live, BT, H, st);
    if (rc) return rc;
    // compacted row q of a chunk is position rowmap[r0 + q]: the GRPO row kernel
    // writes that token's results and, with gradients, its dlogits over the logits
    auto grpo_step = [&](T* Lg, int64_t r0, int64_t cs) {
      return grpo_rows_launch(grad ? (void*)Lg : nullptr, Lg, r0, cs, in, scratch, dtype, st, rowmap, n_live);
    };
    rc = chunked_lm_head<T>(Xc, (const T*)weight, BT, H, V, C, ws, lay, grad, (T*)dhidden, (T*)dweight, n_live,
                            rowmap, grpo_step, st);
    if (rc) return rc;
    // masked tokens and position L: zero rows of dhidden
    rc = finish_rows<T>(grad ? (T*)dhidden : nullptr, nullptr, nullptr, inv, BT, H, st);
    if (rc) return rc;
    return grpo_finalize_launch(in, scratch, loss_out, kl_out, clip_out, lse_rows, loss_rows, kl_rows, clip_rows,
                                st);
  };
  return fl_dispatch(dtype, run);
}

}  // extern "C"
