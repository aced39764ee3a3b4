// Log-sum-exp loss family for gfx950: CrossEntropy (fused loss + gradient,
// inference forward), selective log-softmax and the GRPO loss with its
// gradient fused into the forward pass.
//
// Row engine. One workgroup owns one vocabulary row at a time (persistent
// grid of the blocks the CUs hold, rows strided by gridDim.x). When
// the row fits, it is held in VGPRs: NCH packed 16-byte vectors per lane over
// a 256-, 512- or 1024-lane workgroup, the smallest form that holds the row
// (a 32000-entry bf16 row is 16 vectors per lane of 256 lanes, four blocks a
// CU; a 128256-entry row 16 vectors per lane of 1024 lanes, 64 VGPRs),
// so the row crosses HBM once: read, max, sum of 2^(x*c - m), then the
// gradient p * g is written straight from the registers, p recomputed in fp32
// and rounded once as the reference does. The target column is left out of
// the reduction and its term added from the target logit afterwards, so its
// gradient -(1 - p_t) * g is formed from the other columns' mass instead of
// p_t - 1 (which cancels in fp32 when p_t is near 1). Rows that do not fit use
// a streaming variant that keeps a per-lane online (max, sum) and reads the
// row a second time for the gradient.
//
// All exponentials run on v_exp_f32 (2^x) with log2(e)/T folded into one
// multiply-add per element; log-sum-exp is kept in the log2 domain and
// converted once per row.
#include "hk_common.h"
#include "hk_internal.h"
#include "../../include/hilda_kernel_amd.h"

#include <algorithm>
#include <math.h>
#include <type_traits>

namespace hk {
namespace {

// ---------------------------------------------------------------------------
// register-resident row helpers
// ---------------------------------------------------------------------------
// max(a, b, c) in one instruction (fmaxf would add a canonicalising max per operand)
__device__ __forceinline__ float max3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

template <typename T, int VEC, int NCH, int BLOCK, int NFULL = 0>
struct RowRegs {
  static_assert(NFULL <= NCH, "full vectors");
  Pack<T, VEC> v[NCH];

  // Addressing: vector j of lane t covers columns [j*BLOCK*VEC + t*VEC, +VEC).
  // The j-dependent part is uniform (row pointer + constant) and the lane part
  // is one 32-bit VGPR. Whether vector j is full, partial or absent depends
  // only on the uniform remainder n - j*BLOCK*VEC, so those cases are scalar
  // branches; only a partial vector needs a per-lane test. Column indices are
  // 32-bit: the host rejects rows of 2^31 or more elements.
  // Vectors j < NFULL are full in every row that the caller hands over (it
  // guarantees n >= NFULL * kSpan): their loads and stores need no test, so
  // the compiler can count the loads in flight and wait for each vector's
  // load in turn rather than for all of them at the first vector. The
  // reduction's tests stay scalar branches even where they always pass: each
  // vector's work then stays a block of its own, which keeps the compiler
  // from overlapping the vectors' temporaries (and spilling).
  static constexpr int kSpan = BLOCK * VEC;
  __device__ __forceinline__ static int lane_col() { return (int)threadIdx.x * VEC; }
  // element offset of vector j for a lane at column tc, as an unsigned 32-bit
  // value: the address is then one 64-bit base plus a zero-extended VGPR offset
  // (the global_load saddr form) rather than one 64-bit base per vector.
  __device__ __forceinline__ static uint32_t off(int j, int tc) { return (uint32_t)(j * kSpan) + (uint32_t)tc; }

  // The lanes of a partial vector past the row end load the row's first
  // elements (an in-bounds address) and keep them: the reduction reads them as
  // -inf (mask_tail) and the stores skip them. Masking at load time instead
  // would make the wave wait for that load, and so for every store and load
  // issued before it, at the end of each refill.
  __device__ __forceinline__ void load(const T* __restrict__ row, int n) {
    const int tc = lane_col();
    const Pack<T, VEC> ninf = splat_pack<T, VEC>(-INFINITY);
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int lim = n - j * kSpan;  // uniform
      if (j < NFULL || lim >= kSpan) {
        v[j] = load_pack<T, VEC>(row + off(j, tc));
      } else if (lim > 0) {
        v[j] = load_pack<T, VEC>(row + off(j, tc < lim ? tc : 0));  // in-bounds address
      } else {
        v[j] = ninf;  // defined on every path, so no value flows in from the previous row
      }
    }
  }

  // The unpacked floats of vector j with the lanes past the row end at -inf.
  __device__ __forceinline__ static void mask_tail(int j, int n, float (&x)[VEC]) {
    const int lim = n - j * kSpan;  // uniform
    if (lim < kSpan) {
      const bool in_row = lane_col() < lim;
#pragma unroll
      for (int e = 0; e < VEC; ++e) x[e] = in_row ? x[e] : -INFINITY;
    }
  }

  __device__ __forceinline__ void opaque() {
#pragma unroll
    for (int j = 0; j < NCH; ++j) make_opaque(v[j]);
  }

  // The reduction of this lane, leaving out the element at column `target`
  // (< 0: none): m = max of x*c (log2 domain) and s = sum 2^(x*c - m) over the
  // lane's other elements; the registers keep x. The caller adds the target's
  // own term from its logit after the block reduction (target_merge), which
  // gives 1 - p_t without the cancellation of computing it from p_t in fp32
  // when p_t is close to 1. The target's vector is a uniform test, and only
  // that vector's unpacked floats are masked (rewriting the registers would
  // make the compiler carry every vector through phi copies).
  // *xt_out (when given) receives the target's own x in the lane that holds
  // it, the one lane of the block for which owns_target() is true.
  __device__ __forceinline__ void reduce_lane(int n, float c, int target, float* m_out, float* s_out,
                                              float* xt_out = nullptr) {
    const int jt = target >= 0 ? target / kSpan : -1;  // uniform
    const int rel = target - jt * kSpan - lane_col();  // in [0, VEC) in the owning lane only
    float m = -INFINITY, xt = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      if (j * kSpan < n) {
        float x[VEC];
        unpack(v[j], x);
        mask_tail(j, n, x);
        if (j == jt) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            xt = e == rel ? x[e] : xt;
            x[e] = e == rel ? -INFINITY : x[e];
          }
        }
#pragma unroll
        for (int e = 0; e + 1 < VEC; e += 2) m = max3(m, x[e], x[e + 1]);
        if constexpr (VEC & 1) m = fmaxf(m, x[VEC - 1]);
      }
      __builtin_amdgcn_sched_barrier(0);  // one vector's floats live at a time
    }
    m *= c;
    opaque();  // unpack again below rather than keep all the floats of the max pass live
    const float mo = m == -INFINITY ? 0.f : m;  // an all-padding lane: every e is 2^-inf = 0
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      if (j * kSpan < n) {
        float x[VEC];
        unpack(v[j], x);
        mask_tail(j, n, x);
        if (j == jt) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) x[e] = e == rel ? -INFINITY : x[e];
        }
#pragma unroll
        for (int e = 0; e < VEC; ++e) s += exp2_fast(fmaf(x[e], c, -mo));
      }
      __builtin_amdgcn_sched_barrier(0);  // one vector's floats live at a time
    }
    *m_out = m;
    *s_out = s;
    if (xt_out) *xt_out = xt;
  }

  // Whether this lane holds column `target` (of a row of n > target columns).
  __device__ __forceinline__ static bool owns_target(int target) {
    return target >= 0 && (target % kSpan) / VEC == (int)threadIdx.x;
  }

  // Gradient of the row, p_j * g = 2^(x_j*c - lse2) * g computed in fp32 and
  // rounded once to T (the arithmetic of kernels/cross_entropy.py:159-166),
  // without the one-hot term (the caller patches the target element); then the
  // row at `next` loaded into the same registers, so the row's stores and the
  // next row's loads are in flight together. Recomputing the exponential here
  // instead of keeping 2^(x*c - m) from the sum pass measured as fast. The
  // loads follow all of the row's stores: issuing each beside its vector's
  // store measured 3% slower on CrossEntropy [8192, 128256] and 2% on GRPO
  // (HBM serves a run of writes, then a run of reads, better than the two
  // interleaved). With this order, staging the next row's first half into LDS
  // by DMA during the reduction (a second row in flight) measured no faster.
  __device__ __forceinline__ void store_prob_grad_then_load(T* out, int n, float c, float lse2, float g,
                                                            const T* next) {
    const int tc = lane_col();
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int lim = n - j * kSpan;  // uniform
      if (j < NFULL || lim > 0) {
        float x[VEC];
        unpack(v[j], x);
#pragma unroll
        for (int e = 0; e < VEC; ++e) x[e] = exp2_fast(fmaf(x[e], c, -lse2)) * g;
        if (j < NFULL || lim >= kSpan || tc < lim) store_pack_nt<T, VEC>(out + off(j, tc), pack<T, VEC>(x));
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int lim = n - j * kSpan;  // uniform
      if (j < NFULL || lim > 0) v[j] = load_pack<T, VEC>(next + off(j, lim >= kSpan || tc < lim ? tc : 0));  // see load()
    }
  }
};

// The row length as a per-iteration scalar. Hiding it from loop-invariant
// code motion keeps the per-vector bounds tests inside the row loop (a few
// scalar ops per row) instead of hoisting 3*NCH 64-bit masks into SGPRs,
// which spills them.
__device__ __forceinline__ int row_len(int64_t v) {
  int n = (int)v;
  asm volatile("" : "+s"(n));
  return n;
}

template <typename T, int VEC, int BLOCK>
__device__ __forceinline__ void fill_row(T* __restrict__ out, int n, float value) {
  const Pack<T, VEC> z = splat_pack<T, VEC>(value);
  for (int col = (int)threadIdx.x * VEC; col < n; col += BLOCK * VEC)
    store_pack_nt<T, VEC>(out + col, z);
}

// (m, s) <- merge with (m2, s2), where s is a sum of 2^(v - m)
__device__ __forceinline__ void lse2_merge(float& m, float& s, float m2, float s2) {
  const float M = fmaxf(m, m2);
  const float a = m == -INFINITY ? 0.f : s * exp2_fast(m - M);
  const float b = m2 == -INFINITY ? 0.f : s2 * exp2_fast(m2 - M);
  m = M;
  s = a + b;
}

// Block-wide (max, sum) of per-lane (m, s) pairs, one LDS exchange: *M the
// block max, *S the sum scaled to it. `red` holds kRedStride floats per
// parity; alternating `parity` between consecutive calls lets the exchange go
// without a trailing barrier. With X, the same exchange also broadcasts one
// lane's value: the lane with `own` set (exactly one in the block) passes x
// and every lane receives it in *X, as a uniform (scalar) value.
template <int NW>
struct BlockRed {
  static constexpr int kStride = 2 * NW + 4;  // m[NW], s[NW], x, padding to 16 bytes
  static constexpr int kFloats = 2 * kStride;
};

template <int NW>
__device__ __forceinline__ void block_lse2_ms(float m, float s, float* red, int parity, float* M, float* S,
                                              float x = 0.f, bool own = false, float* X = nullptr) {
  static_assert(NW > 1, "the exchange goes through LDS");
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) lse2_merge(m, s, __shfl_xor(m, o, kWave), __shfl_xor(s, o, kWave));
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  float* r = red + parity * BlockRed<NW>::kStride;
  if (lane == 0) {
    r[wave] = m;
    r[NW + wave] = s;
  }
  if (X && own) r[2 * NW] = x;
  // A barrier for LDS traffic only: each wave's LDS writes have completed
  // before it arrives. __syncthreads() would also wait for every global load
  // the wave has in flight, such as the next row's refill in the forward-only
  // loop. (One asm statement, so the compiler moves no memory access across
  // the barrier.)
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  m = r[0];
  s = r[NW];
#pragma unroll
  for (int i = 1; i < NW; ++i) lse2_merge(m, s, r[i], r[NW + i]);
  *M = m;
  *S = s;
  if (X) *X = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, r[2 * NW])));
}

// The row's log2-sum-exp from the (max, sum) of every column but the target,
// (M, R), and the target's x*c, xtc: the target's term 2^(xtc) joins the sum,
// and *rest = R / S is 1 - p_t, the mass outside the target, exact where
// 1 - 2^(xtc - lse2) would cancel. has_target false: lse2 of (M, R), rest 1.
// Both results are uniform: they are returned through readfirstlane so they
// sit in scalar registers, off the row's VGPR budget.
__device__ __forceinline__ float target_merge(float M, float R, float xtc, bool has_target, float* rest) {
  float m = M, s = R;
  if (has_target) lse2_merge(m, s, xtc, 1.f);
  const float r = M == -INFINITY ? 0.f : R * exp2_fast(M - m);
  const float q = s > 0.f ? r * rcp_fast(s) : 0.f;  // (v_rcp_f32: 1 ulp)
  *rest = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, q)));
  const float lse2 = m + log2_fast(s);
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, lse2)));
}

// Streaming row log-sum-exp (any length): per-lane online (max, sum), then a
// block combine. With REST, *rest = 1 - p_target from a second sum that leaves
// the target column out (see reduce_lane).
constexpr int kStreamU = 4;  // packs of a lane in flight in the streaming row forms
template <typename T, int VEC, int BLOCK, bool REST = false>
__device__ __forceinline__ float row_lse2_stream(const T* __restrict__ row, int n, float c, float* red,
                                                 int target = -1, float* rest = nullptr) {
  float m = -INFINITY, s = 0.f, r = 0.f;
  // kStreamU packs of a lane loaded before any is used (one memory round trip
  // for up to kStreamU x BLOCK packs), then folded in the same order as one at a time
  constexpr int U = kStreamU;
  const int nv = n / VEC;
  for (int i0 = (int)threadIdx.x; i0 < nv; i0 += BLOCK * U) {
    Pack<T, VEC> pk[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i0 + u * BLOCK < nv) pk[u] = load_pack<T, VEC>(row + (i0 + u * BLOCK) * VEC);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int col = (i0 + u * BLOCK) * VEC;
      if (col >= n) break;
      float x[VEC];
      unpack(pk[u], x);
      float tm = x[0];
#pragma unroll
      for (int e = 1; e < VEC; ++e) tm = fmaxf(tm, x[e]);
      const float mn = fmaxf(m, tm * c);
      const float sc = m == -INFINITY ? 0.f : exp2_fast(m - mn);
      float add = 0.f, add_r = 0.f;
      const int rel = target - col;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float p = exp2_fast(fmaf(x[e], c, -mn));
        add += p;
        if constexpr (REST) add_r += e == rel ? 0.f : p;
      }
      s = s * sc + add;
      if constexpr (REST) r = r * sc + add_r;
      m = mn;
    }
  }
  const float M = block_max<BLOCK / kWave>(m, red);
  const float f = (m == -INFINITY) ? 0.f : exp2_fast(m - M);
  const float S = block_sum<BLOCK / kWave>(s * f, red);
  if constexpr (REST) {
    const float R = block_sum<BLOCK / kWave>(r * f, red);
    *rest = S > 0.f ? R / S : 0.f;
  }
  return M + log2_fast(S);
}

// out[j] = p_j * g with p_j = 2^(x_j*c - lse2), and at the target column
// -rest * g (= (p_t - 1) * g, rest from row_lse2_stream<REST>).
template <typename T, int VEC, int BLOCK>
__device__ __forceinline__ void store_grad_stream(T* __restrict__ out, const T* __restrict__ row, int n, float c,
                                                  float lse2, int target, float rest, float g) {
  for (int col = (int)threadIdx.x * VEC; col < n; col += BLOCK * VEC) {
    float x[VEC];
    unpack(load_pack<T, VEC>(row + col), x);
    const int rel = target - col;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float p = exp2_fast(fmaf(x[e], c, -lse2));
      x[e] = (e == rel ? -rest : p) * g;
    }
    store_pack_nt<T, VEC>(out + col, pack<T, VEC>(x));
  }
}

// The target column of a row (col < 0: none) and its logit times c.
struct RowTarget {
  int col;
  float xtc;
};
struct NoTarget {
  template <class Ctx>
  __device__ RowTarget operator()(const Ctx&) const { return RowTarget{-1, 0.f}; }
};

// Forward-only row loop, register-resident: the block's rows (row, row + G,
// ...) that next_live accepts, each held in VGPRs. A row's lanes reduce their
// (max, sum) from the registers, then refill them with the next row before the
// block-wide combine, so the next row's loads are in flight during the
// exchange and the caller's per-row epilogue. emit(row, lse2, ctx) runs on
// every lane with the row's log2-sum-exp of x * c; ctx = pre(row) runs before
// the row's reduction (for loads that should overlap it). target_of(ctx)
// names a column that the reduction leaves out and adds back afterwards
// (target_merge), exactly as the gradient kernels do: with the target column
// named, as the GRPO forward-only path does, a forward-only call returns
// bitwise the same results as the gradient form. The CrossEntropy inference
// and selective log-softmax forwards name none (NoTarget) and reduce over
// every column, so their results agree with the gradient forms' to rounding.
template <typename T, int VEC, int NCH, int BLOCK, class RowPtr, class NextLive, class Pre, class TargetOf,
          class Emit>
__device__ __forceinline__ void lse_rows_resident(int n, float c, int64_t rows, float* red, RowPtr row_ptr,
                                                  NextLive next_live, Pre pre, TargetOf target_of, Emit emit) {
  int64_t row = next_live((int64_t)blockIdx.x);
  if (row >= rows) return;
  RowRegs<T, VEC, NCH, BLOCK> r;
  r.load(row_ptr(row), n);
  int parity = 0;
  for (;;) {
    const int64_t next = next_live(row + (int64_t)gridDim.x);
    auto ctx = pre(row);
    const RowTarget tg = target_of(ctx);
    float m, s;
    r.reduce_lane(n, c, tg.col, &m, &s);
    r.opaque();
    __builtin_amdgcn_sched_barrier(0);  // the refill may not start before the row is reduced (register reuse)
    if (next < rows) r.load(row_ptr(next), n);
    float M, S, rest;
    block_lse2_ms<BLOCK / kWave>(m, s, red, parity, &M, &S);
    const float lse2 = target_merge(M, S, tg.xtc, tg.col >= 0, &rest);
    parity ^= 1;
    emit(row, lse2, ctx);
    if (next >= rows) break;
    row = next;
  }
}

// The register-resident forms (block, vectors per lane), smallest first; a row
// of nv vectors takes the first form with block * nch >= nv (choose_row_cfg).
struct RowForm {
  int block, nch;
};
constexpr RowForm kRowForms[] = {{256, 1},   {256, 2},   {256, 4},    {256, 8},    {256, 12},   {512, 8},
                                 {512, 12},  {512, 16},  {1024, 12},  {1024, 16},  {1024, 20},  {1024, 24}};

// Vectors per lane that are full in every row a form serves: such a row is
// longer than the previous form's capacity.
constexpr int full_vectors(int nch, int block) {
  int prev = 0;
  for (const RowForm& f : kRowForms) {
    if (f.block == block && f.nch == nch) return prev / block;
    prev = f.block * f.nch;
  }
  return 0;
}


// ---------------------------------------------------------------------------
// CrossEntropy
// ---------------------------------------------------------------------------
struct CeArgs {
  const int64_t* targets;
  float* loss_rows;
  float* lse_rows;  // inference path only
  const int* n_valid;
  const float* row_scale;  // optional per-row gradient factor
  int64_t rows, V, ld_in, ld_out, ignore_index;
  int has_ignore;
  int scale_by_n_valid;
  const int* rows_lim;  // optional device-side bound: rows cut to *rows_lim - rows_off
  int64_t rows_off;
  // optional plan (ce_plan_kernel): the rows that get a gradient are
  // rowmap[0 .. *n_live), dealt out to the blocks in turn
  const int* rowmap;
  const int* n_live;
};

// Applies CeArgs::rows_lim (a uniform scalar load) to the kernel's copy of the arguments.
__device__ __forceinline__ void ce_bound(CeArgs& a) {
  if (a.rows_lim) a.rows = min(a.rows, max((int64_t)0, (int64_t)*a.rows_lim - a.rows_off));
}

__device__ __forceinline__ float ce_scale(const CeArgs& a) {
  return a.scale_by_n_valid ? 1.f / fmaxf((float)*a.n_valid, 1.f) : 1.f;
}

// Training forward: loss_r = (lse - x_t) * s and dlogits = (softmax - onehot) * s
// (kernels/cross_entropy.py:114-166). Ignored rows: loss 0 and a zero row,
// never read.
template <typename T, int VEC, int NCH, int BLOCK, bool RESIDENT>
__global__ __launch_bounds__(BLOCK) void ce_fwd_grad_kernel(T* dlogits, const T* logits, CeArgs a) {
  // dlogits may alias logits (in-place use): every element is read before the
  // same thread overwrites it, and a row's stores are issued before the next
  // row's loads of the same vector, so the pointers are not declared __restrict__.
  __shared__ float red[BlockRed<BLOCK / kWave>::kFloats];
  ce_bound(a);
  const float scale = ce_scale(a);
  const int64_t G = gridDim.x;
  auto is_live = [&](int64_t t) { return !(a.has_ignore && t == a.ignore_index) && t >= 0 && t < a.V; };
  if constexpr (RESIDENT) {
    using Regs = RowRegs<T, VEC, NCH, BLOCK, full_vectors(NCH, BLOCK)>;
    const int n = row_len(a.V);
    // dead rows (ignored or out of range) first: a zero (NaN) row, never read
    for (int64_t row = blockIdx.x; row < a.rows; row += G) {
      const int64_t t = a.targets[row];
      if (!is_live(t)) {
        const bool ignored = a.has_ignore && t == a.ignore_index;
        fill_row<T, VEC, BLOCK>(dlogits + row * a.ld_out, n, ignored ? 0.f : NAN);
        if (threadIdx.x == 0) a.loss_rows[row] = ignored ? 0.f : NAN;
      }
    }
    // Then the live rows. Row r's gradient stores go out with the loads of the
    // next live row r' (register refill). The per-row scalars (targets, row
    // scale) are scalar loads, so waiting for them never waits for the vector
    // loads in flight; the search for the row after r' runs at the end of the
    // iteration, while r's stores and r''s loads are in flight. The target
    // logit comes out of the registers, broadcast by the block exchange.
    // The block's live rows: with a plan, rowmap[q] for q = blockIdx.x,
    // + G, ... (every such row is live, and the blocks' counts differ by one
    // at most); without one, rows q = blockIdx.x, + G, ... that are live.
    struct LiveRow {
      int64_t q, row, t;  // q >= nq: none
    };
    const int64_t nq = a.rowmap ? (int64_t)scalar_load(a.n_live) : a.rows;
    auto next_live = [&](int64_t from) {
      LiveRow x{from, 0, 0};
      for (; x.q < nq; x.q += G) {
        x.row = a.rowmap ? (int64_t)scalar_load(a.rowmap + x.q) : x.q;
        x.t = scalar_load(a.targets + x.row);
        if (is_live(x.t)) break;
      }
      return x;
    };
    LiveRow cur = next_live(blockIdx.x);
    if (cur.q >= nq) return;
    Regs r;
    r.load(logits + cur.row * a.ld_in, n);
    LiveRow next = next_live(cur.q + G);
    int parity = 0;
    for (;;) {
      const int n = row_len(a.V);  // per iteration (see row_len)
      const int64_t row = cur.row;
      const int t = (int)cur.t;
      const T* in = logits + row * a.ld_in;
      // The refill is unconditional (the last row re-reads itself, from L2,
      // and the data is not used), so the registers carry one definition
      // around the loop and every path has the same loads in flight.
      const T* src = next.q < nq ? logits + next.row * a.ld_in : in;
      const float gscale = a.row_scale ? scale * scalar_load(a.row_scale + row) : scale;
      float m, s, xt, M, R, X, rest;
      r.reduce_lane(n, kLog2e, t, &m, &s, &xt);
      block_lse2_ms<BLOCK / kWave>(m, s, red, parity, &M, &R, xt, Regs::owns_target(t), &X);
      const float lse2 = target_merge(M, R, X * kLog2e, true, &rest);
      parity ^= 1;
      r.opaque();
      T* out = dlogits + row * a.ld_out;
      r.store_prob_grad_then_load(out, n, kLog2e, lse2, gscale, src);
      // the target element: (p_t - 1) * g = -(1 - p_t) * g, stored after (and
      // over) the vector store of the same thread
      if (Regs::owns_target(t)) out[t] = from_f32<T>(-rest * gscale);
      if (threadIdx.x == 0) a.loss_rows[row] = (lse2 * kLn2 - X) * scale;
      if (next.q >= nq) break;
      cur = next;
      next = next_live(cur.q + G);
    }
  } else {
    __shared__ float red1[BLOCK / kWave];
    for (int64_t row = blockIdx.x; row < a.rows; row += G) {
      const int64_t t = a.targets[row];
      T* out = dlogits + row * a.ld_out;
      const T* in = logits + row * a.ld_in;
      if (!is_live(t)) {
        const bool ignored = a.has_ignore && t == a.ignore_index;
        fill_row<T, VEC, BLOCK>(out, (int)a.V, ignored ? 0.f : NAN);
        if (threadIdx.x == 0) a.loss_rows[row] = ignored ? 0.f : NAN;
        continue;
      }
      const float xt = to_f32<T>(in[t]);
      const float gscale = a.row_scale ? scale * a.row_scale[row] : scale;
      float rest;
      const float lse2 = row_lse2_stream<T, VEC, BLOCK, true>(in, (int)a.V, kLog2e, red1, (int)t, &rest);
      if (threadIdx.x == 0) a.loss_rows[row] = (lse2 * kLn2 - xt) * scale;
      store_grad_stream<T, VEC, BLOCK>(out, in, (int)a.V, kLog2e, lse2, (int)t, rest, gscale);
    }
  }
}

// Inference forward (kernels/cross_entropy.py:32-65): lse and lse - x_t (0 if
// ignored, NaN for a target out of range). Every row's lse is computed,
// ignored rows included.
struct TargetLogit {
  int64_t t;
  float xt;
};

template <typename T, int VEC, int NCH, int BLOCK, bool RESIDENT>
__global__ __launch_bounds__(BLOCK) void ce_fwd_kernel(const T* __restrict__ logits, CeArgs a) {
  __shared__ float red[BlockRed<BLOCK / kWave>::kFloats];
  ce_bound(a);
  auto target = [&](int64_t row) {
    const int64_t t = a.targets[row];
    const bool in_range = t >= 0 && t < a.V;
    return TargetLogit{t, in_range ? to_f32<T>(logits[row * a.ld_in + t]) : 0.f};
  };
  auto emit = [&](int64_t row, float lse2, TargetLogit tx) {
    if (threadIdx.x == 0) {
      const float lse = lse2 * kLn2;
      float loss;
      if (a.has_ignore && tx.t == a.ignore_index) loss = 0.f;
      else if (tx.t < 0 || tx.t >= a.V) loss = NAN;
      else loss = lse - tx.xt;
      if (a.lse_rows) a.lse_rows[row] = lse;
      a.loss_rows[row] = loss;
    }
  };
  if constexpr (RESIDENT) {
    lse_rows_resident<T, VEC, NCH, BLOCK>(
        row_len(a.V), kLog2e, a.rows, red, [&](int64_t row) { return logits + row * a.ld_in; },
        [](int64_t q) { return q; }, target, NoTarget{}, emit);
  } else {
    // the target logit is read after the row (its address waits on the target
    // load, which would hold back the row's loads behind it)
    for (int64_t row = blockIdx.x; row < a.rows; row += gridDim.x) {
      const float lse2 = row_lse2_stream<T, VEC, BLOCK>(logits + row * a.ld_in, (int)a.V, kLog2e, red);
      if (threadIdx.x == 0) emit(row, lse2, target(row));
    }
  }
}

// n_valid = #targets != ignore_index (all rows when there is no ignore index)
__global__ __launch_bounds__(1024) void count_valid_kernel(int* __restrict__ n_valid, const int64_t* __restrict__ t,
                                                           int64_t rows, int64_t ignore_index, int has_ignore) {
  __shared__ float red[16];
  float c = 0.f;
  for (int64_t i = threadIdx.x; i < rows; i += 1024) c += (!has_ignore || t[i] != ignore_index) ? 1.f : 0.f;
  // counts up to 2^24 are exact in fp32; larger inputs use the int path below
  c = block_sum<16>(c, red);
  if (threadIdx.x == 0) *n_valid = rows < (1 << 24) ? (int)c : -1;
  if (rows >= (1 << 24)) {
    __syncthreads();
    if (threadIdx.x == 0) {
      int64_t n = 0;
      for (int64_t i = 0; i < rows; ++i) n += (!has_ignore || t[i] != ignore_index);
      *n_valid = (int)(n > 0x7fffffff ? 0x7fffffff : n);
    }
  }
}

// The CrossEntropy launch plan, one block: *n_valid = the rows whose target is
// not the ignore index (the divisor of 'mean') and rowmap[0 .. *n_live) the rows
// that get a gradient (target not ignored and inside [0, V)), in order, so the
// persistent grid can deal them out evenly. Rows are taken 1024 at a time
// (row s*1024 + thread, up to kSteps steps a pass): each wave's ballot of its
// 64 rows is counted into LDS, one barrier, then every wave knows the live
// rows before its own and writes its live rows packed (coalesced stores).
// rows < 2^31 (the launcher checks).
__global__ __launch_bounds__(1024) void ce_plan_kernel(int* __restrict__ n_valid, int* __restrict__ rowmap,
                                                       int* __restrict__ n_live, const int64_t* __restrict__ t,
                                                       int64_t rows, int64_t V, int64_t ignore_index,
                                                       int has_ignore) {
  constexpr int kSteps = 8;
  __shared__ int cnt[kSteps][16];
  __shared__ int vcnt[16];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const uint64_t below = (1ull << lane) - 1ull;
  int live_base = 0, valid_total = 0;  // the same in every lane
  for (int64_t p0 = 0; p0 < rows; p0 += kSteps * 1024) {
    uint64_t bal[kSteps];
    int valid = 0;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      const int64_t r = p0 + s * 1024 + threadIdx.x;
      const int64_t tr = r < rows ? t[r] : 0;
      const bool v = r < rows && (!has_ignore || tr != ignore_index);
      valid += v;
      bal[s] = __ballot(v && tr >= 0 && tr < V);
    }
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) valid += __shfl_xor(valid, o, kWave);
    if (lane == 0) {
#pragma unroll
      for (int s = 0; s < kSteps; ++s) cnt[s][wave] = __popcll(bal[s]);
      vcnt[wave] = valid;
    }
    __syncthreads();
    // rowmap order: step, then wave, then lane
    int run = live_base;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      int before = 0, step_total = 0;
      for (int w = 0; w < 16; ++w) {
        const int c = cnt[s][w];
        step_total += c;
        before += w < wave ? c : 0;
      }
      if (bal[s] >> lane & 1ull) rowmap[run + before + __popcll(bal[s] & below)] = (int)(p0 + s * 1024 + threadIdx.x);
      run += step_total;
    }
    int vt = 0;
    for (int w = 0; w < 16; ++w) vt += vcnt[w];
    live_base = run;
    valid_total += vt;
    __syncthreads();  // cnt and vcnt are rewritten by the next pass
  }
  if (threadIdx.x == 0) {
    *n_valid = valid_total;
    *n_live = live_base;
  }
}

// out[0] = sum(loss_rows) (fp64 accumulation), divided by max(n_valid, 1) when requested
__global__ __launch_bounds__(1024) void sum_rows_kernel(float* __restrict__ out, const float* __restrict__ v,
                                                        int64_t n, const int* __restrict__ n_valid, int divide) {
  __shared__ double red[16];
  constexpr int U = 8;  // loads of a lane in flight before its adds (the adds keep the order i, i + 1024, ...)
  double s = 0.0;
  for (int64_t i0 = threadIdx.x; i0 < n; i0 += U * 1024) {
    float x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) x[u] = i0 + u * 1024 < n ? v[i0 + u * 1024] : 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i0 + u * 1024 < n) s += (double)x[u];
  }
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, kWave);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x / 64] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
    for (int i = 0; i < 16; ++i) t += red[i];
    if (divide) t /= (double)(*n_valid > 1 ? *n_valid : 1);
    out[0] = (float)t;
  }
}

// out = in * g (g scalar or per row); with g_prev, out = in * g / g_prev (0 where g_prev = 0).
// skip_if_one: a scalar g equal to 1 (and no g_prev) leaves the data untouched.
// A flat grid-stride walk with U loads of a lane in flight before its stores,
// the shape of the fastest streaming copy (one 256-lane block per CU). out may
// alias in: a lane reads each of its elements before it writes that element.
template <typename T, int VEC, int U = 4>
__global__ __launch_bounds__(256) void scale_rows_kernel(T* out, const T* in, const float* __restrict__ g,
                                                         const float* __restrict__ g_prev, int per_row,
                                                         int skip_if_one, int64_t rows, int64_t cols, int64_t ld_in,
                                                         int64_t ld_out) {
  if (!per_row && skip_if_one && g_prev == nullptr && g[0] == 1.f && out == in) return;
  const int64_t nv = cols / VEC;
  const int64_t total = rows * nv;
  const double rinv = 1.0 / (double)nv;
  const int64_t stride = (int64_t)gridDim.x * 256;
  float f0 = g[0];
  if (!per_row && g_prev) f0 = g_prev[0] != 0.f ? f0 / g_prev[0] : 0.f;
  for (int64_t i0 = (int64_t)blockIdx.x * 256 + threadIdx.x; i0 < total; i0 += U * stride) {
    Pack<T, VEC> x[U];
    int64_t r[U], cv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + u * stride;
      // row of vector i: a double-precision quotient, corrected by one step
      int64_t q = (int64_t)((double)i * rinv);
      q -= q * nv > i;
      q += (q + 1) * nv <= i;
      r[u] = q;
      cv[u] = (i - q * nv) * VEC;
      if (i < total) x[u] = load_pack<T, VEC>(in + q * ld_in + cv[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (i0 + u * stride < total) {
        float f = f0;
        if (per_row) {
          f = g[r[u]];
          if (g_prev) {
            const float pv = g_prev[r[u]];
            f = pv != 0.f ? f / pv : 0.f;
          }
        }
        float v[VEC];
        unpack(x[u], v);
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[e] *= f;
        store_pack<T, VEC>(out + r[u] * ld_out + cv[u], pack<T, VEC>(v));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// selective log-softmax and GRPO
// ---------------------------------------------------------------------------
__device__ __forceinline__ float load_mask(const void* m, int dt, int64_t off) {
  switch (dt) {
    case HK_F32: return ((const float*)m)[off];
    case HK_F16: return (float)((const _Float16*)m)[off];
    case HK_BF16: return (float)((const __bf16*)m)[off];
    case HK_U8: return (float)((const uint8_t*)m)[off];
    case HK_I32: return (float)((const int32_t*)m)[off];
    case HK_I64: return (float)((const int64_t*)m)[off];
  }
  return 1.f;
}

struct GrpoArgs {
  const int64_t* ids;
  int64_t ids_sB, ids_sL;
  const float* adv;
  const float* old_logp;
  int64_t old_sB, old_sL;
  const float* ref_logp;
  int64_t ref_sB, ref_sL;
  const void* mask;
  int mask_dt;
  int64_t mask_sB, mask_sL;
  int64_t B, L, V;
  float inv_T, beta, eps_lo, eps_hi;
  float* lse_rows;       // [B, L] outputs
  float* loss_rows;
  float* kl_rows;
  float* clip_rows;
  float* logp_out;       // selective log-softmax output [B, L]
};

// logp[b, l] = x[b, l, id] / T - logsumexp(x[b, l, :] / T) for unmasked l < L
// (kernels/grpo_loss.py:29-62); logits are (B, L+1, V) contiguous. Masked
// tokens get 0 and their rows are not read.
template <typename T, int VEC, int NCH, int BLOCK, bool RESIDENT>
__global__ __launch_bounds__(BLOCK) void selective_log_softmax_kernel(const T* __restrict__ logits, GrpoArgs a) {
  __shared__ float red[BlockRed<BLOCK / kWave>::kFloats];
  const int64_t rows = a.B * a.L;
  const float c = kLog2e * a.inv_T;
  auto row_ptr = [&](int64_t r) {
    const int64_t b = r / a.L, l = r - b * a.L;
    return logits + (b * (a.L + 1) + l) * a.V;
  };
  auto masked = [&](int64_t r) {
    const int64_t b = r / a.L, l = r - b * a.L;
    return a.mask && load_mask(a.mask, a.mask_dt, b * a.mask_sB + l * a.mask_sL) == 0.f;
  };
  auto target = [&](int64_t r) {
    const int64_t b = r / a.L, l = r - b * a.L;
    const int64_t id = a.ids[b * a.ids_sB + l * a.ids_sL];
    const bool in_range = id >= 0 && id < a.V;
    return TargetLogit{id, in_range ? to_f32<T>(row_ptr(r)[id]) : 0.f};
  };
  auto emit = [&](int64_t r, float lse2, TargetLogit tx) {
    if (threadIdx.x == 0)
      a.logp_out[r] = (tx.t >= 0 && tx.t < a.V) ? tx.xt * a.inv_T - lse2 * kLn2 : NAN;
  };
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x)
    if (threadIdx.x == 0 && masked(r)) a.logp_out[r] = 0.f;
  if constexpr (RESIDENT) {
    const int64_t G = gridDim.x;
    auto next_live = [&](int64_t q) {
      while (q < rows && masked(q)) q += G;
      return q;
    };
    lse_rows_resident<T, VEC, NCH, BLOCK>(row_len(a.V), c, rows, red, row_ptr, next_live, target, NoTarget{},
                                          emit);
  } else {
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
      if (masked(r)) continue;
      const float lse2 = row_lse2_stream<T, VEC, BLOCK>(row_ptr(r), (int)a.V, c, red);
      if (threadIdx.x == 0) emit(r, lse2, target(r));  // (after the row, as in the CE kernel)
    }
  }
}

// Per-token inputs of the fused GRPO kernel, gathered by grpo_prep_kernel so
// the hot kernel carries a handful of arguments instead of ~30 (its row loop
// otherwise runs out of SGPRs and spills).
struct alignas(16) GrpoTok {
  int32_t id;   // completion token id (-1 if out of range)
  float old;    // old policy log-prob (unused when the call has none)
  float ref;    // reference log-prob (unused when beta == 0)
  float adv;    // advantage of the sequence
  float m;      // mask value (0: token skipped)
  float gs;     // m / (max(len_b, 1) * B) / T: dloss / T at unit upstream gradient
  float pad0, pad1;
};
// A token record as one scalar load (s_load_dwordx8): a field-by-field copy
// may be split into loads that the scalar unit has no form for, and those go
// to the vector unit.
__device__ __forceinline__ GrpoTok load_tok(const GrpoTok* p) {
  typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
  static_assert(sizeof(GrpoTok) == sizeof(u32x8), "one 32-byte record");
  return __builtin_bit_cast(GrpoTok, scalar_load(reinterpret_cast<const u32x8*>(p)));
}
struct alignas(16) GrpoOut {
  float lse, loss, kl, clip;
};

struct GrpoHot {
  const GrpoTok* tok;
  GrpoOut* out;
  int64_t B, L, V;
  int64_t W, ld;  // row width the kernel reads (V, or more with -inf padding past V) and row stride
  int64_t row0, nrows;  // the launch covers rows [row0, row0 + nrows) of the (B, L+1) positions
  // optional compaction: launch row q is position rowmap[row0 + q], and only
  // q < *nlim - row0 exist (a device-side bound)
  const int* rowmap;
  const int* nlim;
  float inv_T, beta, eps_lo, eps_hi;
  int has_old;
};

// GRPO forward with the gradient fused in (kernels/grpo_loss.py:87-159 forward,
// :166-234 backward at unit upstream gradient). Rows are positions
// [row0, row0 + nrows) of the B*(L+1) logits rows; `logits` and `dlogits`
// point at row row0. The last position and masked tokens get a zero gradient row.
// The per-token loss terms from logp (kernels/grpo_loss.py:103-133): the
// result row and d loss / d logp.
__device__ __forceinline__ GrpoOut grpo_terms(const GrpoHot& a, const GrpoTok& tk, float lse, float logp,
                                             float* dlogp_out) {
  const float old = a.has_old ? tk.old : logp;
  const float coef1 = exp_fast(logp - old);
  const float A = tk.adv;
  const float coef2 = fminf(fmaxf(coef1, 1.f - a.eps_lo), 1.f + a.eps_hi);
  const float l1 = coef1 * A, l2 = coef2 * A;
  float loss = -fminf(l1, l2);
  float kl = 0.f;
  float dlogp = l2 >= l1 ? -coef1 * A : 0.f;
  if (a.beta != 0.f) {
    const float d = tk.ref - logp;
    const float ed = exp_fast(d);
    kl = ed - d - 1.f;
    loss += a.beta * kl;
    dlogp += a.beta * (1.f - ed);
  }
  *dlogp_out = dlogp;
  const bool clipped = (coef1 < 1.f - a.eps_lo && A < 0.f) || (coef1 > 1.f + a.eps_hi && A > 0.f);
  return GrpoOut{lse, loss, kl, clipped ? 1.f : 0.f};
}

template <typename T, int VEC, int NCH, int BLOCK, bool RESIDENT, bool GRAD>
__global__ __launch_bounds__(BLOCK) void grpo_kernel(T* dlogits, const T* logits, GrpoHot a) {
  // dlogits may alias logits (FusedLinear-GRPO writes the gradient over the
  // chunk's logits): every element is read by the thread that later
  // overwrites it (the gradient path takes the id logit from the registers,
  // the forward-only paths read it before the row's reduction barriers) and a
  // row's stores are issued before the next row's loads of the same vector,
  // so the pointers are not declared __restrict__.
  __shared__ float red[BlockRed<BLOCK / kWave>::kFloats];
  const int64_t rows =
      a.nlim ? min(a.nrows, max((int64_t)0, (int64_t)*a.nlim - a.row0)) : a.nrows;  // row below: local to the launch
  const int64_t G = gridDim.x;
  const float c = kLog2e * a.inv_T;
  // a row is live when it is a token position (l < L) with a nonzero mask
  auto pos = [&](int64_t row) -> int64_t { return a.rowmap ? a.rowmap[a.row0 + row] : a.row0 + row; };
  auto live = [&](int64_t row, GrpoTok* tk) {
    const int64_t g = pos(row), b = g / (a.L + 1), l = g - b * (a.L + 1);
    if (l == a.L) return false;
    *tk = a.tok[b * a.L + l];
    return tk->m != 0.f;
  };
  auto token = [&](int64_t row) {
    const int64_t g = pos(row), b = g / (a.L + 1);
    return g - b;  // b * L + l
  };
  // dead rows: a zero gradient row (never read) and zero results
  for (int64_t row = blockIdx.x; row < rows; row += G) {
    GrpoTok tk{};
    if (!live(row, &tk)) {
      if constexpr (GRAD) fill_row<T, VEC, BLOCK>(dlogits + row * a.ld, (int)a.W, 0.f);
      const int64_t g = pos(row), b = g / (a.L + 1), l = g - b * (a.L + 1);
      if (l < a.L && threadIdx.x == 0) a.out[b * a.L + l] = GrpoOut{0.f, 0.f, 0.f, 0.f};
    }
  }
  if constexpr (RESIDENT && (GRAD || BLOCK < 1024)) {
    // Without the gradient (256/512 lanes) the same loop minus the stores, the
    // next row's loads issued right after this row's lane reduction: the same
    // reduction, exchange and merge as with the gradient, so the losses are
    // equal bit for bit, and no per-row global load (token record, id logit)
    // waits behind the row's vector loads.
    // Live rows, pipelined as in the CE kernel: the register refill rides
    // with the gradient stores, the per-row records are scalar loads (the
    // search for the row after next runs at the end of the iteration) and the
    // id logit comes out of the registers through the block exchange.
    using Regs = RowRegs<T, VEC, NCH, BLOCK, full_vectors(NCH, BLOCK)>;
    // (the token's id rides along; the rest of its record is loaded again
    // when the row starts, in time for the loss terms after the exchange)
    struct LiveRow {
      int64_t row, tok_i;  // row >= rows: none
      int id;
    };
    auto next_live = [&](int64_t from) {
      LiveRow q{from, 0, -1};
      for (; q.row < rows; q.row += G) {
        const int64_t g = a.rowmap ? scalar_load(a.rowmap + a.row0 + q.row) : a.row0 + q.row;
        const int64_t b = g / (a.L + 1), l = g - b * (a.L + 1);
        if (l == a.L) continue;
        q.tok_i = b * a.L + l;
        const GrpoTok tk = load_tok(a.tok + q.tok_i);
        q.id = tk.id;
        if (tk.m != 0.f) break;
      }
      return q;
    };
    LiveRow cur = next_live(blockIdx.x);
    if (cur.row >= rows) return;
    Regs r;
    r.load(logits + cur.row * a.ld, row_len(a.W));
    LiveRow next = next_live(cur.row + G);
    int parity = 0;
    for (;;) {
      const int n = row_len(a.W);  // per iteration (see row_len)
      const int64_t row = cur.row;
      const int id = cur.id;
      const T* in = logits + row * a.ld;
      const T* src = next.row < rows ? logits + next.row * a.ld : in;  // unconditional (see the CE kernel)
      const GrpoTok tk = load_tok(a.tok + cur.tok_i);
      float m, s, xt, M, R, X, rest;
      r.reduce_lane(n, c, id, &m, &s, &xt);
      if constexpr (!GRAD) {
        r.opaque();
        __builtin_amdgcn_sched_barrier(0);  // the refill may not start before the row is reduced (register reuse)
        if (next.row < rows) r.load(src, n);
      }
      block_lse2_ms<BLOCK / kWave>(m, s, red, parity, &M, &R, xt, Regs::owns_target(id), &X);
      const float xid = id >= 0 ? X : 0.f;
      const float lse2 = target_merge(M, R, xid * c, id >= 0, &rest);
      parity ^= 1;
      if constexpr (GRAD) r.opaque();
      const float lse = lse2 * kLn2;
      const float logp = id >= 0 ? xid * a.inv_T - lse : NAN;
      float dlogp;
      const GrpoOut res = grpo_terms(a, tk, lse, logp, &dlogp);
      if constexpr (GRAD) {
        // d loss / d logits_j = -dlogp * (p_j - [j == id]) * dloss / T
        const float g = -dlogp * tk.gs;
        T* out = dlogits + row * a.ld;
        r.store_prob_grad_then_load(out, n, c, lse2, g, src);
        // the id element: (p_id - 1) * g = -(1 - p_id) * g (see reduce_lane)
        if (Regs::owns_target(id)) out[id] = from_f32<T>(-rest * g);
      }
      if (threadIdx.x == 0) a.out[cur.tok_i] = res;
      if (next.row >= rows) break;
      cur = next;
      next = next_live(cur.row + G);
    }
  } else {
    // streaming, or forward only on 1024-lane rows: there the refill's extra
    // register pressure spills, so each row loads after the previous one
    int parity = 0;
    for (int64_t row = blockIdx.x; row < rows; row += G) {
      GrpoTok tk{};
      if (!live(row, &tk)) continue;
      T* out = GRAD ? dlogits + row * a.ld : nullptr;
      const T* in = logits + row * a.ld;
      const int n = row_len(a.W);
      // the id logit is read before the reduction's barriers: dlogits may alias
      // logits, and no lane stores before every lane has passed them
      const float xid = tk.id >= 0 ? to_f32<T>(in[tk.id]) : 0.f;
      float lse2, rest = 0.f;
      if constexpr (RESIDENT) {  // (forward only: the gradient form's arithmetic, see lse_rows_resident)
        RowRegs<T, VEC, NCH, BLOCK> r;
        r.load(in, n);
        float m, s, M, S;
        r.reduce_lane(n, c, tk.id, &m, &s);
        block_lse2_ms<BLOCK / kWave>(m, s, red, parity, &M, &S);
        lse2 = target_merge(M, S, xid * c, tk.id >= 0, &rest);
        parity ^= 1;
      } else {
        lse2 = row_lse2_stream<T, VEC, BLOCK, GRAD>(in, n, c, red, tk.id, &rest);
      }
      const float lse = lse2 * kLn2;
      const float logp = tk.id >= 0 ? xid * a.inv_T - lse : NAN;
      float dlogp;
      const GrpoOut res = grpo_terms(a, tk, lse, logp, &dlogp);
      if (threadIdx.x == 0) a.out[token(row)] = res;
      if constexpr (GRAD) store_grad_stream<T, VEC, BLOCK>(out, in, n, c, lse2, tk.id, rest, -dlogp * tk.gs);
    }
  }
}

// One block per sequence b: len_b = sum_l mask[b, l], then the token records;
// the per-token results start at zero (rows a launch skips keep them).
__global__ __launch_bounds__(1024) void grpo_prep_kernel(GrpoArgs a, GrpoTok* __restrict__ tok,
                                                         GrpoOut* __restrict__ res) {
  __shared__ float red[16];
  const int64_t b = blockIdx.x;
  float s = 0.f;
  for (int64_t l = threadIdx.x; l < a.L; l += 1024)
    s += a.mask ? load_mask(a.mask, a.mask_dt, b * a.mask_sB + l * a.mask_sL) : 1.f;
  s = block_sum<16>(s, red);
  const float inv_len = 1.f / (fmaxf(s, 1.f) * (float)a.B);
  const float A = a.adv[b];
  for (int64_t l = threadIdx.x; l < a.L; l += 1024) {
    GrpoTok t{};
    const int64_t id = a.ids[b * a.ids_sB + l * a.ids_sL];
    t.id = (id >= 0 && id < a.V) ? (int32_t)id : -1;
    t.old = a.old_logp ? a.old_logp[b * a.old_sB + l * a.old_sL] : 0.f;
    t.ref = a.ref_logp ? a.ref_logp[b * a.ref_sB + l * a.ref_sL] : 0.f;
    t.adv = A;
    t.m = a.mask ? load_mask(a.mask, a.mask_dt, b * a.mask_sB + l * a.mask_sL) : 1.f;
    t.gs = t.m * inv_len * a.inv_T;
    tok[b * a.L + l] = t;
    res[b * a.L + l] = GrpoOut{0.f, 0.f, 0.f, 0.f};
  }
}

// Finalize, first pass: one block per (sequence b, chunk c) of kFinChunk
// tokens, one token a lane. Scatters the per-token rows and writes the chunk's
// [sum m*loss, sum m, sum m*kl, sum m*clip] (fp64) to part[b * chunks + c].
// Many small blocks: every load of the pass is in flight at once.
constexpr int kFinChunk = 256;
struct alignas(16) GrpoPart {
  double loss, m, kl, clip;
};

__device__ __forceinline__ double wave_sum_f64(double v) {
  for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__global__ __launch_bounds__(kFinChunk) void grpo_partial_kernel(GrpoArgs a, const GrpoTok* __restrict__ tok,
                                                                 const GrpoOut* __restrict__ res,
                                                                 GrpoPart* __restrict__ part, int64_t chunks) {
  constexpr int NW = kFinChunk / kWave;
  __shared__ double red[4][NW];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int64_t b = blockIdx.x / chunks, c = blockIdx.x - b * chunks;
  const int64_t l = c * kFinChunk + threadIdx.x;
  double ls = 0.0, ms = 0.0, ks = 0.0, cs = 0.0;
  if (l < a.L) {
    const int64_t o = b * a.L + l;
    const double m = tok[o].m;
    const GrpoOut r = res[o];
    ls = m * r.loss;
    ms = m;
    ks = m * r.kl;
    cs = m * r.clip;
    a.lse_rows[o] = r.lse;
    a.loss_rows[o] = r.loss;
    a.kl_rows[o] = r.kl;
    a.clip_rows[o] = r.clip;
  }
  ls = wave_sum_f64(ls);
  ms = wave_sum_f64(ms);
  ks = wave_sum_f64(ks);
  cs = wave_sum_f64(cs);
  if (lane == 0) {
    red[0][wave] = ls;
    red[1][wave] = ms;
    red[2][wave] = ks;
    red[3][wave] = cs;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    GrpoPart p{0.0, 0.0, 0.0, 0.0};
    for (int w = 0; w < NW; ++w) {
      p.loss += red[0][w];
      p.m += red[1][w];
      p.kl += red[2][w];
      p.clip += red[3][w];
    }
    part[blockIdx.x] = p;
  }
}

// Finalize, second pass (one block):
// out = [mean_b(sum_l m*loss / max(len_b,1)), sum m*kl / max(sum m,1), sum m*clip / max(sum m,1)]
// (kernels/grpo_loss.py:290-295). Each wave owns whole sequences (b = wave,
// wave + 16, ...) and sums their chunk partials; one block-wide combine at the
// end. A fixed order throughout: the result does not depend on scheduling.
__global__ __launch_bounds__(1024) void grpo_finalize_kernel(GrpoArgs a, const GrpoPart* __restrict__ part,
                                                             int64_t chunks, float* __restrict__ loss_out,
                                                             float* __restrict__ kl_out,
                                                             float* __restrict__ clip_out) {
  __shared__ double red[4][16];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  double loss = 0.0, msum = 0.0, kls = 0.0, clips = 0.0;
  for (int64_t b = wave; b < a.B; b += 16) {
    double ls = 0.0, ms = 0.0, ks = 0.0, cs = 0.0;
    for (int64_t c = lane; c < chunks; c += kWave) {
      const GrpoPart p = part[b * chunks + c];
      ls += p.loss;
      ms += p.m;
      ks += p.kl;
      cs += p.clip;
    }
    ls = wave_sum_f64(ls);
    ms = wave_sum_f64(ms);
    loss += ls / (ms > 1.0 ? ms : 1.0);
    msum += ms;
    kls += wave_sum_f64(ks);
    clips += wave_sum_f64(cs);
  }
  if (lane == 0) {
    red[0][wave] = loss;
    red[1][wave] = msum;
    red[2][wave] = kls;
    red[3][wave] = clips;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double t[4] = {0.0, 0.0, 0.0, 0.0};
    for (int i = 0; i < 16; ++i)
      for (int k = 0; k < 4; ++k) t[k] += red[k][i];
    const double d = t[1] > 1.0 ? t[1] : 1.0;
    loss_out[0] = (float)(t[0] / (double)a.B);
    if (kl_out) kl_out[0] = (float)(t[2] / d);
    clip_out[0] = (float)(t[3] / d);
  }
}

// Stable compaction of the live rows of [0, rows): rowmap[0 .. n) lists them in
// order, inv[r] is a row's place in that list (-1 when dead), *n_live = n. One
// block: per 1024 rows, a wave ballot and an exclusive scan of the 16 wave counts.
template <class Pred>
__global__ __launch_bounds__(1024) void compact_rows_kernel(int* __restrict__ rowmap, int* __restrict__ inv,
                                                            int* __restrict__ n_live, int64_t rows, Pred pred) {
  __shared__ int wcount[16];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  int base = 0;  // live rows before this 1024-row step (every lane keeps the same value)
  for (int64_t r0 = 0; r0 < rows; r0 += 1024) {
    const int64_t r = r0 + threadIdx.x;
    const bool f = r < rows && pred(r);
    const uint64_t bal = __ballot(f);
    if (lane == 0) wcount[wave] = __popcll(bal);
    __syncthreads();
    int before = base, total = base;
    for (int w = 0; w < 16; ++w) {
      before += w < wave ? wcount[w] : 0;
      total += wcount[w];
    }
    const int k = before + __popcll(bal & ((1ull << lane) - 1ull));
    if (r < rows) {
      inv[r] = f ? k : -1;
      if (f) rowmap[k] = (int)r;
    }
    base = total;
    __syncthreads();  // wcount is rewritten by the next step
  }
  if (threadIdx.x == 0) *n_live = base;
}

// CrossEntropy rows: live unless the target is the ignore index.
struct CeLive {
  const int64_t* targets;
  int64_t ignore_index;
  __device__ bool operator()(int64_t r) const { return targets[r] != ignore_index; }
};

// GRPO positions of the (B, L+1) rows: live when l < L and the mask is nonzero.
struct GrpoLive {
  const void* mask;
  int mask_dt;
  int64_t mask_sB, mask_sL, L;
  __device__ bool operator()(int64_t r) const {
    const int64_t b = r / (L + 1), l = r - b * (L + 1);
    return l < L && (!mask || load_mask(mask, mask_dt, b * mask_sB + l * mask_sL) != 0.f);
  }
};

// ---------------------------------------------------------------------------
// host-side configuration
// ---------------------------------------------------------------------------
template <typename T> struct Tag { using type = T; };

template <typename F>
int dispatch_t(int dt, F&& f) {
  switch (dt) {
    case HK_F32: return f(Tag<float>{});
    case HK_F16: return f(Tag<_Float16>{});
    case HK_BF16: return f(Tag<__bf16>{});
  }
  set_error("invalid logits dtype code %d", dt);
  return HK_EINVAL;
}

// (block, vectors per lane) pairs with a register-resident instantiation
struct RowCfg {
  int block;
  int nch;  // 0: streaming
  int vec;  // elements per vector
};

RowCfg choose_row_cfg(int64_t V, int esize, bool vec_ok) {
  RowCfg c{1024, 0, vec_ok ? 16 / esize : 1};
  if (!vec_ok) return c;
  const int64_t nv = V / c.vec;
  for (const RowForm& f : kRowForms)
    if (nv <= (int64_t)f.block * f.nch) return RowCfg{f.block, f.nch, c.vec};
  return c;
}

template <typename F>
int dispatch_cfg(const RowCfg& c, F&& f) {
  using std::integral_constant;
  if (c.nch == 0) return f(integral_constant<int, 1024>{}, integral_constant<int, 0>{});
  if (c.block == 256) {
    switch (c.nch) {
      case 1: return f(integral_constant<int, 256>{}, integral_constant<int, 1>{});
      case 2: return f(integral_constant<int, 256>{}, integral_constant<int, 2>{});
      case 4: return f(integral_constant<int, 256>{}, integral_constant<int, 4>{});
      case 8: return f(integral_constant<int, 256>{}, integral_constant<int, 8>{});
      case 12: return f(integral_constant<int, 256>{}, integral_constant<int, 12>{});
    }
  } else if (c.block == 512) {
    switch (c.nch) {
      case 8: return f(integral_constant<int, 512>{}, integral_constant<int, 8>{});
      case 12: return f(integral_constant<int, 512>{}, integral_constant<int, 12>{});
      case 16: return f(integral_constant<int, 512>{}, integral_constant<int, 16>{});
    }
  } else {
    switch (c.nch) {
      case 12: return f(integral_constant<int, 1024>{}, integral_constant<int, 12>{});
      case 16: return f(integral_constant<int, 1024>{}, integral_constant<int, 16>{});
      case 20: return f(integral_constant<int, 1024>{}, integral_constant<int, 20>{});
      case 24: return f(integral_constant<int, 1024>{}, integral_constant<int, 24>{});
    }
  }
  set_error("internal: bad row config (%d, %d)", c.block, c.nch);
  return HK_EINVAL;
}

// The kernels take the leading full_vectors() vectors of a register-resident
// form as full without testing them; choose_row_cfg's order guarantees it.
bool form_fits(int64_t V, const RowCfg& c) {
  const int64_t need = (int64_t)full_vectors(c.nch, c.block) * c.block * c.vec;
  if (V >= need && V <= (int64_t)c.nch * c.block * c.vec) return true;
  set_error("internal: a row of %lld elements given to the (%d x %d) form", (long long)V, c.block, c.nch);
  return false;
}

// A persistent grid: `rounds` times the blocks the CUs hold at once for this
// kernel (its occupancy), or one per row when there are fewer rows. With two
// rounds, the second round's blocks start as the first round's finish, which
// evens out rows of uneven cost: GRPO's prefix-masked positions, strided over
// the grid, give some blocks a third more live rows than others (C4 1.70 ms
// with one round, 1.65 with two), and CrossEntropy's 1024-lane form gains 1%
// ([8192, 128256]: 744 against 750 us). The smaller CrossEntropy forms keep
// one round, where each block's next-row prefetch covers more rows (2048 x
// 32000: 64 against 70 us).
int64_t resident_grid(const void* kernel, int64_t rows, int block, int rounds = 1) {
  const int dev = current_device();
  const int cu = dev >= 0 ? cu_count(dev) : 256;
  const int64_t g = (int64_t)(cu > 0 ? cu : 256) * blocks_per_cu(kernel, block) * rounds;
  return rows < g ? (rows > 0 ? rows : 1) : g;
}

bool valid_float_dtype(int dt) { return dt == HK_F32 || dt == HK_F16 || dt == HK_BF16; }
bool valid_mask_dtype(int dt) {
  return dt == HK_F32 || dt == HK_F16 || dt == HK_BF16 || dt == HK_U8 || dt == HK_I32 || dt == HK_I64;
}
int esize(int dt) { return dt == HK_F32 ? 4 : 2; }

}  // namespace
}  // namespace hk

namespace hk {

namespace {
GrpoArgs grpo_args(const GrpoInputs& in) {
  GrpoArgs a{};
  a.ids = in.ids;
  a.ids_sB = in.ids_sB;
  a.ids_sL = in.ids_sL;
  a.adv = in.adv;
  a.old_logp = in.old_logp;
  a.old_sB = in.old_sB;
  a.old_sL = in.old_sL;
  a.ref_logp = in.ref_logp;
  a.ref_sB = in.ref_sB;
  a.ref_sL = in.ref_sL;
  a.mask = in.mask;
  a.mask_dt = in.mask_dt;
  a.mask_sB = in.mask_sB;
  a.mask_sL = in.mask_sL;
  a.B = in.B;
  a.L = in.L;
  a.V = in.V;
  a.inv_T = 1.f / in.temperature;
  a.beta = in.beta;
  a.eps_lo = in.eps_lo;
  a.eps_hi = in.eps_hi;
  return a;
}
}  // namespace

int64_t grpo_fin_chunks(int64_t L) { return (L + kFinChunk - 1) / kFinChunk; }

size_t grpo_scratch_bytes(int64_t B, int64_t L) {
  // token records, per-token results, then the finalize's chunk partials
  return (size_t)(B * L) * (sizeof(GrpoTok) + sizeof(GrpoOut)) + (size_t)(B * grpo_fin_chunks(L)) * sizeof(GrpoPart) +
         256;
}

int grpo_check(const GrpoInputs& in) {
  HK_REQUIRE(in.B > 0 && in.L >= 0 && in.V > 0, "invalid shape B=%lld L=%lld V=%lld", (long long)in.B,
             (long long)in.L, (long long)in.V);
  HK_REQUIRE(in.temperature > 0.f, "temperature must be positive");
  HK_REQUIRE(!in.mask || valid_mask_dtype(in.mask_dt), "invalid mask dtype code %d", in.mask_dt);
  HK_REQUIRE(in.beta == 0.f || in.ref_logp != nullptr, "beta != 0 needs ref_logp");
  HK_REQUIRE(in.V < (1LL << 31) - 4096, "V=%lld too large", (long long)in.V);
  HK_REQUIRE(in.ids && in.adv, "null pointer argument");
  return HK_OK;
}

int grpo_prep_launch(const GrpoInputs& in, void* scratch, hipStream_t st) {
  if (in.L == 0) return HK_OK;
  hipLaunchKernelGGL(grpo_prep_kernel, dim3((unsigned)in.B), dim3(1024), 0, st, grpo_args(in), (GrpoTok*)scratch,
                     (GrpoOut*)((char*)scratch + (size_t)(in.B * in.L) * sizeof(GrpoTok)));
  return check_launch("grpo_prep_kernel");
}

int grpo_rows_launch(void* dlogits, const void* logits, int64_t row0, int64_t nrows, const GrpoInputs& in,
                     void* scratch, int dtype, hipStream_t st, const int* rowmap, const int* n_live, int64_t width,
                     int64_t ld) {
  if (nrows <= 0) return HK_OK;
  if (width <= 0) width = in.V;
  if (ld <= 0) ld = width;
  HK_REQUIRE(width >= in.V && ld >= width, "GRPO rows: width %lld / stride %lld below V = %lld", (long long)width,
             (long long)ld, (long long)in.V);
  GrpoHot h{};
  h.rowmap = rowmap;
  h.nlim = n_live;
  h.tok = (const GrpoTok*)scratch;
  h.out = (GrpoOut*)((char*)scratch + (size_t)(in.B * in.L) * sizeof(GrpoTok));
  h.B = in.B;
  h.L = in.L;
  h.V = in.V;
  h.W = width;
  h.ld = ld;
  h.row0 = row0;
  h.nrows = nrows;
  h.inv_T = 1.f / in.temperature;
  h.beta = in.beta;
  h.eps_lo = in.eps_lo;
  h.eps_hi = in.eps_hi;
  h.has_old = in.old_logp != nullptr;
  const int es = esize(dtype);
  const bool vec_ok = width % (16 / es) == 0 && (ld * es) % 16 == 0 && aligned_to(logits, 16) &&
                      (!dlogits || aligned_to(dlogits, 16));
  const RowCfg cfg = choose_row_cfg(width, es, vec_ok);
  return dispatch_t(dtype, [&](auto tt) {
    using T = typename decltype(tt)::type;
    return dispatch_cfg(cfg, [&](auto blk, auto nch) {
      constexpr int BLOCK = decltype(blk)::value;
      constexpr int NCH = decltype(nch)::value;
      auto run = [&](auto kern, int block) {
        const dim3 grid((unsigned)resident_grid((const void*)kern, nrows, block, 2));
        hipLaunchKernelGGL(kern, grid, dim3(block), 0, st, (T*)dlogits, (const T*)logits, h);
        return check_launch("grpo_kernel");
      };
      auto go = [&](auto grad_c) {
        constexpr bool GRAD = decltype(grad_c)::value;
        if (cfg.vec == 1) return run(grpo_kernel<T, 1, 1, 1024, false, GRAD>, 1024);
        if constexpr (NCH == 0) {
          return run(grpo_kernel<T, 16 / sizeof(T), 1, BLOCK, false, GRAD>, BLOCK);
        } else {
          // the resident form takes its leading full vectors untested (see form_fits)
          if (!form_fits(width, cfg)) return HK_EINVAL;
          return run(grpo_kernel<T, 16 / sizeof(T), NCH, BLOCK, true, GRAD>, BLOCK);
        }
      };
      if (dlogits) return go(std::true_type{});
      return go(std::false_type{});
    });
  });
}

int grpo_finalize_launch(const GrpoInputs& in, const void* scratch, float* loss_out, float* kl_out, float* clip_out,
                         float* lse_rows, float* loss_rows, float* kl_rows, float* clip_rows, hipStream_t st) {
  GrpoArgs a = grpo_args(in);
  a.lse_rows = lse_rows;
  a.loss_rows = loss_rows;
  a.kl_rows = kl_rows;
  a.clip_rows = clip_rows;
  const size_t n = (size_t)(in.B * in.L);
  const GrpoTok* tok = (const GrpoTok*)scratch;
  const GrpoOut* res = (const GrpoOut*)((const char*)scratch + n * sizeof(GrpoTok));
  GrpoPart* part = (GrpoPart*)((char*)scratch + n * (sizeof(GrpoTok) + sizeof(GrpoOut)));
  const int64_t chunks = grpo_fin_chunks(in.L);
  HK_REQUIRE(in.B * chunks < (1LL << 31), "B=%lld L=%lld: too many finalize blocks", (long long)in.B,
             (long long)in.L);
  if (chunks > 0) {
    hipLaunchKernelGGL(grpo_partial_kernel, dim3((unsigned)(in.B * chunks)), dim3(kFinChunk), 0, st, a, tok, res,
                       part, chunks);
    const int rc = check_launch("grpo_partial_kernel");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(grpo_finalize_kernel, dim3(1), dim3(1024), 0, st, a, (const GrpoPart*)part, chunks, loss_out,
                     kl_out, clip_out);
  return check_launch("grpo_finalize_kernel");
}

int ce_compact_launch(int* rowmap, int* inv, int* n_live, const int64_t* targets, int64_t rows,
                      int64_t ignore_index, hipStream_t st) {
  hipLaunchKernelGGL(compact_rows_kernel<CeLive>, dim3(1), dim3(1024), 0, st, rowmap, inv, n_live, rows,
                     CeLive{targets, ignore_index});
  return check_launch("compact_rows_kernel");
}

int grpo_compact_launch(int* rowmap, int* inv, int* n_live, const GrpoInputs& in, hipStream_t st) {
  hipLaunchKernelGGL(compact_rows_kernel<GrpoLive>, dim3(1), dim3(1024), 0, st, rowmap, inv, n_live,
                     in.B * (in.L + 1), GrpoLive{in.mask, in.mask_dt, in.mask_sB, in.mask_sL, in.L});
  return check_launch("compact_rows_kernel");
}

int ce_plan_launch(int* n_valid, int* rowmap, int* n_live, const int64_t* targets, int64_t rows, int64_t V,
                   int64_t ignore_index, int has_ignore, hipStream_t st) {
  hipLaunchKernelGGL(ce_plan_kernel, dim3(1), dim3(1024), 0, st, n_valid, rowmap, n_live, targets, rows, V,
                     ignore_index, has_ignore);
  return check_launch("ce_plan_kernel");
}

int count_valid_launch(int* n_valid, const int64_t* targets, int64_t rows, int64_t ignore_index, int has_ignore,
                       hipStream_t st) {
  hipLaunchKernelGGL(count_valid_kernel, dim3(1), dim3(1024), 0, st, n_valid, targets, rows, ignore_index,
                     has_ignore);
  return check_launch("count_valid_kernel");
}

int sum_rows_launch(float* out, const float* v, int64_t n, const int* n_valid, int divide, hipStream_t st) {
  hipLaunchKernelGGL(sum_rows_kernel, dim3(1), dim3(1024), 0, st, out, v, n, n_valid, divide);
  return check_launch("sum_rows_kernel");
}

// Row configuration of a forward-only (read-only) row kernel: register-resident
// rows on 256 lanes up to 2048 vectors a row (16384 16-bit logits), where the
// next row's loads overlap the block combine; longer rows stream on 1024
// lanes, which measured as fast or faster for them than holding the row (a
// long resident row leaves few blocks a CU).
RowCfg choose_read_cfg(int64_t V, int esize, bool vec_ok) {
  const RowCfg c = choose_row_cfg(V, esize, vec_ok);
  if (c.nch > 0 && c.block == 256 && c.nch <= 8) return c;
  return RowCfg{1024, 0, c.vec};
}

// The inference forward over a.rows rows of a.V logits (row stride a.ld_in).
int ce_lse_launch(const void* logits, const CeArgs& a, int dtype, hipStream_t st) {
  const int es = esize(dtype);
  const bool vec_ok = a.V % (16 / es) == 0 && aligned_to(logits, 16) && (a.ld_in * es) % 16 == 0;
  const RowCfg cfg = choose_read_cfg(a.V, es, vec_ok);
  return dispatch_t(dtype, [&](auto tt) {
    using T = typename decltype(tt)::type;
    return dispatch_cfg(cfg, [&](auto blk, auto nch) {
      constexpr int BLOCK = decltype(blk)::value;
      constexpr int NCH = decltype(nch)::value;
      auto run = [&](auto kern, int block) {
        const dim3 grid((unsigned)resident_grid((const void*)kern, a.rows, block));
        hipLaunchKernelGGL(kern, grid, dim3(block), 0, st, (const T*)logits, a);
        return check_launch("ce_fwd_kernel");
      };
      if (cfg.vec == 1) return run(ce_fwd_kernel<T, 1, 1, 1024, false>, 1024);
      // (choose_read_cfg keeps resident rows on 256 lanes, 8 vectors at most)
      constexpr bool kResident = NCH > 0 && BLOCK == 256 && NCH <= 8;
      if constexpr (!kResident) return run(ce_fwd_kernel<T, 16 / sizeof(T), 1, 1024, false>, 1024);
      else return run(ce_fwd_kernel<T, 16 / sizeof(T), NCH, 256, true>, 256);
    });
  });
}

int ce_rows_launch(void* dlogits, float* loss_rows, const void* logits, const int64_t* targets, int64_t rows,
                   int64_t V, int64_t ld_in, int64_t ld_out, int64_t ignore_index, int has_ignore, const int* n_valid,
                   int scale_by_n_valid, const float* row_scale, int dtype, hipStream_t st, const int* rows_lim,
                   int64_t rows_off, const int* rowmap, const int* n_live) {
  if (rows == 0) return HK_OK;
  const int es = esize(dtype);
  CeArgs a{};
  a.rows_lim = rows_lim;
  a.rows_off = rows_off;
  a.rowmap = rowmap;
  a.n_live = n_live;
  a.targets = targets;
  a.loss_rows = loss_rows;
  a.n_valid = n_valid;
  a.row_scale = row_scale;
  a.rows = rows;
  a.V = V;
  a.ld_in = ld_in;
  a.ld_out = ld_out;
  a.ignore_index = ignore_index;
  a.has_ignore = has_ignore;
  a.scale_by_n_valid = scale_by_n_valid;
  if (!dlogits) {  // loss rows only
    return ce_lse_launch(logits, a, dtype, st);
  }
  const int vec = 16 / es;
  const bool vec_ok = V % vec == 0 && aligned_to(logits, 16) && aligned_to(dlogits, 16) && (ld_in * es) % 16 == 0 &&
                      (ld_out * es) % 16 == 0;
  const RowCfg cfg = choose_row_cfg(V, es, vec_ok);
  return dispatch_t(dtype, [&](auto tt) {
    using T = typename decltype(tt)::type;
    return dispatch_cfg(cfg, [&](auto blk, auto nch) {
      constexpr int BLOCK = decltype(blk)::value;
      constexpr int NCH = decltype(nch)::value;
      auto run = [&](auto kern, int block) {
        // the 1024-lane forms (one block a CU) take two rounds (see resident_grid)
        const dim3 grid((unsigned)resident_grid((const void*)kern, rows, block, block == 1024 ? 2 : 1));
        hipLaunchKernelGGL(kern, grid, dim3(block), 0, st, (T*)dlogits, (const T*)logits, a);
        return check_launch("ce_fwd_grad_kernel");
      };
      if (cfg.vec == 1) return run(ce_fwd_grad_kernel<T, 1, 1, 1024, false>, 1024);
      if constexpr (NCH == 0) {
        return run(ce_fwd_grad_kernel<T, 16 / sizeof(T), 1, BLOCK, false>, BLOCK);
      } else {
        if (!form_fits(V, cfg)) return HK_EINVAL;
        return run(ce_fwd_grad_kernel<T, 16 / sizeof(T), NCH, BLOCK, true>, BLOCK);
      }
    });
  });
}

}  // namespace hk

using namespace hk;

extern "C" {

// [0, 256): the valid-row and live-row counts; then, when the workspace
// holds it, the launch plan's row list (4 bytes a row).
namespace {
size_t ce_plan_bytes(int64_t rows) { return rows < (1LL << 31) ? ((size_t)rows * 4 + 255) / 256 * 256 : 0; }
}  // namespace

size_t hk_cross_entropy_workspace_size(int64_t rows) {
  return 256 + ce_plan_bytes(rows > 0 ? rows : 0);
}

int hk_cross_entropy_fwd_grad(void* dlogits, float* loss_rows, float* loss_out, const void* logits,
                              const int64_t* targets, int64_t rows, int64_t V, int64_t ld_logits, int64_t ld_dlogits,
                              int64_t ignore_index, int reduction, int dtype, void* workspace, size_t workspace_bytes,
                              hk_stream_t stream) {
  HK_REQUIRE(valid_float_dtype(dtype), "invalid logits dtype code %d", dtype);
  HK_REQUIRE(rows >= 0 && V > 0, "invalid shape rows=%lld V=%lld", (long long)rows, (long long)V);
  HK_REQUIRE(ld_logits >= V && ld_dlogits >= V, "row stride smaller than V");
  HK_REQUIRE(V < (1LL << 31) - 4096, "V=%lld too large", (long long)V);
  HK_REQUIRE(reduction >= HK_REDUCTION_NONE && reduction <= HK_REDUCTION_SUM, "invalid reduction %d", reduction);
  HK_REQUIRE(workspace && workspace_bytes >= 256, "workspace must hold at least 256 bytes");
  HK_REQUIRE(rows == 0 || (dlogits && loss_rows && logits && targets), "null pointer argument");
  hipStream_t st = (hipStream_t)stream;
  int* n_valid = (int*)workspace;
  // ignore_index == -1 is the reference's "ignore nothing" sentinel (cross_entropy.py:197-198,219-225)
  const int has_ignore = ignore_index != -1;
  if (rows > 0) {
    // with room for the plan, the live rows are dealt out evenly over the
    // grid (a 256-byte workspace, the older minimum, still works: rows are
    // then strided over the grid whether they are live or not)
    const size_t plan = ce_plan_bytes(rows);
    const bool planned = plan > 0 && workspace_bytes >= 256 + plan;
    int* n_live = n_valid + 1;
    int* rowmap = planned ? (int*)((char*)workspace + 256) : nullptr;
    int rc = planned ? ce_plan_launch(n_valid, rowmap, n_live, targets, rows, V, ignore_index, has_ignore, st)
                     : count_valid_launch(n_valid, targets, rows, ignore_index, has_ignore, st);
    if (rc) return rc;
    rc = ce_rows_launch(dlogits, loss_rows, logits, targets, rows, V, ld_logits, ld_dlogits, ignore_index, has_ignore,
                        n_valid, reduction == HK_REDUCTION_MEAN, nullptr, dtype, st, nullptr, 0, rowmap,
                        planned ? n_live : nullptr);
    if (rc) return rc;
  }
  // the rows are already scaled by 1/max(n_valid, 1) for 'mean'
  if (loss_out) return sum_rows_launch(loss_out, loss_rows, rows, nullptr, 0, st);
  return HK_OK;
}

int hk_cross_entropy_fwd(float* lse_rows, float* loss_rows, float* loss_out, const void* logits,
                         const int64_t* targets, int64_t rows, int64_t V, int64_t ld_logits, int64_t ignore_index,
                         int reduction, int dtype, void* workspace, size_t workspace_bytes, hk_stream_t stream) {
  HK_REQUIRE(valid_float_dtype(dtype), "invalid logits dtype code %d", dtype);
  HK_REQUIRE(rows >= 0 && V > 0, "invalid shape rows=%lld V=%lld", (long long)rows, (long long)V);
  HK_REQUIRE(ld_logits >= V, "row stride smaller than V");
  HK_REQUIRE(V < (1LL << 31) - 4096, "V=%lld too large", (long long)V);
  HK_REQUIRE(reduction >= HK_REDUCTION_NONE && reduction <= HK_REDUCTION_SUM, "invalid reduction %d", reduction);
  HK_REQUIRE(workspace && workspace_bytes >= 256, "workspace must hold at least 256 bytes");
  HK_REQUIRE(rows == 0 || (lse_rows && loss_rows && logits && targets), "null pointer argument");
  hipStream_t st = (hipStream_t)stream;
  int* n_valid = (int*)workspace;
  const int has_ignore = ignore_index != -1;
  if (rows > 0) {
    int rc = count_valid_launch(n_valid, targets, rows, ignore_index, has_ignore, st);
    if (rc) return rc;
    CeArgs a{};
    a.targets = targets;
    a.loss_rows = loss_rows;
    a.lse_rows = lse_rows;
    a.rows = rows;
    a.V = V;
    a.ld_in = ld_logits;
    a.ignore_index = ignore_index;
    a.has_ignore = has_ignore;
    rc = ce_lse_launch(logits, a, dtype, st);
    if (rc) return rc;
  }
  if (loss_out)
    return sum_rows_launch(loss_out, loss_rows, rows, rows > 0 ? n_valid : nullptr,
                           rows > 0 && reduction == HK_REDUCTION_MEAN, st);
  return HK_OK;
}

int hk_scale_rows(void* out, const void* in, const float* g, const float* g_prev, int per_row, int skip_if_one,
                  int64_t rows, int64_t cols, int64_t ld_in, int64_t ld_out, int dtype, hk_stream_t stream) {
  HK_REQUIRE(valid_float_dtype(dtype), "invalid dtype code %d", dtype);
  HK_REQUIRE(rows >= 0 && cols >= 0, "invalid shape");
  HK_REQUIRE(ld_in >= cols && ld_out >= cols, "row stride smaller than cols");
  if (rows == 0 || cols == 0) return HK_OK;
  HK_REQUIRE(out && in && g, "null pointer argument");
  const int es = esize(dtype);
  const int vec = 16 / es;
  const bool vec_ok = cols % vec == 0 && aligned_to(in, 16) && aligned_to(out, 16) && (ld_in * es) % 16 == 0 &&
                      (ld_out * es) % 16 == 0;
  hipStream_t st = (hipStream_t)stream;
  return dispatch_t(dtype, [&](auto tt) {
    using T = typename decltype(tt)::type;
    const int64_t total = rows * (vec_ok ? cols / vec : cols);
    // grid-stride over one block per CU: a call that turns out to be a no-op
    // (g == 1, decided on the device) then costs one short launch, not 64K blocks
    const int dev = current_device();
    if (dev < 0) return (int)hipErrorNoDevice;
    const int64_t cap = (int64_t)cu_count(dev);
    const int64_t blocks = std::min<int64_t>(std::max<int64_t>(cdiv(total, 256 * 4), 1), cap);
    const dim3 grid((unsigned)blocks);
    if (vec_ok)
      hipLaunchKernelGGL((scale_rows_kernel<T, 16 / sizeof(T)>), grid, dim3(256), 0, st, (T*)out, (const T*)in, g,
                         g_prev, per_row, skip_if_one, rows, cols, ld_in, ld_out);
    else
      hipLaunchKernelGGL((scale_rows_kernel<T, 1>), grid, dim3(256), 0, st, (T*)out, (const T*)in, g, g_prev, per_row,
                         skip_if_one, rows, cols, ld_in, ld_out);
    return check_launch("scale_rows_kernel");
  });
}

int hk_selective_log_softmax(float* logp, const void* logits, const int64_t* ids, int64_t ids_sB, int64_t ids_sL,
                             const void* mask, int mask_dtype, int64_t mask_sB, int64_t mask_sL, int64_t B, int64_t L,
                             int64_t V, float temperature, int dtype, hk_stream_t stream) {
  HK_REQUIRE(valid_float_dtype(dtype), "invalid logits dtype code %d", dtype);
  HK_REQUIRE(B >= 0 && L >= 0 && V > 0, "invalid shape B=%lld L=%lld V=%lld", (long long)B, (long long)L,
             (long long)V);
  HK_REQUIRE(temperature > 0.f, "temperature must be positive");
  HK_REQUIRE(!mask || valid_mask_dtype(mask_dtype), "invalid mask dtype code %d", mask_dtype);
  HK_REQUIRE(V < (1LL << 31) - 4096, "V=%lld too large", (long long)V);
  if (B * L == 0) return HK_OK;
  HK_REQUIRE(logp && logits && ids, "null pointer argument");
  GrpoArgs a{};
  a.ids = ids;
  a.ids_sB = ids_sB;
  a.ids_sL = ids_sL;
  a.mask = mask;
  a.mask_dt = mask_dtype;
  a.mask_sB = mask_sB;
  a.mask_sL = mask_sL;
  a.B = B;
  a.L = L;
  a.V = V;
  a.inv_T = 1.f / temperature;
  a.logp_out = logp;
  const int es = esize(dtype);
  const bool vec_ok = V % (16 / es) == 0 && aligned_to(logits, 16);
  const RowCfg cfg = choose_read_cfg(V, es, vec_ok);
  hipStream_t st = (hipStream_t)stream;
  return dispatch_t(dtype, [&](auto tt) {
    using T = typename decltype(tt)::type;
    return dispatch_cfg(cfg, [&](auto blk, auto nch) {
      constexpr int BLOCK = decltype(blk)::value;
      constexpr int NCH = decltype(nch)::value;
      auto run = [&](auto kern, int block) {
        const dim3 grid((unsigned)resident_grid((const void*)kern, B * L, block, 2));
        hipLaunchKernelGGL(kern, grid, dim3(block), 0, st, (const T*)logits, a);
        return check_launch("selective_log_softmax_kernel");
      };
      if (cfg.vec == 1) return run(selective_log_softmax_kernel<T, 1, 1, 1024, false>, 1024);
      // (choose_read_cfg keeps resident rows on 256 lanes, 8 vectors at most)
      constexpr bool kResident = NCH > 0 && BLOCK == 256 && NCH <= 8;
      if constexpr (!kResident) {
        // rows of up to 8192 vectors stream on 512 lanes, four blocks a CU in
        // flight (6% faster at V 32000 bf16); longer rows on 1024 (3-4% faster
        // there than on 512)
        if (V / (16 / (int64_t)sizeof(T)) <= 8192)
          return run(selective_log_softmax_kernel<T, 16 / sizeof(T), 1, 512, false>, 512);
        return run(selective_log_softmax_kernel<T, 16 / sizeof(T), 1, 1024, false>, 1024);
      } else {
        return run(selective_log_softmax_kernel<T, 16 / sizeof(T), NCH, 256, true>, 256);
      }
    });
  });
}

size_t hk_grpo_workspace_size(int64_t B, int64_t L) {
  if (B < 0 || L < 0) return 0;
  return grpo_scratch_bytes(B, L);
}

int hk_grpo_loss_fwd(void* dlogits, float* loss_out, float* kl_out, float* clip_out, float* lse_rows,
                     float* loss_rows, float* kl_rows, float* clip_rows, const void* logits, const int64_t* ids,
                     int64_t ids_sB, int64_t ids_sL, const float* advantages, const float* old_logp, int64_t old_sB,
                     int64_t old_sL, const float* ref_logp, int64_t ref_sB, int64_t ref_sL, const void* mask,
                     int mask_dtype, int64_t mask_sB, int64_t mask_sL, int64_t B, int64_t L, int64_t V,
                     float temperature, float beta, float eps_low, float eps_high, int dtype, void* workspace,
                     size_t workspace_bytes, hk_stream_t stream) {
  HK_REQUIRE(valid_float_dtype(dtype), "invalid logits dtype code %d", dtype);
  const GrpoInputs in{ids,  ids_sB,    ids_sL,  advantages, old_logp, old_sB,      old_sL,  ref_logp,
                      ref_sB, ref_sL,  mask,    mask_dtype, mask_sB,  mask_sL,     B,       L,
                      V,    temperature, beta,  eps_low,    eps_high};
  if (const int rc = grpo_check(in)) return rc;
  HK_REQUIRE(workspace && workspace_bytes >= hk_grpo_workspace_size(B, L), "workspace too small");
  HK_REQUIRE(aligned_to(workspace, 16), "workspace must be 16-byte aligned");
  HK_REQUIRE(loss_out && clip_out && logits && (L == 0 || (lse_rows && loss_rows && kl_rows && clip_rows)),
             "null pointer argument");
  hipStream_t st = (hipStream_t)stream;
  int rc = grpo_prep_launch(in, workspace, st);
  if (rc) return rc;
  rc = grpo_rows_launch(dlogits, logits, 0, B * (L + 1), in, workspace, dtype, st);
  if (rc) return rc;
  return grpo_finalize_launch(in, workspace, loss_out, kl_out, clip_out, lse_rows, loss_rows, kl_rows, clip_rows, st);
}

}  // extern "C"
