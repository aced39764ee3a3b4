// Rotary position embedding (rotate-half convention) for gfx950.
//
// For every row (b, h, t) of head_dim D and every i < D/2, with c, s the
// cos/sin of position t:
//   y[i]       = x[i] c - x[i + D/2] s
//   y[i + D/2] = x[i + D/2] c + x[i] s
// The backward is the same map with -s (kernels/rope.py:139-172); here the
// sign is a kernel argument, so no negated sin table is materialised.
//
// The kernel is stride-aware in the three row dimensions for both input and
// output, so the [B,T,H,D] storage behind a (B,H,T,D) transposed view needs
// no copy in either direction. q and k go through one launch. The host orders the three row dimensions by
// input stride, innermost smallest, so consecutive lanes walk memory in
// order; each lane rotates VEC pairs with two 16-byte loads and stores.
// Arithmetic is fp32 (cos/sin are read in their own dtype and widened).
#include "hk_common.h"
#include "../../include/hilda_kernel_amd.h"

#include <algorithm>
#include <type_traits>
#include <vector>

namespace hk {
namespace {

constexpr int kThreads = 256;

struct RopeGeom {
  uint32_t n1, n2;            // sizes of the middle and inner row dims
  int64_t is0, is1, is2;      // input strides (elements)
  int64_t os0, os1, os2;      // output strides
  int64_t cs0, cs1, cs2;      // cos/sin strides (0 where broadcast)
  uint32_t chunks;            // (D/2) / VEC
  int half;                   // D/2
};

// One work item: VEC rotate-half pairs of one row.
template <typename T, typename C, int VEC>
__device__ __forceinline__ void rope_item(T* __restrict__ out, const T* __restrict__ in, const C* __restrict__ cosp,
                                          const C* __restrict__ sinp, const RopeGeom& g, uint32_t idx, float sgn) {
  const uint32_t chunk = idx % g.chunks;
  uint32_t row = idx / g.chunks;
  const uint32_t i2 = row % g.n2;
  row /= g.n2;
  const uint32_t i1 = row % g.n1;
  const uint32_t i0 = row / g.n1;
  const int64_t e = (int64_t)chunk * VEC;
  const int64_t io = i0 * g.is0 + i1 * g.is1 + i2 * g.is2 + e;
  const int64_t oo = i0 * g.os0 + i1 * g.os1 + i2 * g.os2 + e;
  const int64_t co = i0 * g.cs0 + i1 * g.cs1 + i2 * g.cs2 + e;

  Pack<T, VEC> p1 = load_pack<T, VEC>(in + io);
  Pack<T, VEC> p2 = load_pack<T, VEC>(in + io + g.half);
  Pack<C, VEC> pc = load_pack<C, VEC>(cosp + co);
  Pack<C, VEC> ps = load_pack<C, VEC>(sinp + co);
  float x1[VEC], x2[VEC], c[VEC], s[VEC];
  unpack(p1, x1);
  unpack(p2, x2);
  unpack(pc, c);
  unpack(ps, s);
  float y1[VEC], y2[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    const float si = sgn * s[i];
    y1[i] = x1[i] * c[i] - x2[i] * si;
    y2[i] = x2[i] * c[i] + x1[i] * si;
  }
  store_pack<T, VEC>(out + oo, pack<T, VEC>(y1));
  store_pack<T, VEC>(out + oo + g.half, pack<T, VEC>(y2));
}

template <typename T, typename C>
struct RopeSeg {
  T* out;
  const T* in;
  const C* cos;
  const C* sin;
  RopeGeom g;
  uint32_t total;  // work items
};

// Work items [0, a.total) rotate tensor a, the rest tensor b: q and k in one
// launch (a lone 34 MB k launch spends half its time ramping up and draining).
template <typename T, typename C, int VEC>
__global__ __launch_bounds__(kThreads) void rope_kernel(RopeSeg<T, C> a, RopeSeg<T, C> b, float sgn) {
  const uint32_t idx = blockIdx.x * kThreads + threadIdx.x;
  if (idx < a.total) rope_item<T, C, VEC>(a.out, a.in, a.cos, a.sin, a.g, idx, sgn);
  else if (idx - a.total < b.total) rope_item<T, C, VEC>(b.out, b.in, b.cos, b.sin, b.g, idx - a.total, sgn);
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

bool div_ok(int64_t v, int vec) { return v % vec == 0; }

// One tensor's rotation, split along its outermost row dimension into pieces
// of fewer than 2^31 work items.
struct RopePlan {
  int64_t n0, outer_step;
  int64_t is0, os0, cs0;
  RopeGeom g;
  int64_t per_outer;
};

int plan_rope(int64_t B, int64_t H, int64_t T, int64_t D, int64_t in_sB, int64_t in_sH, int64_t in_sT,
              int64_t out_sB, int64_t out_sH, int64_t out_sT, int64_t cos_B, int64_t cos_sB, int64_t cos_sT, int vec,
              RopePlan* p, bool* vec_ok) {
  HK_REQUIRE(B >= 0 && H >= 0 && T >= 0 && D > 0, "invalid shape B=%lld H=%lld T=%lld D=%lld", (long long)B,
             (long long)H, (long long)T, (long long)D);
  HK_REQUIRE(D % 2 == 0, "head_dim D=%lld must be even", (long long)D);
  HK_REQUIRE(cos_B == 1 || cos_B == B, "cos/sin batch dim %lld must be 1 or B=%lld", (long long)cos_B,
             (long long)B);
  HK_REQUIRE(in_sB >= 0 && in_sH >= 0 && in_sT >= 0 && out_sB >= 0 && out_sH >= 0 && out_sT >= 0 && cos_sB >= 0 &&
                 cos_sT >= 0,
             "negative strides are not supported");
  // order the row dims by input stride, innermost (smallest) last
  struct Dim { int64_t n, is, os, cs; };
  Dim d[3] = {{B, in_sB, out_sB, cos_B == 1 ? 0 : cos_sB}, {H, in_sH, out_sH, 0}, {T, in_sT, out_sT, cos_sT}};
  std::stable_sort(d, d + 3, [](const Dim& a, const Dim& b) { return a.is > b.is; });
  const int64_t half = D / 2;
  bool ok = div_ok(half, vec);
  for (auto& x : d) ok = ok && div_ok(x.is, vec) && div_ok(x.os, vec) && div_ok(x.cs, vec);
  *vec_ok = ok;
  const int v = ok ? vec : 1;
  p->g.n1 = (uint32_t)d[1].n;
  p->g.n2 = (uint32_t)d[2].n;
  p->g.is0 = d[0].is; p->g.is1 = d[1].is; p->g.is2 = d[2].is;
  p->g.os0 = d[0].os; p->g.os1 = d[1].os; p->g.os2 = d[2].os;
  p->g.cs0 = d[0].cs; p->g.cs1 = d[1].cs; p->g.cs2 = d[2].cs;
  p->g.chunks = (uint32_t)(half / v);
  p->g.half = (int)half;
  p->n0 = d[0].n;
  p->is0 = d[0].is; p->os0 = d[0].os; p->cs0 = d[0].cs;
  HK_REQUIRE((int64_t)d[1].n * d[2].n * p->g.chunks < (1LL << 31), "inner row dims too large");
  p->per_outer = (int64_t)d[1].n * d[2].n * p->g.chunks;
  p->outer_step = p->per_outer > 0 ? std::max<int64_t>(1, ((1LL << 31) - 1) / p->per_outer) : 1;
  return HK_OK;
}

// Rotate one or two tensors; pieces of the two are paired into launches.
template <typename TX, typename TC, int VEC>
int run_rope(void* const* outs, const void* const* ins, const void* cos, const void* sin, const RopePlan* plans,
             int n, float sgn, hipStream_t st) {
  std::vector<RopeSeg<TX, TC>> segs;
  for (int t = 0; t < n; ++t) {
    const RopePlan& p = plans[t];
    if (p.per_outer == 0) continue;
    for (int64_t o = 0; o < p.n0; o += p.outer_step) {
      const int64_t no = std::min(p.outer_step, p.n0 - o);
      RopeSeg<TX, TC> sg;
      sg.out = (TX*)outs[t] + o * p.os0;
      sg.in = (const TX*)ins[t] + o * p.is0;
      sg.cos = (const TC*)cos + o * p.cs0;
      sg.sin = (const TC*)sin + o * p.cs0;
      sg.g = p.g;
      sg.total = (uint32_t)(no * p.per_outer);
      segs.push_back(sg);
    }
  }
  for (size_t i = 0; i < segs.size();) {
    RopeSeg<TX, TC> a = segs[i++];
    RopeSeg<TX, TC> b = a;
    b.total = 0;
    if (i < segs.size() && (uint64_t)a.total + segs[i].total < (1ULL << 31)) b = segs[i++];
    const uint64_t total = (uint64_t)a.total + b.total;
    hipLaunchKernelGGL((rope_kernel<TX, TC, VEC>), dim3((unsigned)cdiv((int64_t)total, (int64_t)kThreads)),
                       dim3(kThreads), 0, st, a, b, sgn);
    int rc = check_launch("rope_kernel");
    if (rc) return rc;
  }
  return HK_OK;
}

int rope_impl(void* const* outs, const void* const* ins, const int64_t* H, const int64_t (*in_s)[3],
              const int64_t (*out_s)[3], int n, const void* cos, const void* sin, int64_t B, int64_t T, int64_t D,
              int64_t cos_B, int64_t cos_sB, int64_t cos_sT, int dtype_x, int dtype_cs, int inverse,
              hk_stream_t stream) {
  HK_REQUIRE(dtype_cs == kF32 || dtype_cs == kF16 || dtype_cs == kBF16, "invalid cos/sin dtype %d", dtype_cs);
  return dispatch_t(dtype_x, [&](auto tx) {
    using TX = typename decltype(tx)::type;
    return dispatch_t(dtype_cs, [&](auto tc) {
      using TC = typename decltype(tc)::type;
      constexpr int V = 16 / sizeof(TX);
      RopePlan plans[2];
      bool vec = aligned_to(cos, sizeof(TC) * V) && aligned_to(sin, sizeof(TC) * V);
      bool any = false;
      for (int t = 0; t < n; ++t) {
        bool vt = false;
        int rc = plan_rope(B, H[t], T, D, in_s[t][0], in_s[t][1], in_s[t][2], out_s[t][0], out_s[t][1], out_s[t][2],
                           cos_B, cos_sB, cos_sT, V, &plans[t], &vt);
        if (rc) return rc;
        if (plans[t].per_outer == 0) continue;
        HK_REQUIRE(outs[t] && ins[t], "null pointer argument");
        any = true;
        vec = vec && vt && aligned_to(ins[t], 16) && aligned_to(outs[t], 16);
      }
      if (!any) return HK_OK;
      HK_REQUIRE(cos && sin, "null pointer argument");
      const float sgn = inverse ? -1.f : 1.f;
      if (vec) return run_rope<TX, TC, V>(outs, ins, cos, sin, plans, n, sgn, (hipStream_t)stream);
      // scalar path: plan again with one element per work item
      for (int t = 0; t < n; ++t) {
        bool vt;
        plan_rope(B, H[t], T, D, in_s[t][0], in_s[t][1], in_s[t][2], out_s[t][0], out_s[t][1], out_s[t][2], cos_B,
                  cos_sB, cos_sT, 1, &plans[t], &vt);
      }
      return run_rope<TX, TC, 1>(outs, ins, cos, sin, plans, n, sgn, (hipStream_t)stream);
    });
  });
}

}  // namespace
}  // namespace hk

using namespace hk;

extern "C" {

int hk_rope(void* out, const void* in, const void* cos, const void* sin, int64_t B, int64_t H, int64_t T, int64_t D,
            int64_t in_sB, int64_t in_sH, int64_t in_sT, int64_t out_sB, int64_t out_sH, int64_t out_sT,
            int64_t cos_B, int64_t cos_sB, int64_t cos_sT, int dtype_x, int dtype_cs, int inverse,
            hk_stream_t stream) {
  void* outs[1] = {out};
  const void* ins[1] = {in};
  const int64_t h[1] = {H};
  const int64_t is[1][3] = {{in_sB, in_sH, in_sT}};
  const int64_t os[1][3] = {{out_sB, out_sH, out_sT}};
  return rope_impl(outs, ins, h, is, os, 1, cos, sin, B, T, D, cos_B, cos_sB, cos_sT, dtype_x, dtype_cs, inverse,
                   stream);
}

int hk_rope_qk(void* q_out, const void* q_in, int64_t Hq, int64_t q_in_sB, int64_t q_in_sH, int64_t q_in_sT,
               int64_t q_out_sB, int64_t q_out_sH, int64_t q_out_sT, void* k_out, const void* k_in, int64_t Hk,
               int64_t k_in_sB, int64_t k_in_sH, int64_t k_in_sT, int64_t k_out_sB, int64_t k_out_sH,
               int64_t k_out_sT, const void* cos, const void* sin, int64_t B, int64_t T, int64_t D, int64_t cos_B,
               int64_t cos_sB, int64_t cos_sT, int dtype_x, int dtype_cs, int inverse, hk_stream_t stream) {
  void* outs[2] = {q_out, k_out};
  const void* ins[2] = {q_in, k_in};
  const int64_t h[2] = {Hq, Hk};
  const int64_t is[2][3] = {{q_in_sB, q_in_sH, q_in_sT}, {k_in_sB, k_in_sH, k_in_sT}};
  const int64_t os[2][3] = {{q_out_sB, q_out_sH, q_out_sT}, {k_out_sB, k_out_sH, k_out_sT}};
  return rope_impl(outs, ins, h, is, os, 2, cos, sin, B, T, D, cos_B, cos_sB, cos_sT, dtype_x, dtype_cs, inverse,
                   stream);
}

}  // extern "C"
