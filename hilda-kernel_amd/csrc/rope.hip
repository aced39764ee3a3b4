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
// no copy in either direction. The host orders the three row dimensions by
// input stride, innermost smallest, so consecutive lanes walk memory in
// order; each lane rotates VEC pairs with two 16-byte loads and stores.
// Arithmetic is fp32 (cos/sin are read in their own dtype and widened).
#include "hk_common.h"
#include "../../include/hilda_kernel_amd.h"

#include <algorithm>
#include <type_traits>

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

template <typename T, typename C, int VEC>
__global__ __launch_bounds__(kThreads) void rope_kernel(T* __restrict__ out, const T* __restrict__ in,
                                                        const C* __restrict__ cosp, const C* __restrict__ sinp,
                                                        RopeGeom g, uint32_t total, float sgn) {
  const uint32_t idx = blockIdx.x * kThreads + threadIdx.x;
  if (idx >= total) return;
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

}  // namespace
}  // namespace hk

using namespace hk;

extern "C" {

int hk_rope(void* out, const void* in, const void* cos, const void* sin, int64_t B, int64_t H, int64_t T, int64_t D,
            int64_t in_sB, int64_t in_sH, int64_t in_sT, int64_t out_sB, int64_t out_sH, int64_t out_sT,
            int64_t cos_B, int64_t cos_sB, int64_t cos_sT, int dtype_x, int dtype_cs, int inverse,
            hk_stream_t stream) {
  HK_REQUIRE(B >= 0 && H >= 0 && T >= 0 && D > 0, "invalid shape B=%lld H=%lld T=%lld D=%lld", (long long)B,
             (long long)H, (long long)T, (long long)D);
  HK_REQUIRE(D % 2 == 0, "head_dim D=%lld must be even", (long long)D);
  HK_REQUIRE(cos_B == 1 || cos_B == B, "cos/sin batch dim %lld must be 1 or B=%lld", (long long)cos_B,
             (long long)B);
  HK_REQUIRE(in_sB >= 0 && in_sH >= 0 && in_sT >= 0 && out_sB >= 0 && out_sH >= 0 && out_sT >= 0 && cos_sB >= 0 &&
                 cos_sT >= 0,
             "negative strides are not supported");
  const int64_t rows = B * H * T;
  if (rows == 0) return HK_OK;
  HK_REQUIRE(out && in && cos && sin, "null pointer argument");
  HK_REQUIRE(dtype_cs == kF32 || dtype_cs == kF16 || dtype_cs == kBF16, "invalid cos/sin dtype %d", dtype_cs);

  // order the row dims by input stride, innermost (smallest) last
  struct Dim { int64_t n, is, os, cs; };
  Dim d[3] = {{B, in_sB, out_sB, cos_B == 1 ? 0 : cos_sB}, {H, in_sH, out_sH, 0}, {T, in_sT, out_sT, cos_sT}};
  std::stable_sort(d, d + 3, [](const Dim& a, const Dim& b) { return a.is > b.is; });

  const int64_t half = D / 2;
  return dispatch_t(dtype_x, [&](auto tx) {
    using TX = typename decltype(tx)::type;
    return dispatch_t(dtype_cs, [&](auto tc) {
      using TC = typename decltype(tc)::type;
      constexpr int V = 16 / sizeof(TX);
      bool vec = div_ok(half, V) && aligned_to(in, 16) && aligned_to(out, 16) && aligned_to(cos, sizeof(TC) * V) &&
                 aligned_to(sin, sizeof(TC) * V);
      for (auto& x : d) vec = vec && div_ok(x.is, V) && div_ok(x.os, V) && div_ok(x.cs, V);
      auto run = [&](auto vec_c) {
        constexpr int VEC = decltype(vec_c)::value;
        RopeGeom g;
        g.n1 = (uint32_t)d[1].n;
        g.n2 = (uint32_t)d[2].n;
        g.is0 = d[0].is; g.is1 = d[1].is; g.is2 = d[2].is;
        g.os0 = d[0].os; g.os1 = d[1].os; g.os2 = d[2].os;
        g.cs0 = d[0].cs; g.cs1 = d[1].cs; g.cs2 = d[2].cs;
        g.chunks = (uint32_t)(half / VEC);
        g.half = (int)half;
        HK_REQUIRE((int64_t)d[1].n * d[2].n * g.chunks < (1LL << 31), "inner row dims too large");
        // split the outer dim so each launch indexes fewer than 2^31 work items
        const int64_t per_outer = (int64_t)d[1].n * d[2].n * g.chunks;
        const int64_t outer_step = std::max<int64_t>(1, ((1LL << 31) - 1) / per_outer);
        const float sgn = inverse ? -1.f : 1.f;
        for (int64_t o = 0; o < d[0].n; o += outer_step) {
          const int64_t no = std::min(outer_step, d[0].n - o);
          const uint32_t total = (uint32_t)(no * per_outer);
          hipLaunchKernelGGL((rope_kernel<TX, TC, VEC>), dim3((unsigned)cdiv(total, kThreads)), dim3(kThreads), 0,
                             (hipStream_t)stream, (TX*)out + o * d[0].os, (const TX*)in + o * d[0].is,
                             (const TC*)cos + o * d[0].cs, (const TC*)sin + o * d[0].cs, g, total, sgn);
          int rc = check_launch("rope_kernel");
          if (rc) return rc;
        }
        return HK_OK;
      };
      if (vec) return run(std::integral_constant<int, V>{});
      return run(std::integral_constant<int, 1>{});
    });
  });
}

}  // extern "C"
