// Column sums of fp32 partial rows: out[c] = sum over g < groups of
// part[g * ld + c], added in fp64 in a fixed order and rounded once. The
// norm and AttnRes backwards write one partial row of dW per workgroup and
// finish with this pass.
//
// A 256-lane block covers 32 columns (one 128-byte line of every partial
// row) with 8 lanes of 16-byte vectors, and 32 slices of the groups
// (g = slice, slice + 32, ...). Each lane issues kU loads before it adds them,
// so the 512 partial rows of a 2-blocks-a-CU launch take two memory round
// trips; the slices then meet in LDS. The 64-column form with scalar loads,
// four in flight, took eight round trips and a third longer.
#pragma once
#include "hk_common.h"

namespace hk {

constexpr int kColsumCols = 32;   // columns per block: 8 lanes of 4
constexpr int kColsumLanes = 256; // 32 slices of 8 lanes

// Columns c < split go to out0[c], the rest to out1[c - split].
template <typename W, bool VEC4, int kU = 8>
__global__ __launch_bounds__(kColsumLanes) void colsum_kernel(W* __restrict__ out0, W* __restrict__ out1,
                                                              const float* __restrict__ part, int64_t groups,
                                                              int64_t cols, int64_t ld, int64_t split) {
  constexpr int kLanesPerLine = kColsumCols / 4;              // 8
  constexpr int kNSlice = kColsumLanes / kLanesPerLine;       // 32
  __shared__ double red[kNSlice][kColsumCols + 1];
  const int q = threadIdx.x % kLanesPerLine, s = threadIdx.x / kLanesPerLine;
  const int64_t c0 = (int64_t)blockIdx.x * kColsumCols + q * 4;
  double acc[4] = {0.0, 0.0, 0.0, 0.0};
  for (int64_t g = s; g < groups; g += (int64_t)kNSlice * kU) {
    float v[kU][4];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t gg = g + (int64_t)u * kNSlice;
      const float* p = part + gg * ld + c0;
      if constexpr (VEC4) {
        const u32x4 r = gg < groups && c0 < cols ? *reinterpret_cast<const u32x4*>(p) : u32x4{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) v[u][i] = bits_f32(r[i]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[u][i] = gg < groups && c0 + i < cols ? p[i] : 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] += (double)v[u][i];
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) red[s][q * 4 + i] = acc[i];
  __syncthreads();
  if ((int)threadIdx.x < kColsumCols) {
    const int64_t c = (int64_t)blockIdx.x * kColsumCols + threadIdx.x;
    if (c < cols) {
      double t = 0.0;
#pragma unroll 8
      for (int i = 0; i < kNSlice; ++i) t += red[i][threadIdx.x];
      if (c < split) out0[c] = from_f32<W>((float)t);
      else out1[c - split] = from_f32<W>((float)t);
    }
  }
}

// Launch colsum_kernel on `stream`; the 16-byte form when every partial row
// starts on a 16-byte boundary.
template <typename W>
inline void colsum_launch(W* out0, W* out1, const float* part, int64_t groups, int64_t cols, int64_t ld,
                          int64_t split, hipStream_t stream) {
  const dim3 grid((unsigned)((cols + kColsumCols - 1) / kColsumCols));
  const bool vec4 = cols % 4 == 0 && ld % 4 == 0 && (reinterpret_cast<uintptr_t>(part) % 16) == 0;
  if (vec4)
    hipLaunchKernelGGL((colsum_kernel<W, true>), grid, dim3(kColsumLanes), 0, stream, out0, out1, part, groups, cols,
                       ld, split);
  else
    hipLaunchKernelGGL((colsum_kernel<W, false>), grid, dim3(kColsumLanes), 0, stream, out0, out1, part, groups,
                       cols, ld, split);
}

}  // namespace hk
