// Streaming device copies that bound what an HBM-bound op can reach. They are
// measurement references for the benchmark (an op's bytes against a copy of
// the same bytes, moved by the best access order found and by the access order
// of the register-resident row kernels); nothing in the operator path calls
// them.
//
// HK_COPY_FLAT: grid-stride over 16-byte vectors, four loads in flight per
//   lane before their four stores, one 256-lane block per CU: at any moment
//   the whole GPU sweeps one contiguous window of a few MiB, which keeps the
//   HBM pages it opens few and full.
// HK_COPY_ROWS: one 1024-lane block per CU and per row of `row_bytes`, the
//   row held in registers (up to 24 16-byte vectors a lane), its stores
//   issued with the loads of the block's next row (rows strided by the grid):
//   the order of the CrossEntropy / GRPO gradient kernels, without their
//   arithmetic.
// hk_stream_mix: an op's byte mix without its arithmetic: n_read streams read
//   and n_write streams written, all of one length, in the flat order, two
//   256-lane blocks a CU, one 16-byte vector of every stream in flight per
//   lane (the best launch shape measured for 2-9 read streams). An op that
//   reads three rows and writes one (the fused-add norm backward) is compared
//   with 3 reads + 1 write here, which HBM serves faster than a copy of the
//   same bytes; one with 8 + 1 (the AttnRes forward), slower.
#include "hk_common.h"
#include "../../include/hilda_kernel_amd.h"

namespace hk {
namespace {

template <int U>
__global__ __launch_bounds__(256) void copy_flat_kernel(u32x4* __restrict__ d, const u32x4* __restrict__ s,
                                                        int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + (U - 1) * stride < n; i += U * stride) {
    u32x4 r[U];
#pragma unroll
    for (int u = 0; u < U; ++u) r[u] = s[i + u * stride];
#pragma unroll
    for (int u = 0; u < U; ++u) d[i + u * stride] = r[u];
  }
  for (; i < n; i += stride) d[i] = s[i];
}

template <int NCH>
__global__ __launch_bounds__(1024) void copy_rows_kernel(u32x4* d, const u32x4* s, int64_t rows, int cols) {
  int64_t row = blockIdx.x;
  if (row >= rows) return;
  u32x4 v[NCH];
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = j * 1024 + (int)threadIdx.x;
    if (c < cols) v[j] = s[row * cols + c];
  }
  for (;;) {
    const int64_t next = row + gridDim.x;
    const u32x4* src = s + (next < rows ? next : row) * cols;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int c = j * 1024 + (int)threadIdx.x;
      if (c < cols) {
        __builtin_nontemporal_store(v[j], d + row * cols + c);
        v[j] = src[c];
      }
    }
    if (next >= rows) break;
    row = next;
  }
}

constexpr int kMixMaxRead = 9, kMixMaxWrite = 8;

// d[w][i] = (xor over k < n_read of s[k][i]) + w for every vector i of n, the
// streams `stride` vectors apart.
__global__ __launch_bounds__(256) void mix_kernel(u32x4* __restrict__ d, const u32x4* __restrict__ s, int64_t n,
                                                  int64_t stride_v, int n_read, int n_write) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    u32x4 r[kMixMaxRead];
#pragma unroll
    for (int k = 0; k < kMixMaxRead; ++k)
      if (k < n_read) r[k] = s[k * stride_v + i];
    u32x4 a = r[0];
#pragma unroll
    for (int k = 1; k < kMixMaxRead; ++k)
      if (k < n_read) a ^= r[k];
#pragma unroll
    for (int w = 0; w < kMixMaxWrite; ++w)
      if (w < n_write) __builtin_nontemporal_store(a + (uint32_t)w, d + w * stride_v + i);
  }
}

}  // namespace
}  // namespace hk

using namespace hk;

extern "C" int hk_stream_copy(void* dst, const void* src, int64_t rows, int64_t row_bytes, int mode,
                              hk_stream_t stream) {
  HK_REQUIRE(mode == HK_COPY_FLAT || mode == HK_COPY_ROWS, "invalid copy mode %d", mode);
  HK_REQUIRE(rows >= 0 && row_bytes >= 0 && row_bytes % 16 == 0, "rows=%lld row_bytes=%lld: rows of whole 16-byte "
             "vectors", (long long)rows, (long long)row_bytes);
  HK_REQUIRE(mode == HK_COPY_FLAT || row_bytes <= 24 * 1024 * 16,
             "HK_COPY_ROWS holds rows of at most %d bytes", 24 * 1024 * 16);
  if (rows == 0 || row_bytes == 0) return HK_OK;
  HK_REQUIRE(dst && src && aligned_to(dst, 16) && aligned_to(src, 16), "16-byte aligned pointers required");
  hipStream_t st = (hipStream_t)stream;
  u32x4* d = (u32x4*)dst;
  const u32x4* s = (const u32x4*)src;
  const int dev = current_device();
  const int cu = dev >= 0 && cu_count(dev) > 0 ? cu_count(dev) : 256;
  if (mode == HK_COPY_FLAT) {
    hipLaunchKernelGGL(copy_flat_kernel<4>, dim3((unsigned)cu), dim3(256), 0, st, d, s, rows * (row_bytes / 16));
    return check_launch("copy_flat_kernel");
  }
  const int cols = (int)(row_bytes / 16);
  const dim3 grid((unsigned)(rows < cu ? rows : cu));
  if (cols <= 16 * 1024)
    hipLaunchKernelGGL(copy_rows_kernel<16>, grid, dim3(1024), 0, st, d, s, rows, cols);
  else if (cols <= 20 * 1024)
    hipLaunchKernelGGL(copy_rows_kernel<20>, grid, dim3(1024), 0, st, d, s, rows, cols);
  else
    hipLaunchKernelGGL(copy_rows_kernel<24>, grid, dim3(1024), 0, st, d, s, rows, cols);
  return check_launch("copy_rows_kernel");
}

extern "C" int hk_stream_mix(void* dst, const void* src, int64_t bytes, int64_t stride, int n_read, int n_write,
                             hk_stream_t stream) {
  HK_REQUIRE(n_read >= 1 && n_read <= kMixMaxRead && n_write >= 1 && n_write <= kMixMaxWrite,
             "n_read=%d n_write=%d: 1..%d streams read, 1..%d written", n_read, n_write, kMixMaxRead, kMixMaxWrite);
  HK_REQUIRE(bytes >= 0 && bytes % 16 == 0, "bytes=%lld: whole 16-byte vectors per stream", (long long)bytes);
  HK_REQUIRE(stride >= bytes && stride % 16 == 0, "stride=%lld: at least bytes=%lld, a multiple of 16",
             (long long)stride, (long long)bytes);
  if (bytes == 0) return HK_OK;
  HK_REQUIRE(dst && src && aligned_to(dst, 16) && aligned_to(src, 16), "16-byte aligned pointers required");
  const int dev = current_device();
  const int cu = dev >= 0 && cu_count(dev) > 0 ? cu_count(dev) : 256;
  hipLaunchKernelGGL(mix_kernel, dim3((unsigned)(2 * cu)), dim3(256), 0, (hipStream_t)stream, (u32x4*)dst,
                     (const u32x4*)src, bytes / 16, stride / 16, n_read, n_write);
  return check_launch("mix_kernel");
}
