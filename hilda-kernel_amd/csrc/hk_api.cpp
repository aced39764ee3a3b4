// Host-side support for the C ABI: thread-local error text, per-device
// property cache, ABI version. No device memory is allocated here.
#include "hk_common.h"
#include "../../include/hilda_kernel_amd.h"

#include <mutex>
#include <stdarg.h>
#include <stdio.h>

namespace hk {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

namespace {
constexpr int kMaxDevices = 64;
std::once_flag g_cu_once[kMaxDevices];
int g_cu_count[kMaxDevices];
}  // namespace

int cu_count(int device) {
  if (device < 0 || device >= kMaxDevices) return 0;
  std::call_once(g_cu_once[device], [device] {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) n = 0;
    g_cu_count[device] = n;
  });
  return g_cu_count[device];
}

int blocks_per_cu(const void* kernel, int block) {
  // a handful of kernels ask; a linear table under one lock is enough
  constexpr int kSlots = 256;
  static std::mutex mu;
  static const void* keys[kSlots];
  static int vals[kSlots];
  static int used = 0;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < used; ++i)
    if (keys[i] == kernel) return vals[i];
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, block, 0) != hipSuccess || n < 1) {
    (void)hipGetLastError();  // not a launch failure: fall back to one block a CU
    n = 1;
  }
  if (used < kSlots) {
    keys[used] = kernel;
    vals[used] = n;
    ++used;
  }
  return n;
}

int current_device() {
  int d = -1;
  hipError_t e = hipGetDevice(&d);
  if (e != hipSuccess) {
    set_error("hipGetDevice failed: %s", hipGetErrorString(e));
    return -1;
  }
  return d;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("launch of %s failed: %s", what, hipGetErrorString(e));
    return (int)e;
  }
  return HK_OK;
}

hipStream_t side_stream(int device) {
  // per host thread: a stream another thread is capturing into is never handed out
  thread_local hipStream_t streams[kMaxDevices] = {};
  if (device < 0 || device >= kMaxDevices) {
    set_error("device %d out of range for the side-stream table", device);
    return nullptr;
  }
  if (!streams[device]) {
    hipStream_t s = nullptr;
    const hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) {
      set_error("hipStreamCreateWithFlags failed: %s", hipGetErrorString(e));
      return nullptr;
    }
    streams[device] = s;
  }
  return streams[device];
}

int stream_after(hipStream_t to, hipStream_t from) {
  hipEvent_t ev = nullptr;
  HK_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
  hipError_t e = hipEventRecord(ev, from);
  if (e == hipSuccess) e = hipStreamWaitEvent(to, ev, 0);
  // (released by the runtime once the recorded work has completed)
  const hipError_t d = hipEventDestroy(ev);
  if (e == hipSuccess) e = d;
  if (e != hipSuccess) {
    set_error("stream fork/join failed: %s", hipGetErrorString(e));
    return (int)e;
  }
  return HK_OK;
}

}  // namespace hk

extern "C" {

int hk_abi_version(void) { return HK_ABI_VERSION; }

const char* hk_last_error(void) { return hk::g_last_error; }

int hk_device_cu_count(int device) {
  int n = hk::cu_count(device);
  if (n <= 0) {
    hk::set_error("could not read the CU count of device %d", device);
    return HK_EINVAL;
  }
  return n;
}

}  // extern "C"
