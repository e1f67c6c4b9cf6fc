// Error state, version and device queries shared by every entry point.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "mi_common.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace mi {

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = '\0'; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MI_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return MI_OK;
}

int num_cus() {
  static std::mutex mu;
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Workgroup i of a launch runs on XCD (i mod n): probed once per device with
// a small kernel that records each workgroup's XCC_ID hardware register.
namespace {
__global__ void xcc_probe_kernel(int* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = int(__builtin_amdgcn_s_getreg((31 << 11) | 20) & 0xF);
}
}  // namespace

int xcd_round_robin(hipStream_t stream, bool probe) {
  static std::mutex mu;
  static int cached[64];
  static bool done[64] = {false};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  {
    std::lock_guard<std::mutex> lock(mu);
    if (done[dev]) return cached[dev];
  }
  if (!probe) return 0;
  // never inside a stream capture: the probe allocates and synchronises
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
    (void)hipGetLastError();
    return 0;
  }
  constexpr int kBlocks = 1024;
  int* d = nullptr;
  int result = 0;
  if (hipMalloc(&d, kBlocks * sizeof(int)) == hipSuccess) {
    int h[kBlocks];
    hipLaunchKernelGGL(xcc_probe_kernel, dim3(kBlocks), dim3(64), 0, stream, d);
    if (hipGetLastError() == hipSuccess &&
        hipMemcpyAsync(h, d, sizeof(h), hipMemcpyDeviceToHost, stream) == hipSuccess &&
        hipStreamSynchronize(stream) == hipSuccess) {
      int n = 0;
      for (int i = 0; i < kBlocks; ++i) n = h[i] + 1 > n ? h[i] + 1 : n;
      bool rr = n > 0;
      for (int i = 0; i < kBlocks && rr; ++i) rr = (h[i] == i % n);
      result = rr ? n : 0;
    }
    (void)hipFree(d);
  }
  (void)hipGetLastError();
  std::lock_guard<std::mutex> lock(mu);
  cached[dev] = result;
  done[dev] = true;
  return result;
}

}  // namespace mi

extern "C" const char* mi_last_error(void) { return g_last_error; }

extern "C" int mi_version(void) { return 200; }
