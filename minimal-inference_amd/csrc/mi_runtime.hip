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

}  // namespace mi

extern "C" const char* mi_last_error(void) { return g_last_error; }

extern "C" int mi_version(void) { return 200; }
