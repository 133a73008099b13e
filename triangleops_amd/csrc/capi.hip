// Error reporting and device queries for the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "capi.hpp"

namespace {
thread_local char g_err[512] = "";
}

namespace tops {

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int num_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

}  // namespace tops

extern "C" const char* tops_last_error(void) { return g_err; }

extern "C" int tops_abi_version(void) { return 1; }
