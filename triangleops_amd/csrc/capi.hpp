// Host-side helpers shared by the C-ABI entry points: per-thread error text, argument
// checks and launch-error capture.  No entry point allocates device memory.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/triangleops_amd.h"

namespace tops {

// Records a printf-style message for tops_last_error() on this thread; returns `code`.
int fail(int code, const char* fmt, ...);

// Compute units of the current device (queried once per device).
int num_cus();

// Converts the launch status into a return code.
inline int launched(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TOPS_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return TOPS_OK;
}

}  // namespace tops

#define TOPS_REQUIRE(cond, ...)                              \
  do {                                                       \
    if (!(cond)) return ::tops::fail(TOPS_EINVAL, __VA_ARGS__); \
  } while (0)
