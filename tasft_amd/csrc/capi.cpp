// Error channel and version query of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include <hip/hip_runtime.h>

#include "common.h"

namespace tasft {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return set_error(kErrLaunch, "%s: launch failed: %s", what, hipGetErrorString(err));
  return kOk;
}

}  // namespace tasft

extern "C" const char* tasft_last_error(void) { return tasft::g_last_error; }

extern "C" int tasft_abi_version(void) { return 9; }
