// Error reporting and version entry points of the C ABI.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace {
thread_local char g_err[512] = "";
}

int skinny_set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int skinny_check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return skinny_set_error(SKINNY_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
  return SKINNY_OK;
}

extern "C" int skinny_abi_version(void) { return SKINNY_ABI_VERSION; }

extern "C" const char* skinny_last_error(void) { return g_err; }
