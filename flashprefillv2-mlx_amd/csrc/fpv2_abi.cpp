// Host-side ABI glue: version, thread-local error string, launch checks.
#include <stdarg.h>
#include <stdio.h>

#include "fpv2_common.h"

namespace fpv2 {

namespace {
thread_local char g_error[512] = "";
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return status;
}

int check_launch(const char* kernel) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(FPV2_ERR_LAUNCH, "%s: launch failed: %s", kernel, hipGetErrorString(e));
  g_error[0] = '\0';
  return FPV2_OK;
}

}  // namespace fpv2

extern "C" int fpv2_abi_version(void) { return FPV2_ABI_VERSION; }

extern "C" const char* fpv2_last_error(void) { return fpv2::g_error; }
