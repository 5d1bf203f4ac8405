// Error reporting and ABI identification for libkadconv_hip.so.
#include <stdarg.h>
#include <stdio.h>

#include "kad_common.h"

namespace kad {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(KAD_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return KAD_OK;
}

}  // namespace kad

extern "C" int kad_abi_version(void) { return KAD_ABI_VERSION; }
extern "C" const char* kad_last_error(void) { return kad::g_last_error; }
