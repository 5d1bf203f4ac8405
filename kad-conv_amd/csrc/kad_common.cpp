// Error reporting and ABI identification for libkadconv_hip.so.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "kad_common.h"

namespace kad {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  // format into a scratch buffer first: callers may pass the previous message as an argument
  char buf[sizeof(g_last_error)];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  memcpy(g_last_error, buf, sizeof(buf));
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
