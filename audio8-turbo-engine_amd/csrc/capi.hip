// Library identification and error reporting of the C ABI (include/a8attn.h).
#include <dlfcn.h>
#include <stdarg.h>
#include <stdio.h>

#include "a8_common.h"

namespace a8 {

static thread_local char g_err[512];

int set_error(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

}  // namespace a8

#ifndef A8_SRC_HASH
#define A8_SRC_HASH "unknown"
#endif
// "a8attn <version> gfx950 src:<hash of the sources it was built from>"
extern "C" const char *a8_version(void) { return "a8attn 0.2.0 gfx950 src:" A8_SRC_HASH; }

extern "C" const char *a8_last_error(void) { return a8::g_err; }

extern "C" const char *a8_hip_runtime_path(void) {
  Dl_info info;
  if (dladdr(reinterpret_cast<void *>(&hipLaunchKernel), &info) && info.dli_fname) return info.dli_fname;
  return "";
}
