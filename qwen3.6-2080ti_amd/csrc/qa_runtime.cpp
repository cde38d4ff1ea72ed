// Library-level entry points: error string, version, arch.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "qa_common.h"

namespace qa {

static thread_local std::string g_last_error;

static void vset(const char* fmt, va_list ap) {
  char buf[1024];
  vsnprintf(buf, sizeof(buf), fmt, ap);
  g_last_error = buf;
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vset(fmt, ap);
  va_end(ap);
}

int fail(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vset(fmt, ap);
  va_end(ap);
  return 1;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail("%s: launch failed: %s", what, hipGetErrorString(err));
  return 0;
}

}  // namespace qa

extern "C" const char* qa_last_error(void) { return qa::g_last_error.c_str(); }

extern "C" int32_t qa_version(void) { return 1; }

extern "C" const char* qa_arch(void) { return "gfx950"; }
