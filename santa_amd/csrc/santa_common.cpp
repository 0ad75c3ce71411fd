// santa_common.cpp -- error reporting and version of the C ABI.
#include <cstdarg>
#include <cstdio>

#include "santa_amd.h"
#include "santa_internal.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace santa {

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int clear_error() {
  g_last_error[0] = '\0';
  return SANTA_OK;
}

}  // namespace santa

extern "C" const char* santa_last_error(void) { return g_last_error; }

extern "C" const char* santa_version(void) { return "santa_amd 0.1.0 (gfx950)"; }
