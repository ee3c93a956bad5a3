// Error reporting for the C ABI (thread-local last-error message) and the roctx
// range of each call.
#include <rocprofiler-sdk-roctx/roctx.h>

#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace astr {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
  va_end(args);
  return code;
}

int hip_fail(hipError_t err, const char* what) {
  snprintf(g_last_error, sizeof(g_last_error), "%s: %s", what, hipGetErrorString(err));
  return (int)err;
}

CallRange::CallRange(const char* name) { roctxRangePushA(name); }
CallRange::~CallRange() { roctxRangePop(); }

}  // namespace astr

extern "C" const char* astr_last_error(void) { return astr::g_last_error; }

extern "C" const char* astr_version(void) { return "aster_kv 0.1.0 gfx950"; }
