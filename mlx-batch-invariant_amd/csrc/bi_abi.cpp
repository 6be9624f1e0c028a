// Library-wide ABI entry points: version and thread-local error reporting.
#include <stdio.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "bi_internal.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace bi {

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int launch_error(int hip_error, const char* what) {
  return fail(BI_ELAUNCH, "%s: HIP error %d (%s)", what, hip_error,
              hipGetErrorString(static_cast<hipError_t>(hip_error)));
}

}  // namespace bi

extern "C" int bi_abi_version(void) { return BI_ABI_VERSION; }

extern "C" const char* bi_last_error(void) { return g_last_error; }
