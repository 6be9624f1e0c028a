// Shared host-side helpers of libbi.so: status/error reporting and argument
// validation. Device code lives in bi_gemm.hip and bi_sdpa.hip.
#pragma once

#include <stdint.h>
#include <stdarg.h>

#include "bi.h"
#include "bi_testing.h"

namespace bi {

// Records a printf-style message as this thread's last error and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Maps a HIP launch/runtime error (as an int) to BI_ELAUNCH with its message.
int launch_error(int hip_error, const char* what);

inline int elem_size(int dtype) {
  return dtype == BI_F32 ? 4 : (dtype == BI_F16 || dtype == BI_BF16) ? 2 : 0;
}

}  // namespace bi
