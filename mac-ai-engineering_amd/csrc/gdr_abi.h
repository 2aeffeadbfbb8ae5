// Host-side helpers of the C ABI shared by the library's sources: the calling thread's last error message (what
// macai_gdr_last_error returns), the launch check and the alignment rule.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "macai_gdr.h"

inline thread_local char g_err[512] = "";

inline int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

inline int launched(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MACAI_GDR_ELAUNCH, "%s: HIP launch failed: %s", what, hipGetErrorString(e));
  g_err[0] = 0;
  return MACAI_GDR_OK;
}

inline bool aligned16(const void* p) { return p == nullptr || ((uintptr_t)p & 15u) == 0; }
