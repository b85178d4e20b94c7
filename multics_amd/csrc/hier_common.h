// Shared helpers for the hierattn HIP library: error reporting and launch checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "hierattn.h"

namespace hier {

// Thread-local last error message, read through hier_last_error().
extern thread_local char g_last_error[512];

inline int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
inline int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

inline void clear_error() { g_last_error[0] = 0; }

// Bytes spanned by a [rows][H][D] bf16 view with element strides ss and sh:
// ((rows - 1) * ss + (H - 1) * sh + D) * 2, in 128-bit arithmetic so that no
// caller-given stride can overflow it.  Strides must be non-negative.
inline __int128 span_bytes(int64_t rows, int64_t ss, int64_t sh, int64_t H, int64_t D) {
  const __int128 r = rows > 0 ? rows - 1 : 0, h = H > 0 ? H - 1 : 0;
  return (r * ss + h * sh + D) * 2;
}

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(HIER_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
  return HIER_OK;
}

// Workgroup barrier for LDS data only: waits for this wave's LDS operations,
// not for its outstanding global loads or LDS copies (__syncthreads' fence
// would wait for those too).
__device__ __forceinline__ void barrier_lds() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

}  // namespace hier

#define HIER_REQUIRE(cond, code, ...) \
  do {                                \
    if (!(cond)) return ::hier::fail(code, __VA_ARGS__); \
  } while (0)
