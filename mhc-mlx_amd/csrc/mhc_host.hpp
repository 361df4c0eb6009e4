// Host-side helpers for the C ABI: status codes, the per-thread error
// message, cached device properties and launch bookkeeping.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>
#include <string.h>

#include <algorithm>

#include "mhc_hip.h"

namespace mhc {

// Records a formatted message for mhc_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...);
void clear_error();

// Status for an invalid argument.
#define MHC_CHECK_ARG(cond, ...)                          \
  do {                                                    \
    if (!(cond)) return ::mhc::set_error(MHC_ERR_INVALID_ARG, __VA_ARGS__); \
  } while (0)

// Status for a HIP runtime failure (positive hipError_t).
#define MHC_CHECK_HIP(expr)                                                  \
  do {                                                                       \
    hipError_t e_ = (expr);                                                  \
    if (e_ != hipSuccess)                                                    \
      return ::mhc::set_error((int)e_, "%s failed: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

// After a kernel launch: surface launch-configuration errors immediately.
#define MHC_CHECK_LAUNCH(name)                                                 \
  do {                                                                         \
    hipError_t e_ = hipGetLastError();                                         \
    if (e_ != hipSuccess)                                                      \
      return ::mhc::set_error((int)e_, "launch of %s failed: %s", name, hipGetErrorString(e_)); \
  } while (0)

// Number of compute units of the current device (cached per device id).
int device_cu_count();

inline bool aligned(const void* p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % (uintptr_t)bytes) == 0; }

__host__ __device__ inline int next_pow2(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

__host__ __device__ inline int round_up(int v, int m) { return (v + m - 1) / m * m; }

}  // namespace mhc
