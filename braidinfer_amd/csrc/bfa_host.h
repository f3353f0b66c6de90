// Host-side helpers for the C ABI entry points: argument checks, error text,
// launch-status translation.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "braidinfer_amd.h"

namespace bfa {

// Records a printf-style message for bfa_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Checks hipGetLastError() after a launch; BFA_OK or BFA_ERR_LAUNCH.
int check_launch(const char* what);

// Current value of planner override `key` (BFA_TUNE_*), -1 when unset.
int tuning(int key);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline bool is_float_dtype(int dt) {
  return dt == BFA_DTYPE_F32 || dt == BFA_DTYPE_F16 || dt == BFA_DTYPE_BF16;
}
inline int dtype_size(int dt) {
  switch (dt) {
    case BFA_DTYPE_F32: return 4;
    case BFA_DTYPE_F16: return 2;
    case BFA_DTYPE_BF16: return 2;
    case BFA_DTYPE_I32: return 4;
    case BFA_DTYPE_I64: return 8;
    default: return 0;
  }
}

__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace bfa

#define BFA_REQUIRE(cond, ...)                                      \
  do {                                                              \
    if (!(cond)) return ::bfa::set_error(BFA_ERR_INVALID, __VA_ARGS__); \
  } while (0)
