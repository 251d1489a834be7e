// Host-side helpers of the C ABI: per-thread error text and argument checks.
#pragma once

#include <stdint.h>

#include "../../include/fdl.h"

namespace fdl {

// Records `fmt` (printf-style) as the calling thread's last error and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the calling thread's last error and returns FDL_OK.
int ok();

}  // namespace fdl

#define FDL_REQUIRE(cond, code, ...)      \
  do {                                    \
    if (!(cond)) return fdl::fail((code), __VA_ARGS__); \
  } while (0)

#define FDL_REQUIRE_PTR(p) FDL_REQUIRE((p) != nullptr, FDL_ERR_NULL, "%s: %s is NULL", __func__, #p)

#define FDL_REQUIRE_ALIGNED(p, n)                                                       \
  FDL_REQUIRE((reinterpret_cast<uintptr_t>(p) % (n)) == 0, FDL_ERR_SHAPE,              \
              "%s: %s is not %d-byte aligned", __func__, #p, (int)(n))

// Checks a HIP call made while enqueueing work.
#define FDL_HIP_CHECK(expr)                                                              \
  do {                                                                                   \
    hipError_t e_ = (expr);                                                              \
    if (e_ != hipSuccess)                                                                \
      return fdl::fail(FDL_ERR_HIP, "%s: %s failed: %s", __func__, #expr,               \
                       hipGetErrorString(e_));                                           \
  } while (0)
