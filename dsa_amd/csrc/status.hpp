// Status codes and the thread-local error message behind dsa_last_error().
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/dsa_amd.h"

namespace dsa {

// Records a formatted message for dsa_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Returns DSA_STATUS_OK, or records the pending HIP launch error.
int check_launch(const char* what);

// Returns DSA_STATUS_OK if `err` is hipSuccess, else records it.
int check_hip(hipError_t err, const char* what);

}  // namespace dsa

#define DSA_REQUIRE(cond, ...)                                          \
  do {                                                                  \
    if (!(cond)) return ::dsa::fail(DSA_STATUS_INVALID_ARGUMENT, __VA_ARGS__); \
  } while (0)
