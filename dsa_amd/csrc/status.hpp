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

// A fresh nonzero 32-bit stamp for one launch whose workgroups meet at
// barriers of generation-stamped slots.  Stamps follow each other from a
// start drawn per library load (clock and process id), so that slots an
// earlier load of the library stamped are not read as this launch's.
uint32_t next_generation();

// Workgroups of `kernel` (threads per workgroup, dynamic LDS bytes) that are
// resident at once on the current device: the occupancy limit per CU times
// the CU count (cached per device, kernel and LDS size).
int resident_capacity(const void* kernel, int threads, size_t lds, int64_t& capacity);

// An unsigned decimal from the environment, or `fallback` when the variable is
// unset, malformed or not below `limit`.
uint32_t env_limit(const char* name, uint32_t fallback, uint32_t limit);

}  // namespace dsa

#define DSA_REQUIRE(cond, ...)                                          \
  do {                                                                  \
    if (!(cond)) return ::dsa::fail(DSA_STATUS_INVALID_ARGUMENT, __VA_ARGS__); \
  } while (0)
