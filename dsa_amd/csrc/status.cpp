#include "status.hpp"

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <unistd.h>

#include <atomic>
#include <chrono>
#include <mutex>

namespace dsa {

namespace {
thread_local char g_message[512] = "";
}

int fail(int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_message, sizeof(g_message), fmt, args);
  va_end(args);
  return code;
}

int check_hip(hipError_t err, const char* what) {
  if (err == hipSuccess) return DSA_STATUS_OK;
  return fail(DSA_STATUS_HIP_ERROR, "%s: %s", what, hipGetErrorString(err));
}

int check_launch(const char* what) { return check_hip(hipGetLastError(), what); }

namespace {
uint32_t first_generation() {
  const uint64_t t = (uint64_t)std::chrono::steady_clock::now().time_since_epoch().count();
  uint64_t x = t ^ ((uint64_t)getpid() << 32) ^ (uint64_t)reinterpret_cast<uintptr_t>(&t);
  x ^= x >> 33;  // splitmix64 finaliser
  x *= 0xff51afd7ed558ccdull;
  x ^= x >> 33;
  x *= 0xc4ceb9fe1a85ec53ull;
  x ^= x >> 33;
  return (uint32_t)x;
}
std::atomic<uint32_t> g_generation{first_generation()};

struct CapacityEntry {
  int device;
  const void* kernel;
  int threads;
  size_t lds;
  int64_t capacity;
};
std::mutex g_capacity_mutex;
CapacityEntry g_capacity[64];
int g_capacity_count = 0;
}  // namespace

uint32_t next_generation() {
  uint32_t gen = 0;
  while (gen == 0) gen = ++g_generation;  // 0 never names a launch (a zeroed slot)
  return gen;
}

int resident_capacity(const void* kernel, int threads, size_t lds, int64_t& capacity) {
  int device = 0;
  if (int st = check_hip(hipGetDevice(&device), "hipGetDevice")) return st;
  std::lock_guard<std::mutex> lock(g_capacity_mutex);
  for (int i = 0; i < g_capacity_count; ++i) {
    const CapacityEntry& e = g_capacity[i];
    if (e.device == device && e.kernel == kernel && e.threads == threads && e.lds == lds) {
      capacity = e.capacity;
      return DSA_STATUS_OK;
    }
  }
  int per_cu = 0;
  int cus = 0;
  if (int st = check_hip(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, lds),
                         "hipOccupancyMaxActiveBlocksPerMultiprocessor"))
    return st;
  if (int st = check_hip(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device),
                         "hipDeviceGetAttribute"))
    return st;
  capacity = (int64_t)per_cu * cus;
  if (g_capacity_count < 64) g_capacity[g_capacity_count++] = {device, kernel, threads, lds, capacity};
  return DSA_STATUS_OK;
}

uint32_t env_limit(const char* name, uint32_t fallback, uint32_t limit) {
  const char* v = getenv(name);
  if (!v || !*v) return fallback;
  char* end = nullptr;
  const unsigned long n = strtoul(v, &end, 10);
  return (end && *end == 0 && n < limit) ? (uint32_t)n : fallback;
}

}  // namespace dsa

extern "C" const char* dsa_last_error(void) { return dsa::g_message; }

extern "C" int dsa_abi_version(void) { return DSA_ABI_VERSION; }
