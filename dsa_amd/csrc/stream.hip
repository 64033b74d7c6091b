// Measured streaming-read ceiling for the roofline: one launch reads a buffer
// with the grid and load pattern of the decode scoring kernel (256
// workgroups of 4 waves, XCD-aware numbering, each wave streaming 64-key
// units of 256-byte rows with lane (r, g) loading 16 bytes of key r at offset
// 16g + 64c, two units in flight) and only folds the loaded words into a
// register, so its time is what the memory system gives that access stream.
#include "common.hpp"
#include "dsa_amd.h"
#include "select.hpp"
#include "status.hpp"

namespace dsa {
namespace {

constexpr uint32_t kUnitBytes = 64 * 256;

__global__ __launch_bounds__(256) void stream_read_kernel(const uint8_t* data, uint32_t bytes_per_wg, float* sink) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;
  const int g = lane >> 4;
  const uint32_t logical = (blockIdx.x % kXcds) * (gridDim.x / kXcds) + blockIdx.x / kXcds;
  const BufferRsrc rs = make_buffer(data + (size_t)logical * bytes_per_wg, bytes_per_wg);
  const int units = (int)(bytes_per_wg / kUnitBytes);
  const int n = (units - wave + 3) / 4;
  if (n <= 0) return;
  uint4 buf[2][16];
  auto load = [&](int i, uint4 (&b)[16]) {
    const uint32_t base = (uint32_t)(wave + 4 * min(i, n - 1)) * kUnitBytes;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int c = 0; c < 4; ++c) b[4 * t + c] = buffer_load_16(rs, base + (uint32_t)(16 * t + r) * 256u + 16u * g + 64u * c);
  };
  uint32_t acc = 0;
  load(0, buf[0]);
  for (int i = 0; i < n; i += 2) {
    load(i + 1, buf[1]);
#pragma unroll
    for (int c = 0; c < 16; ++c) acc ^= buf[0][c].x ^ buf[0][c].w;
    if (i + 1 >= n) break;
    load(i + 2, buf[0]);
#pragma unroll
    for (int c = 0; c < 16; ++c) acc ^= buf[1][c].x ^ buf[1][c].w;
  }
  if (acc == 0x9e3779b9u) sink[threadIdx.x] = 1.f;  // keeps the loads; practically never taken
}

}  // namespace
}  // namespace dsa

using namespace dsa;

extern "C" int dsa_stream_read(const void* data, int64_t bytes, int32_t workgroups, float* sink, void* stream,
                               void* start_event, void* stop_event) {
  DSA_REQUIRE(data && sink, "null pointer argument");
  DSA_REQUIRE(workgroups >= kXcds && workgroups % kXcds == 0 && workgroups <= 65536,
              "workgroups must be a positive multiple of 8");
  DSA_REQUIRE(bytes > 0 && bytes % ((int64_t)workgroups * kUnitBytes) == 0 &&
                  bytes / workgroups <= (int64_t)0x7fffffff,
              "bytes must split into whole 16 KiB units per workgroup");
  DSA_REQUIRE(reinterpret_cast<uintptr_t>(data) % 16 == 0, "data must be 16-byte aligned");
  launch_timed(stream_read_kernel, dim3(workgroups), dim3(256), 0, static_cast<hipStream_t>(stream),
               static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(stop_event),
               static_cast<const uint8_t*>(data), (uint32_t)(bytes / workgroups), sink);
  return check_launch("stream_read_kernel");
}
