// Per-query head routing: the `width` heads with the largest key value, ties
// to the lower head id (a stable descending argsort truncated to `width`).
// Reference: progressive_kernel.py:37-42 (dynamic_head_ids, key = |w|) and
// verifier_scoring.py:142-159 (dynamic_head_indices, key = |w| or max(w, 0)).
//
// One wave per query row, one lane per head (heads <= 64): each lane counts the
// heads that sort before it, which is its rank in the stable order.
#include "common.hpp"
#include "status.hpp"

namespace dsa {
namespace {

__global__ __launch_bounds__(256) void route_heads_kernel(const float* weights, int64_t rows,
                                                          int heads, int width, int positive,
                                                          int32_t* out32, int64_t* out64) {
  const int lane = threadIdx.x & 63;
  const int64_t row = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  if (row >= rows) return;
  float v = -__builtin_inff();
  if (lane < heads) {
    const float w = weights[row * heads + lane];
    v = positive ? fmaxf(w, 0.f) : fabsf(w);
  }
  int rank = 0;
  for (int j = 0; j < heads; ++j) {
    const float other = __shfl(v, j, kWave);
    rank += (other > v || (other == v && j < lane)) ? 1 : 0;
  }
  if (lane < heads && rank < width) {
    if (out32) out32[row * width + rank] = lane;
    if (out64) out64[row * width + rank] = lane;
  }
}

}  // namespace
}  // namespace dsa

using namespace dsa;

extern "C" int dsa_route_heads(const float* weights, int64_t rows, int64_t heads, int64_t width,
                               int32_t positive_only, int32_t* out_int32, int64_t* out_int64,
                               void* stream) {
  DSA_REQUIRE(weights && (out_int32 || out_int64), "null pointer argument");
  DSA_REQUIRE(rows > 0, "rows must be positive");
  DSA_REQUIRE(heads > 0 && heads <= kWave, "heads %lld outside [1, 64]", (long long)heads);
  DSA_REQUIRE(width > 0 && width <= heads, "invalid head width");
  const int64_t blocks = (rows + 3) / 4;
  hipLaunchKernelGGL(route_heads_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), weights, rows, (int)heads, (int)width,
                     positive_only ? 1 : 0, out_int32, out_int64);
  return check_launch("route_heads_kernel");
}
