// Decode-step projections of the indexer sidecar (reference sidecar.py:74-88:
// wq(hidden), wk(hidden), weights_proj(hidden.float())) for a few tokens.
//
// With at most 16 tokens per step the products are weight-streaming: every
// weight byte is read once and used for <= 16 multiply-adds, so the bound is
// HBM bandwidth over the weights (wq 16 MiB + wk 0.5 MiB bf16 at hidden 2048).
// A platform GEMM tuned for large M leaves most of that bandwidth unused.
//
// project_bf16_kernel: one workgroup per 16 output features, its four waves
// each over a quarter of k, v_mfma_f32_16x16x32_bf16 with the tokens as the
// 16 A rows (zero rows past `tokens`) and the weight rows [n][k] as B
// columns: lane (r, g) loads 16 contiguous bytes of weight row n0 + r and of
// hidden row r at k = 32j + 8g for k-step j, kChunk k-steps in flight per
// wave.  The quarters are summed in LDS in a fixed order; fp32 accumulation,
// outputs rounded once to bf16, as a bf16 Linear stores them.
//
// project_f32_kernel: weights_proj in fp32 (the reference runs it on
// hidden.float()), one workgroup per output feature, 16 tokens per thread,
// fp32 FMAs and a block reduction.
//
// project_pair_kernel: wq and weights_proj of one hidden batch in one launch
// (the two grids side by side), each workgroup running the same code as in
// its own kernel, so the outputs are identical.
#include "common.hpp"
#include "dsa_amd.h"
#include "status.hpp"

namespace dsa {
namespace {

constexpr int kMaxProjTokens = 16;
constexpr int kChunk = 16;  // k-steps (32 k each) in flight per wave
constexpr int kSplitK = 4;  // waves per workgroup, each over a quarter of k

__device__ __forceinline__ uint16_t to_bf16_bits(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Output features [16 * block, 16 * block + 16) of the bf16 projection.
__device__ __forceinline__ void project_bf16_block(const uint16_t* hidden, int64_t hidden_stride, int tokens,
                                                   const uint16_t* weight, int kdim, uint16_t* out,
                                                   int64_t out_stride, int block, floatx4 (&part)[kSplitK][64]) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int n0 = block * 16;
  const BufferRsrc w = make_buffer(weight + (size_t)n0 * kdim, 16u * (uint32_t)kdim * 2u);
  // hidden rows past `tokens` read as zeros (range-checked buffer)
  const uint32_t h_bytes = (uint32_t)((tokens - 1) * hidden_stride + kdim) * 2u;
  const BufferRsrc h = make_buffer(hidden, h_bytes);
  const uint32_t w_row = (uint32_t)r * (uint32_t)kdim * 2u;
  const uint32_t h_row = r < tokens ? (uint32_t)(r * hidden_stride) * 2u : h_bytes;  // at the end: reads 0
  // wave w takes k-steps [w * per, (w + 1) * per), kChunk of them in flight at once
  const int steps = kdim / 32;
  const int per = (steps + kSplitK - 1) / kSplitK;
  const int first = wave * per;
  const int last = min(steps, first + per);
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int base = first; base < last; base += kChunk) {
    uint4 wb[kChunk], hb[kChunk];
#pragma unroll
    for (int j = 0; j < kChunk; ++j) {
      const int step = min(base + j, last - 1);
      const uint32_t k_bytes = (uint32_t)(32 * step + 8 * g) * 2u;
      wb[j] = buffer_load_16(w, w_row + k_bytes);
      hb[j] = buffer_load_16(h, h_row + k_bytes);
    }
#pragma unroll
    for (int j = 0; j < kChunk; ++j)
      if (base + j < last) acc = mfma_16x16x32(Bf16Tag{}, hb[j], wb[j], acc);
  }
  part[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  const floatx4 a0 = part[0][lane], a1 = part[1][lane], a2 = part[2][lane], a3 = part[3][lane];
  // lane (r, g) holds C[token 4g + i][feature n0 + r], summed over the k quarters in a fixed order
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = 4 * g + i;
    if (t < tokens) out[(size_t)t * out_stride + n0 + r] = to_bf16_bits((a0[i] + a1[i]) + (a2[i] + a3[i]));
  }
}

// Output feature n of the fp32 projection.
__device__ __forceinline__ void project_f32_block(const uint16_t* hidden, int64_t hidden_stride, int tokens,
                                                  const float* weight, int kdim, float* out, int64_t out_stride,
                                                  int n, float (&partial)[4][kMaxProjTokens]) {
  const int tid = threadIdx.x;
  const float* wrow = weight + (size_t)n * kdim;
  float acc[kMaxProjTokens];
#pragma unroll
  for (int t = 0; t < kMaxProjTokens; ++t) acc[t] = 0.f;
  for (int k = tid; k < kdim; k += 256) {
    const float wk = wrow[k];
#pragma unroll
    for (int t = 0; t < kMaxProjTokens; ++t)
      if (t < tokens) acc[t] = fmaf(__uint_as_float((uint32_t)hidden[(size_t)t * hidden_stride + k] << 16), wk, acc[t]);
  }
#pragma unroll
  for (int t = 0; t < kMaxProjTokens; ++t) {
    float v = acc[t];
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    acc[t] = v;
  }
  if ((tid & 63) == 0)
#pragma unroll
    for (int t = 0; t < kMaxProjTokens; ++t) partial[tid >> 6][t] = acc[t];
  __syncthreads();
  if (tid < tokens) out[(size_t)tid * out_stride + n] = (partial[0][tid] + partial[1][tid]) + (partial[2][tid] + partial[3][tid]);
}

__global__ __launch_bounds__(256) void project_bf16_kernel(const uint16_t* hidden, int64_t hidden_stride, int tokens,
                                                           const uint16_t* weight, int kdim, uint16_t* out,
                                                           int64_t out_stride) {
  __shared__ floatx4 part[kSplitK][64];
  project_bf16_block(hidden, hidden_stride, tokens, weight, kdim, out, out_stride, blockIdx.x, part);
}

__global__ __launch_bounds__(256) void project_f32_kernel(const uint16_t* hidden, int64_t hidden_stride, int tokens,
                                                          const float* weight, int kdim, float* out,
                                                          int64_t out_stride) {
  __shared__ float partial[4][kMaxProjTokens];
  project_f32_block(hidden, hidden_stride, tokens, weight, kdim, out, out_stride, blockIdx.x, partial);
}

// Both projections of one hidden batch in one grid: workgroups [0, bf16_blocks)
// take the bf16 projection's 16-feature groups, the rest one fp32 feature each.
__global__ __launch_bounds__(256) void project_pair_kernel(const uint16_t* hidden, int64_t hidden_stride, int tokens,
                                                           int kdim, const uint16_t* weight_a, int bf16_blocks,
                                                           uint16_t* out_a, int64_t out_a_stride,
                                                           const float* weight_b, float* out_b, int64_t out_b_stride) {
  __shared__ floatx4 part[kSplitK][64];
  __shared__ float partial[4][kMaxProjTokens];
  const int b = blockIdx.x;
  if (b < bf16_blocks)
    project_bf16_block(hidden, hidden_stride, tokens, weight_a, kdim, out_a, out_a_stride, b, part);
  else
    project_f32_block(hidden, hidden_stride, tokens, weight_b, kdim, out_b, out_b_stride, b - bf16_blocks, partial);
}

}  // namespace
}  // namespace dsa

using namespace dsa;

extern "C" int dsa_project_rows(const void* hidden, int64_t hidden_stride, int64_t tokens, const void* weight,
                                int32_t weight_dtype, int64_t features, int64_t kdim, void* out, int64_t out_stride,
                                void* stream) {
  DSA_REQUIRE(hidden && weight && out, "null pointer argument");
  DSA_REQUIRE(tokens >= 1 && tokens <= kMaxProjTokens, "tokens %lld outside [1, 16]", (long long)tokens);
  DSA_REQUIRE(kdim >= 32 && kdim % 32 == 0 && kdim <= (1 << 20), "kdim %lld must be a multiple of 32",
              (long long)kdim);
  DSA_REQUIRE(hidden_stride >= kdim && hidden_stride % 8 == 0, "hidden_stride must be >= kdim and a multiple of 8");
  DSA_REQUIRE(out_stride >= features, "out_stride < features");
  DSA_REQUIRE(reinterpret_cast<uintptr_t>(hidden) % 16 == 0 && reinterpret_cast<uintptr_t>(weight) % 16 == 0,
              "hidden and weight must be 16-byte aligned");
  DSA_REQUIRE((tokens - 1) * hidden_stride + kdim < (int64_t(1) << 30), "hidden too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* h = static_cast<const uint16_t*>(hidden);
  if (weight_dtype == DSA_DTYPE_BF16) {
    DSA_REQUIRE(features >= 16 && features % 16 == 0, "bf16 features %lld must be a multiple of 16",
                (long long)features);
    DSA_REQUIRE(16 * kdim * 2 < (int64_t(1) << 31), "weight rows too long");
    hipLaunchKernelGGL(project_bf16_kernel, dim3((unsigned)(features / 16)), dim3(64 * kSplitK), 0, s, h, hidden_stride,
                       (int)tokens, static_cast<const uint16_t*>(weight), (int)kdim, static_cast<uint16_t*>(out),
                       out_stride);
    return check_launch("project_bf16_kernel");
  }
  DSA_REQUIRE(weight_dtype == DSA_DTYPE_F32, "weights must be bf16 or fp32 (got %d)", weight_dtype);
  DSA_REQUIRE(features >= 1 && features <= 65535, "features out of range");
  hipLaunchKernelGGL(project_f32_kernel, dim3((unsigned)features), dim3(256), 0, s, h, hidden_stride, (int)tokens,
                     static_cast<const float*>(weight), (int)kdim, static_cast<float*>(out), out_stride);
  return check_launch("project_f32_kernel");
}

extern "C" int dsa_project_rows_pair(const void* hidden, int64_t hidden_stride, int64_t tokens, int64_t kdim,
                                     const void* weight_bf16, int64_t features_bf16, void* out_bf16,
                                     int64_t out_bf16_stride, const float* weight_f32, int64_t features_f32,
                                     float* out_f32, int64_t out_f32_stride, void* stream) {
  DSA_REQUIRE(hidden && weight_bf16 && out_bf16 && weight_f32 && out_f32, "null pointer argument");
  DSA_REQUIRE(tokens >= 1 && tokens <= kMaxProjTokens, "tokens %lld outside [1, 16]", (long long)tokens);
  DSA_REQUIRE(kdim >= 32 && kdim % 32 == 0 && kdim <= (1 << 20), "kdim %lld must be a multiple of 32",
              (long long)kdim);
  DSA_REQUIRE(hidden_stride >= kdim && hidden_stride % 8 == 0, "hidden_stride must be >= kdim and a multiple of 8");
  DSA_REQUIRE(features_bf16 >= 16 && features_bf16 % 16 == 0, "bf16 features %lld must be a multiple of 16",
              (long long)features_bf16);
  DSA_REQUIRE(features_f32 >= 1, "fp32 features out of range");
  DSA_REQUIRE(features_bf16 / 16 + features_f32 <= 0x7fffffffLL, "too many features");
  DSA_REQUIRE(out_bf16_stride >= features_bf16 && out_f32_stride >= features_f32, "output stride < features");
  DSA_REQUIRE(reinterpret_cast<uintptr_t>(hidden) % 16 == 0 && reinterpret_cast<uintptr_t>(weight_bf16) % 16 == 0,
              "hidden and weight must be 16-byte aligned");
  DSA_REQUIRE((tokens - 1) * hidden_stride + kdim < (int64_t(1) << 30), "hidden too large");
  DSA_REQUIRE(16 * kdim * 2 < (int64_t(1) << 31), "weight rows too long");
  const int bf16_blocks = (int)(features_bf16 / 16);
  hipLaunchKernelGGL(project_pair_kernel, dim3((unsigned)(bf16_blocks + features_f32)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(hidden), hidden_stride, (int)tokens,
                     (int)kdim, static_cast<const uint16_t*>(weight_bf16), bf16_blocks, static_cast<uint16_t*>(out_bf16),
                     out_bf16_stride, weight_f32, out_f32, out_f32_stride);
  return check_launch("project_pair_kernel");
}
