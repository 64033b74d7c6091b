// Block summaries used by the temporal pruning bounds:
//   * per-block maxima of score rows (reference replay.py:149-150, approx.py:53-55)
//   * per-block maximum key norms (reference certified.py:51-62)
//   * the certified temporal radius (reference certified.py:18-48)
#include "common.hpp"
#include "status.hpp"

namespace dsa {
namespace {

// One thread per (row, block).
__global__ __launch_bounds__(256) void block_max_kernel(const float* scores, int64_t rows,
                                                        int length, int64_t row_stride, int bs,
                                                        float* out) {
  const int nb = (length + bs - 1) / bs;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = gid / nb;
  const int block = (int)(gid % nb);
  if (row >= rows) return;
  const float* x = scores + row * row_stride;
  const int start = block * bs;
  const int stop = min(length, start + bs);
  float m = -__builtin_inff();
  for (int i = start; i < stop; ++i) m = fmaxf(m, x[i]);
  // numpy's max propagates NaN; fmaxf drops it.  Scores are NaN-free by contract.
  out[row * nb + block] = m;
}

__device__ __forceinline__ float load_as_float(const void* p, int64_t i, int dtype) {
  switch (dtype) {
    case kF32: return static_cast<const float*>(p)[i];
    case kF16: return (float)static_cast<const _Float16*>(p)[i];
    case kBF16: return __uint_as_float(uint32_t(static_cast<const uint16_t*>(p)[i]) << 16);
    default: {
      const uint32_t byte = static_cast<const uint8_t*>(p)[i];
      return __builtin_amdgcn_cvt_pk_f32_fp8(byte, false)[0];
    }
  }
}

// One wave per (block, head).  Squares and sums are taken in float64 (the
// reference works in float64), so the norm does not round below the float64
// value by more than one rounding of the final sqrt.
__global__ __launch_bounds__(256) void block_key_norms_kernel(const void* keys, int64_t tokens,
                                                              int heads, int dim, int bs,
                                                              int dtype, double* out) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t nb = (tokens + bs - 1) / bs;
  if (wid >= nb * heads) return;
  const int64_t block = wid / heads;
  const int head = (int)(wid % heads);
  const int64_t start = block * bs;
  const int64_t stop = min(tokens, start + bs);
  double best = 0.0;
  for (int64_t t = start; t < stop; ++t) {
    const int64_t row = (t * heads + head) * dim;
    double acc = 0.0;
    for (int d = lane; d < dim; d += kWave) {
      const double x = load_as_float(keys, row + d, dtype);
      acc = fma(x, x, acc);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, kWave);
    best = fmax(best, sqrt(acc));
  }
  if (lane == 0) out[block * heads + head] = best;
}

constexpr int kMaxRadiusHeads = 1024;

// Relative rounding allowance of the radius.  Any float64 evaluation of the
// formula (numpy's norm and matrix product included) is within about
// (dim + heads + 4) * 2^-53 of the exact value, so two of them differ by less
// than 2^-38 when dim + heads <= 8188 (the entry point's limit); scaling the
// result by (1 + 2^-36) keeps it at or above the reference's float64 value.
constexpr int kMaxRadiusTerms = 8188;
constexpr double kRadiusRoundUp = 1.0 + 0x1p-36;

// Per head: c_h = |w_now - w_prev| ||q_prev,h|| + |w_now| ||q_now,h - q_prev,h||
// (certified.py:43-47), then out[b] = sum_h norm[b, h] * c_h, all in float64.
__global__ __launch_bounds__(256) void temporal_radius_kernel(const double* q_now,
                                                              const double* q_prev,
                                                              const double* w_now,
                                                              const double* w_prev,
                                                              const double* norms, int64_t blocks,
                                                              int heads, int dim, double* out) {
  __shared__ double coef[kMaxRadiusHeads];
  for (int h = threadIdx.x; h < heads; h += blockDim.x) {
    double prev_sq = 0.0;
    double diff_sq = 0.0;
    for (int d = 0; d < dim; ++d) {
      const double p = q_prev[(int64_t)h * dim + d];
      const double c = q_now[(int64_t)h * dim + d];
      prev_sq = fma(p, p, prev_sq);
      diff_sq = fma(c - p, c - p, diff_sq);
    }
    coef[h] = fabs(w_now[h] - w_prev[h]) * sqrt(prev_sq) + fabs(w_now[h]) * sqrt(diff_sq);
  }
  __syncthreads();
  for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < blocks;
       b += (int64_t)gridDim.x * blockDim.x) {
    double r = 0.0;
    for (int h = 0; h < heads; ++h) r = fma(norms[b * heads + h], coef[h], r);
    out[b] = r * kRadiusRoundUp;
  }
}

// Certified per-block margins of a temporal step over a shared-key cache (one
// key row per token, seen by all 64 heads): the reference's radius
// (certified.py:43-47) with every head's block norm equal to the block's
// largest key norm n_b,
//   radius_b = n_b * sum_h (|w_now - w_prev|_h ||q_prev,h|| + |w_now|_h ||q_now,h - q_prev,h||),
// plus an allowance for the fp32 rounding of the two steps' scores: a score
// computed from bf16/fp16 operands (exact products, fp32 sums over 128 dims
// and 64 heads) is within (128 + 64 + 4) * 2^-24 < 2^-15 of
// sum_h |w_h| ||q_h|| ||k|| of its exact value, so
//   margin_b = n_b * (C + 2^-15 * sum_h (|w_now|_h ||q_now,h|| + |w_prev|_h ||q_prev,h||))
// bounds |score_now - score_prev| of every key of the block as computed here.
// Everything is float64 and the result is scaled by kRadiusRoundUp.  One wave
// per block; each workgroup derives its row's two head sums first.
constexpr double kScoreRoundingAllowance = 0x1p-15;

__global__ __launch_bounds__(256) void certified_margins_kernel(const uint16_t* q_now, const uint16_t* q_prev,
                                                                const float* w_now, const float* w_prev,
                                                                const uint16_t* keys, int64_t key_stride,
                                                                int prev_length, int block_size, int blocks_per_row,
                                                                int q_dtype, double* margins) {
  __shared__ double s_radius[kHeads];
  __shared__ double s_slack[kHeads];
  const int row = blockIdx.y;
  const int tid = threadIdx.x;
  auto q_at = [&](const uint16_t* q, int i) -> double {
    const uint16_t bits = q[(size_t)row * kHeads * kHeadDim + i];
    return q_dtype == kBF16 ? (double)__uint_as_float(uint32_t(bits) << 16)
                            : (double)(float)__builtin_bit_cast(_Float16, bits);
  };
  if (tid < kHeads) {
    double prev_sq = 0.0, now_sq = 0.0, diff_sq = 0.0;
    for (int d = 0; d < kHeadDim; ++d) {
      const double p = q_at(q_prev, tid * kHeadDim + d);
      const double c = q_at(q_now, tid * kHeadDim + d);
      prev_sq = fma(p, p, prev_sq);
      now_sq = fma(c, c, now_sq);
      diff_sq = fma(c - p, c - p, diff_sq);
    }
    const double wn = (double)w_now[(size_t)row * kHeads + tid];
    const double wp = (double)w_prev[(size_t)row * kHeads + tid];
    s_radius[tid] = fabs(wn - wp) * sqrt(prev_sq) + fabs(wn) * sqrt(diff_sq);
    s_slack[tid] = fabs(wn) * sqrt(now_sq) + fabs(wp) * sqrt(prev_sq);
  }
  __syncthreads();
  double radius = 0.0, slack = 0.0;
  for (int h = 0; h < kHeads; ++h) {
    radius += s_radius[h];
    slack += s_slack[h];
  }
  const double coef = radius + kScoreRoundingAllowance * slack;
  const int lane = tid & 63;
  const int b = blockIdx.x * 4 + (tid >> 6);
  if (b >= blocks_per_row) return;
  const int start = b * block_size;
  const int stop = min(prev_length, start + block_size);
  double best = 0.0;
  for (int t = start; t < stop; ++t) {
    // lane l holds dims 2l, 2l + 1 of the key row
    const uint32_t two = reinterpret_cast<const uint32_t*>(keys + ((size_t)row * key_stride + t) * kHeadDim)[lane];
    double x0, x1;
    if (q_dtype == kBF16) {
      x0 = (double)__uint_as_float(two << 16);
      x1 = (double)__uint_as_float(two & 0xffff0000u);
    } else {
      x0 = (double)(float)__builtin_bit_cast(_Float16, (uint16_t)(two & 0xffffu));
      x1 = (double)(float)__builtin_bit_cast(_Float16, (uint16_t)(two >> 16));
    }
    double acc = fma(x0, x0, x1 * x1);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, kWave);
    best = fmax(best, sqrt(acc));
  }
  if (lane == 0) margins[(size_t)row * blocks_per_row + b] = best * coef * kRadiusRoundUp;
}

}  // namespace
}  // namespace dsa

using namespace dsa;

extern "C" int dsa_certified_margins(const void* q_now, const void* q_prev, const float* w_now, const float* w_prev,
                                     const void* keys, int64_t key_stride, int64_t batch, int64_t prev_length,
                                     int32_t block_size, int32_t key_dtype, double* margins, void* stream) {
  DSA_REQUIRE(q_now && q_prev && w_now && w_prev && keys && margins, "null pointer argument");
  DSA_REQUIRE(batch > 0 && batch <= 65535, "batch %lld out of range", (long long)batch);
  DSA_REQUIRE(prev_length > 0 && prev_length <= key_stride && prev_length < (int64_t(1) << 31),
              "prev_length %lld invalid", (long long)prev_length);
  DSA_REQUIRE(block_size > 0, "block_size must be positive");
  DSA_REQUIRE(key_dtype == kBF16 || key_dtype == kF16, "certified margins take bf16/fp16 queries and keys");
  DSA_REQUIRE(reinterpret_cast<uintptr_t>(keys) % 4 == 0, "keys must be 4-byte aligned");
  const int64_t blocks = (prev_length + block_size - 1) / block_size;
  hipLaunchKernelGGL(certified_margins_kernel, dim3((unsigned)((blocks + 3) / 4), (unsigned)batch), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(q_now),
                     static_cast<const uint16_t*>(q_prev), w_now, w_prev, static_cast<const uint16_t*>(keys),
                     key_stride, (int)prev_length, (int)block_size, (int)blocks, (int)key_dtype, margins);
  return check_launch("certified_margins_kernel");
}

extern "C" int dsa_block_max(const float* scores, int64_t rows, int64_t length,
                             int64_t row_stride, int32_t block_size, float* out, void* stream) {
  DSA_REQUIRE(scores && out, "null pointer argument");
  DSA_REQUIRE(rows > 0 && length > 0 && length < (int64_t(1) << 31), "bad shape");
  DSA_REQUIRE(row_stride >= length, "row_stride < length");
  DSA_REQUIRE(block_size > 0, "block_size must be positive");
  const int64_t nb = (length + block_size - 1) / block_size;
  const int64_t total = rows * nb;
  hipLaunchKernelGGL(block_max_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), scores, rows, (int)length, row_stride,
                     (int)block_size, out);
  return check_launch("block_max_kernel");
}

extern "C" int dsa_block_key_norms(const void* keys, int64_t tokens, int64_t heads, int64_t dim,
                                   int32_t block_size, int32_t key_dtype, double* out,
                                   void* stream) {
  DSA_REQUIRE(keys && out, "null pointer argument");
  DSA_REQUIRE(tokens > 0 && heads > 0 && dim > 0, "bad shape");
  DSA_REQUIRE(block_size > 0, "block_size must be positive");
  DSA_REQUIRE(key_dtype >= kF32 && key_dtype <= kFP8E4M3, "unknown dtype %d", key_dtype);
  const int64_t nb = (tokens + block_size - 1) / block_size;
  const int64_t waves = nb * heads;
  hipLaunchKernelGGL(block_key_norms_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), keys, tokens, (int)heads, (int)dim,
                     (int)block_size, (int)key_dtype, out);
  return check_launch("block_key_norms_kernel");
}

extern "C" int dsa_temporal_score_radius(const double* q_now, const double* q_prev,
                                         const double* w_now, const double* w_prev,
                                         const double* block_key_norm, int64_t blocks,
                                         int64_t heads, int64_t dim, double* out, void* stream) {
  DSA_REQUIRE(q_now && q_prev && w_now && w_prev && block_key_norm && out, "null pointer");
  DSA_REQUIRE(blocks > 0 && heads > 0 && heads <= kMaxRadiusHeads && dim > 0, "bad shape");
  DSA_REQUIRE(dim + heads <= kMaxRadiusTerms, "dim + heads must be at most %d", kMaxRadiusTerms);
  const int64_t want = (blocks + 255) / 256;
  const unsigned grid = (unsigned)(want < 1024 ? want : 1024);
  hipLaunchKernelGGL(temporal_radius_kernel, dim3(grid), dim3(256), 0,
                     static_cast<hipStream_t>(stream), q_now, q_prev, w_now, w_prev,
                     block_key_norm, blocks, (int)heads, (int)dim, out);
  return check_launch("temporal_radius_kernel");
}
