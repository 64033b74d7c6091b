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

// Power-of-two blocks of at most 128 keys, read coalesced: wave w takes run
// w of a row, 64 consecutive keys (128 for 128-key blocks: lane l reads keys
// l and l + 64), and reduces each block across its lanes by shuffles; the
// block's first lane writes its maximum.  Same fmaxf from -inf as above.
__global__ __launch_bounds__(256) void block_max_runs_kernel(const float* scores, int64_t rows, int length,
                                                             int64_t row_stride, int bs, int runs_per_row,
                                                             float* out) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t run = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const int64_t row = run / runs_per_row;
  if (row >= rows) return;  // whole waves
  const int span = bs > kWave ? 2 * kWave : kWave;
  const int reach = min(bs, kWave);
  const int base = (int)(run % runs_per_row) * span;
  const float* x = scores + row * row_stride;
  float m = -__builtin_inff();
  if (base + lane < length) m = fmaxf(m, x[base + lane]);
  if (span > kWave && base + kWave + lane < length) m = fmaxf(m, x[base + kWave + lane]);
  for (int off = 1; off < reach; off <<= 1) m = fmaxf(m, __shfl_xor(m, off, kWave));
  const int nb = (length + bs - 1) / bs;
  const int block = (base + lane) / bs;
  if (lane % reach == 0 && block < nb) out[row * nb + block] = m;
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
// Everything is float64 and the result is scaled by kRadiusRoundUp (which
// also covers the summation order).  A workgroup takes a run of whole blocks
// (256 keys, or one block when blocks are longer): the head sums from 16-byte
// query loads (four threads per head), the float64 norm of each key row by
// sixteen lanes, each block's largest norm, then one thread per block the
// margin.
constexpr double kScoreRoundingAllowance = 0x1p-15;
constexpr int kMarginThreads = 256;
constexpr int kMaxMarginBlock = 4096;  // keys per block the entry point accepts

__device__ __forceinline__ double half_to_double(uint32_t bits16, int dtype) {
  return dtype == kBF16 ? (double)__uint_as_float(bits16 << 16)
                        : (double)(float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// Sum of squares of the 8 halves of v, added to acc in order.
__device__ __forceinline__ double sum_squares8(uint4 v, int dtype, double acc) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const double lo = half_to_double(w[i] & 0xffffu, dtype);
    const double hi = half_to_double(w[i] >> 16, dtype);
    acc = fma(lo, lo, acc);
    acc = fma(hi, hi, acc);
  }
  return acc;
}

// kFp8: keys are fp8 e4m3fn rows (128 bytes) with one fp32 scale per 128
// keys; a key's norm is scale * ||k8|| (the key the scoring kernel scores is
// scale * k8), the fp8 values being exact in float64.
template <bool kFp8>
__global__ __launch_bounds__(kMarginThreads) void certified_margins_kernel(const uint16_t* q_now, const uint16_t* q_prev,
                                                                           const float* w_now, const float* w_prev,
                                                                           const void* keys, const float* scales,
                                                                           int64_t key_stride, int prev_length,
                                                                           int block_size, int blocks_per_row,
                                                                           int blocks_per_wg, int q_dtype,
                                                                           double* margins) {
  __shared__ double s_radius[kHeads];
  __shared__ double s_slack[kHeads];
  __shared__ double s_total[2];
  __shared__ unsigned long long s_block_max[kMarginThreads];  // blocks_per_wg <= kMarginThreads
  const int row = blockIdx.y;
  const int tid = threadIdx.x;
  {
    // Head sums: thread t takes head t / 4, dims [32 (t % 4), 32 (t % 4) + 32).
    const int h = tid >> 2;
    const int part = tid & 3;
    const size_t at = ((size_t)row * kHeads + h) * kHeadDim + 32 * part;
    const uint4* pp = reinterpret_cast<const uint4*>(q_prev + at);
    const uint4* pn = reinterpret_cast<const uint4*>(q_now + at);
    double prev_sq = 0.0, now_sq = 0.0, diff_sq = 0.0;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const uint4 a = pp[v];
      const uint4 c = pn[v];
      const uint32_t wa[4] = {a.x, a.y, a.z, a.w};
      const uint32_t wc[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const double p = half_to_double((wa[i >> 1] >> (16 * (i & 1))) & 0xffffu, q_dtype);
        const double n = half_to_double((wc[i >> 1] >> (16 * (i & 1))) & 0xffffu, q_dtype);
        prev_sq = fma(p, p, prev_sq);
        now_sq = fma(n, n, now_sq);
        diff_sq = fma(n - p, n - p, diff_sq);
      }
    }
#pragma unroll
    for (int off = 1; off < 4; off <<= 1) {
      prev_sq += __shfl_xor(prev_sq, off, kWave);
      now_sq += __shfl_xor(now_sq, off, kWave);
      diff_sq += __shfl_xor(diff_sq, off, kWave);
    }
    if (part == 0) {
      const double wn = (double)w_now[(size_t)row * kHeads + h];
      const double wp = (double)w_prev[(size_t)row * kHeads + h];
      s_radius[h] = fabs(wn - wp) * sqrt(prev_sq) + fabs(wn) * sqrt(diff_sq);
      s_slack[h] = fabs(wn) * sqrt(now_sq) + fabs(wp) * sqrt(prev_sq);
    }
  }
  // Key norms of the workgroup's blocks (0 past prev_length): sixteen lanes
  // per key row, one 16-byte vector each, so that one load instruction of a
  // wave reads four whole rows; each block's largest norm by a 64-bit LDS
  // maximum (norms are non-negative, so their bits order as their values).
  if (tid < blocks_per_wg) s_block_max[tid] = 0ull;
  const int lane = tid & (kWave - 1);
  const int sub = lane & 15;
  const int first = blockIdx.x * blocks_per_wg * block_size;
  const int count = blocks_per_wg * block_size;
  constexpr int kRowsPerStep = kMarginThreads / 16;  // 16 key rows per workgroup step
  constexpr int kSteps = 8;                           // steps whose loads are in flight together
  const size_t row_bytes = kFp8 ? kHeadDim : kHeadDim * 2;
  const uint8_t* key_row0 = static_cast<const uint8_t*>(keys) + (size_t)row * key_stride * row_bytes;
  const float* row_scales = kFp8 ? scales + (size_t)row * ((key_stride + 127) / 128) : nullptr;
  __syncthreads();
  for (int i0 = 0; i0 < count; i0 += kRowsPerStep * kSteps) {
    uint4 v[kSteps];  // eight key values per lane (bf16 / fp16, or fp8 widened exactly to bf16)
    float sc[kSteps];
#pragma unroll
    for (int j = 0; j < kSteps; ++j) {
      const int key = min(first + min(i0 + kRowsPerStep * j + (tid >> 4), count - 1), prev_length - 1);
      if constexpr (kFp8) {
        v[j] = fp8x8_to_bf16x8(reinterpret_cast<const uint2*>(key_row0 + (size_t)key * row_bytes)[sub]);
        sc[j] = row_scales[key >> 7];
      } else {
        v[j] = reinterpret_cast<const uint4*>(key_row0 + (size_t)key * row_bytes)[sub];
        sc[j] = 1.f;
      }
    }
#pragma unroll
    for (int j = 0; j < kSteps; ++j) {
      const int i = i0 + kRowsPerStep * j + (tid >> 4);
      double acc = sum_squares8(v[j], kFp8 ? (int)kBF16 : q_dtype, 0.0);
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) acc += __shfl_xor(acc, off, kWave);
      const bool mine = sub == 0 && i < count;
      const double norm = first + i < prev_length ? sqrt(acc) * (double)sc[j] : 0.0;
      if (mine)
        __hip_atomic_fetch_max(&s_block_max[i / block_size], (unsigned long long)__double_as_longlong(norm),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }
  // The heads' totals, once per workgroup (wave 0, one head per lane).
  if (tid < kWave) {
    double radius = s_radius[tid];
    double slack = s_slack[tid];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      radius += __shfl_xor(radius, off, kWave);
      slack += __shfl_xor(slack, off, kWave);
    }
    if (tid == 0) {
      s_total[0] = radius;
      s_total[1] = slack;
    }
  }
  __syncthreads();
  if (tid < blocks_per_wg) {
    const int b = blockIdx.x * blocks_per_wg + tid;
    if (b < blocks_per_row) {
      const double best = __longlong_as_double((long long)s_block_max[tid]);
      margins[(size_t)row * blocks_per_row + b] =
          best * (s_total[0] + kScoreRoundingAllowance * s_total[1]) * kRadiusRoundUp;
    }
  }
}

}  // namespace
}  // namespace dsa

using namespace dsa;

extern "C" int dsa_certified_margins(const void* q_now, const void* q_prev, const float* w_now, const float* w_prev,
                                     const void* keys, const float* key_scales, int64_t key_stride, int64_t batch,
                                     int64_t prev_length, int32_t block_size, int32_t key_dtype, double* margins,
                                     void* stream) {
  DSA_REQUIRE(q_now && q_prev && w_now && w_prev && keys && margins, "null pointer argument");
  DSA_REQUIRE(key_dtype != kFP8E4M3 || key_scales, "fp8 keys need key_scales");
  DSA_REQUIRE(batch > 0 && batch <= 65535, "batch %lld out of range", (long long)batch);
  DSA_REQUIRE(prev_length > 0 && prev_length <= key_stride && prev_length < (int64_t(1) << 31),
              "prev_length %lld invalid", (long long)prev_length);
  DSA_REQUIRE(block_size > 0, "block_size must be positive");
  DSA_REQUIRE(key_dtype == kBF16 || key_dtype == kF16 || key_dtype == kFP8E4M3,
              "certified margins take bf16/fp16 keys (queries of the same dtype) or fp8 keys (bf16 queries)");
  DSA_REQUIRE(block_size <= kMaxMarginBlock, "block_size %d above %d", block_size, kMaxMarginBlock);
  DSA_REQUIRE(reinterpret_cast<uintptr_t>(keys) % 16 == 0 && reinterpret_cast<uintptr_t>(q_now) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(q_prev) % 16 == 0,
              "queries and keys must be 16-byte aligned");
  const int64_t blocks = (prev_length + block_size - 1) / block_size;
  const int per_wg = block_size < kMarginThreads ? kMarginThreads / block_size : 1;
  const dim3 grid((unsigned)((blocks + per_wg - 1) / per_wg), (unsigned)batch);
  auto go = [&](auto kernel, int q_dtype) {
    hipLaunchKernelGGL(kernel, grid, dim3(kMarginThreads), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint16_t*>(q_now), static_cast<const uint16_t*>(q_prev), w_now, w_prev, keys,
                       key_scales, key_stride, (int)prev_length, (int)block_size, (int)blocks, per_wg, q_dtype,
                       margins);
  };
  if (key_dtype == kFP8E4M3)
    go(certified_margins_kernel<true>, (int)kBF16);
  else
    go(certified_margins_kernel<false>, (int)key_dtype);
  return check_launch("certified_margins_kernel");
}

extern "C" int dsa_block_max(const float* scores, int64_t rows, int64_t length,
                             int64_t row_stride, int32_t block_size, float* out, void* stream) {
  DSA_REQUIRE(scores && out, "null pointer argument");
  DSA_REQUIRE(rows > 0 && length > 0 && length < (int64_t(1) << 31), "bad shape");
  DSA_REQUIRE(row_stride >= length, "row_stride < length");
  DSA_REQUIRE(block_size > 0, "block_size must be positive");
  const int64_t nb = (length + block_size - 1) / block_size;
  if (block_size <= 2 * kWave && (block_size & (block_size - 1)) == 0) {
    const int64_t span = block_size > kWave ? 2 * kWave : kWave;
    const int64_t runs = (length + span - 1) / span;
    const int64_t waves = rows * runs;
    DSA_REQUIRE((waves + 3) / 4 < (int64_t(1) << 31), "too many score rows");
    hipLaunchKernelGGL(block_max_runs_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), scores, rows, (int)length, row_stride, (int)block_size,
                       (int)runs, out);
    return check_launch("block_max_runs_kernel");
  }
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
