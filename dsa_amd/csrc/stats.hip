// Statistics of consecutive score rows for the replay analysis tables
// (reference replay.py:403-474: temporal_stats and block_temporal_stats).
//
//   pair_moments_kernel    float64 means and centered second moments of two
//                          rows and of their float32 difference (Pearson's r
//                          and the drift's mean / std), |difference| per key
//   average_ranks_kernel   0-based ascending ranks with ties sharing the mean
//                          of their positions, from a descending sort
//   index_overlap_kernel   |A ∩ B| of two ascending index lists
//   block_streaks_kernel   per block: consecutive steps with the block
//                          maximum below the k-th largest score, the drift of
//                          the block maxima, and the blocks cold for at least
//                          1, 2, 4 and 8 steps
//
// One workgroup per call for the moments (a row is at most a few hundred
// thousand keys); the others are grid-stride.  All sums are float64 with the
// two-pass (mean first) form.
#include "common.hpp"
#include "status.hpp"
#include "waveops.hpp"

namespace dsa {
namespace {

constexpr int kStatThreads = 1024;
constexpr int kStatWaves = kStatThreads / kWave;

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Sum over the workgroup; every thread gets the total.  `red` holds
// kStatWaves doubles and is free again after the call's second barrier.
__device__ __forceinline__ double block_sum_f64(double v, double* red) {
  v = wave_sum_f64(v);
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) red[wave] = v;
  __syncthreads();
  double total = 0.0;
#pragma unroll
  for (int w = 0; w < kStatWaves; ++w) total += red[w];
  __syncthreads();
  return total;
}

template <class T>
__device__ __forceinline__ double difference(T x, T y) {
  if constexpr (sizeof(T) == 4) return (double)(y - x);  // float32 rows subtract in float32
  return (double)y - (double)x;
}

// out: mean x, mean y, sum (x - mx)^2, sum (y - my)^2, sum (x - mx)(y - my),
// mean d, sum (d - md)^2 with d = y - x; abs_delta[i] = |d_i| (nullable).
template <class T>
__global__ __launch_bounds__(kStatThreads) void pair_moments_kernel(const T* x, const T* y, int64_t n, double* out,
                                                                    T* abs_delta) {
  __shared__ double red[kStatWaves];
  double sx = 0.0, sy = 0.0, sd = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += kStatThreads) {
    sx += (double)x[i];
    sy += (double)y[i];
    sd += difference(x[i], y[i]);
  }
  const double mx = block_sum_f64(sx, red) / (double)n;
  const double my = block_sum_f64(sy, red) / (double)n;
  const double md = block_sum_f64(sd, red) / (double)n;
  double sxx = 0.0, syy = 0.0, sxy = 0.0, sdd = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += kStatThreads) {
    const double a = (double)x[i] - mx;
    const double b = (double)y[i] - my;
    const double d = difference(x[i], y[i]);
    sxx += a * a;
    syy += b * b;
    sxy += a * b;
    sdd += (d - md) * (d - md);
    if (abs_delta) abs_delta[i] = (T)fabs(d);
  }
  sxx = block_sum_f64(sxx, red);
  syy = block_sum_f64(syy, red);
  sxy = block_sum_f64(sxy, red);
  sdd = block_sum_f64(sdd, red);
  if (threadIdx.x == 0) {
    out[0] = mx;
    out[1] = my;
    out[2] = sxx;
    out[3] = syy;
    out[4] = sxy;
    out[5] = md;
    out[6] = sdd;
  }
}

// sorted: the row in descending order (ties in any order), order[i] the key
// at position i.  A run of equal values at descending positions [i0, i1)
// holds ascending positions [n - i1, n - i0), whose mean is the rank.
template <class T>
__global__ __launch_bounds__(256) void average_ranks_kernel(const T* sorted, const int64_t* order, int64_t n,
                                                            double* ranks) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const T v = sorted[i];
    int64_t lo = 0, hi = i;  // first position holding v: sorted[p] <= v
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (sorted[mid] > v) lo = mid + 1; else hi = mid;
    }
    const int64_t i0 = lo;
    lo = i + 1;
    hi = n;  // first position past the run: sorted[p] < v
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (sorted[mid] < v) hi = mid; else lo = mid + 1;
    }
    const int64_t i1 = lo;
    ranks[order[i]] = 0.5 * (double)((n - i1) + (n - i0) - 1);
  }
}

__global__ __launch_bounds__(256) void index_overlap_kernel(const int64_t* a, const int64_t* b, int64_t k,
                                                            uint32_t* out) {
  uint32_t hits = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < k; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t x = b[i];
    if (x < 0) continue;
    int64_t lo = 0, hi = k;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      const int64_t m = a[mid];
      if (m >= 0 && m < x) lo = mid + 1; else hi = mid;  // -1 padding sits at the end
    }
    hits += (lo < k && a[lo] == x) ? 1u : 0u;
  }
  hits = (uint32_t)wave_sum_f64((double)hits);
  if ((threadIdx.x & (kWave - 1)) == 0 && hits)
    __hip_atomic_fetch_add(out, hits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ __launch_bounds__(256) void block_streaks_kernel(const float* prev_max, const float* cur_max,
                                                            int64_t blocks, const float* threshold, int32_t* streak,
                                                            double* delta, uint32_t* counts) {
  const float tau = *threshold;
  uint32_t c[4] = {0u, 0u, 0u, 0u};
  for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < blocks;
       b += (int64_t)gridDim.x * blockDim.x) {
    const float m = cur_max[b];
    const int32_t s = m < tau ? streak[b] + 1 : 0;
    streak[b] = s;
    delta[b] = (double)m - (double)prev_max[b];
    c[0] += s >= 1 ? 1u : 0u;
    c[1] += s >= 2 ? 1u : 0u;
    c[2] += s >= 4 ? 1u : 0u;
    c[3] += s >= 8 ? 1u : 0u;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t total = (uint32_t)wave_sum_f64((double)c[j]);
    if ((threadIdx.x & (kWave - 1)) == 0 && total)
      __hip_atomic_fetch_add(&counts[j], total, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

int grid_for(int64_t n) { return (int)((n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024); }

}  // namespace
}  // namespace dsa

using namespace dsa;

extern "C" int dsa_pair_moments(const void* x, const void* y, int32_t dtype, int64_t n, double* out,
                                void* abs_delta, void* stream) {
  DSA_REQUIRE(x && y && out, "null pointer argument");
  DSA_REQUIRE(n > 0, "n must be positive");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == DSA_DTYPE_F32)
    hipLaunchKernelGGL(pair_moments_kernel<float>, dim3(1), dim3(kStatThreads), 0, s,
                       static_cast<const float*>(x), static_cast<const float*>(y), n, out,
                       static_cast<float*>(abs_delta));
  else if (dtype == DSA_DTYPE_F64)
    hipLaunchKernelGGL(pair_moments_kernel<double>, dim3(1), dim3(kStatThreads), 0, s,
                       static_cast<const double*>(x), static_cast<const double*>(y), n, out,
                       static_cast<double*>(abs_delta));
  else
    return fail(DSA_STATUS_INVALID_ARGUMENT, "dsa_pair_moments takes fp32 or fp64 rows (got %d)", dtype);
  return check_launch("pair_moments_kernel");
}

extern "C" int dsa_average_ranks(const void* sorted, int32_t dtype, const int64_t* order, int64_t n, double* ranks,
                                 void* stream) {
  DSA_REQUIRE(sorted && order && ranks, "null pointer argument");
  DSA_REQUIRE(n > 0, "n must be positive");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == DSA_DTYPE_F32)
    hipLaunchKernelGGL(average_ranks_kernel<float>, dim3(grid_for(n)), dim3(256), 0, s,
                       static_cast<const float*>(sorted), order, n, ranks);
  else if (dtype == DSA_DTYPE_F64)
    hipLaunchKernelGGL(average_ranks_kernel<double>, dim3(grid_for(n)), dim3(256), 0, s,
                       static_cast<const double*>(sorted), order, n, ranks);
  else
    return fail(DSA_STATUS_INVALID_ARGUMENT, "dsa_average_ranks takes fp32 or fp64 rows (got %d)", dtype);
  return check_launch("average_ranks_kernel");
}

extern "C" int dsa_index_overlap(const int64_t* a, const int64_t* b, int64_t k, uint32_t* out, void* stream) {
  DSA_REQUIRE(a && b && out, "null pointer argument");
  DSA_REQUIRE(k > 0, "k must be positive");
  hipLaunchKernelGGL(index_overlap_kernel, dim3(grid_for(k)), dim3(256), 0, static_cast<hipStream_t>(stream), a, b,
                     k, out);
  return check_launch("index_overlap_kernel");
}

extern "C" int dsa_block_streaks(const float* prev_max, const float* cur_max, int64_t blocks, const float* threshold,
                                 int32_t* streak, double* delta, uint32_t* counts, void* stream) {
  DSA_REQUIRE(prev_max && cur_max && threshold && streak && delta && counts, "null pointer argument");
  DSA_REQUIRE(blocks > 0, "blocks must be positive");
  hipLaunchKernelGGL(block_streaks_kernel, dim3(grid_for(blocks)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     prev_max, cur_max, blocks, threshold, streak, delta, counts);
  return check_launch("block_streaks_kernel");
}
