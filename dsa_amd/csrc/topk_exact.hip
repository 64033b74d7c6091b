// Exact stable top-k of arbitrary score rows with 64-bit order keys: the
// stable_topk rule (reference metrics.py:9-22: every value above the k-th
// largest, then the lowest indices among the values equal to it) for float64
// rows and for float32 rows with any k and any length.
//
// One 1024-thread workgroup per row, three phases:
//   select: an MSB-first radix select over the order-preserving key (8-bit
//           digits; 8 passes for float64, 4 for float32) finds the k-th
//           largest key and how many of the keys equal to it are taken;
//   gather: the row is swept in index order; a packed block scan of
//           (above, equal) flags places every taken index, so the result is
//           in ascending index order;
//   sort:   for sorted output, a stable LSD radix sort of the taken
//           (key, index) pairs by descending key (the index order of equal
//           keys is kept), giving stable_topk's (-value, index) order.
// The phases re-read the row from memory (L2 after the first pass); this is
// the general-purpose path, not the decode step's.
#include "common.hpp"
#include "dsa_amd.h"
#include "status.hpp"
#include "waveops.hpp"

namespace dsa {
namespace {

constexpr int kExactThreads = 1024;
constexpr int kExactWaves = kExactThreads / kWave;
constexpr int kDigits = 256;

// Order-preserving maps: a larger value gives a larger key; -0.0 is folded
// onto +0.0 (numpy compares them equal, so they tie on the index).
__device__ __forceinline__ uint64_t f64_to_ordered(double d) {
  uint64_t u = (uint64_t)__double_as_longlong(d);
  if (u == 0x8000000000000000ull) u = 0ull;
  return (u >> 63) ? ~u : (u | 0x8000000000000000ull);
}

struct ExactArgs {
  const void* values;  // [rows][row_stride] float64 or float32
  int64_t row_stride;
  int32_t length;
  int32_t k;
  int32_t sorted;
  int64_t* out_idx;  // [rows][k]
  void* out_val;     // [rows][k] in the input dtype, or null
  uint64_t* ws_key;  // [rows][2][k] (sorted output only)
  uint32_t* ws_idx;  // [rows][2][k]
};

template <bool kF64>
__device__ __forceinline__ uint64_t key_at(const void* row, int64_t i) {
  if constexpr (kF64) return f64_to_ordered(static_cast<const double*>(row)[i]);
  else return (uint64_t)float_to_ordered(static_cast<const float*>(row)[i]) << 32;
}

// Output values are copied from the input row at the chosen index, bits and
// all, not rebuilt from the order key (which folds -0.0 onto +0.0).
template <bool kF64>
__device__ __forceinline__ void put_value(void* out, int64_t at, const void* row, int64_t i) {
  if constexpr (kF64) static_cast<double*>(out)[at] = static_cast<const double*>(row)[i];
  else static_cast<float*>(out)[at] = static_cast<const float*>(row)[i];
}

struct ExactShared {
  uint32_t hist[kDigits];
  uint32_t base[kDigits];
  uint32_t chunk_total[kDigits];
  uint32_t wave_count[kExactWaves][kDigits];  // per-wave digit counts, then their per-digit prefix
  uint32_t wsum[2][kExactWaves];
  uint32_t digit, rem;
};

template <bool kF64>
__global__ __launch_bounds__(kExactThreads) void topk_exact_kernel(ExactArgs a) {
  __shared__ __align__(16) ExactShared sh;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = lane_id();
  const uint32_t wave = tid / kWave;
  const int64_t row = blockIdx.x;
  const int n = a.length;
  const uint32_t k = (uint32_t)a.k;
  const uint8_t* rbase = static_cast<const uint8_t*>(a.values) + row * a.row_stride * (kF64 ? 8 : 4);
  constexpr int kPasses = kF64 ? 8 : 4;

  // ---- select: the k-th largest key, and how many keys equal to it are taken
  uint64_t prefix = 0ull;
  uint64_t mask = 0ull;
  uint32_t want = k;
#pragma unroll 1
  for (int pass = 0; pass < kPasses; ++pass) {
    const int shift = 56 - 8 * pass;
    if (tid < (uint32_t)kDigits) sh.hist[tid] = 0u;
    __syncthreads();
    for (int i = (int)tid; i < n; i += kExactThreads) {
      const uint64_t key = key_at<kF64>(rbase, i);
      if ((key & mask) == prefix)
        __hip_atomic_fetch_add(&sh.hist[(uint32_t)(key >> shift) & 0xffu], 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    __syncthreads();
    if (wave == 0) {
      const Locate t = wave_locate<kDigits / kWave>(sh.hist, want, false);
      if (lane == 0) {
        sh.digit = t.digit;
        sh.rem = t.rem;
      }
    }
    __syncthreads();
    // (k <= length keeps the digit found; kNoBin cannot occur)
    prefix |= uint64_t(sh.digit & 0xffu) << shift;
    mask |= uint64_t(0xffu) << shift;
    want = sh.rem;
    __syncthreads();  // sh.digit / sh.rem are rewritten by the next pass
  }
  const uint64_t cut = prefix;
  const uint32_t ties = want;  // keys equal to the cut that are taken, lowest indices first

  // ---- gather: every taken key in index order
  uint64_t* key_a = a.ws_key ? a.ws_key + row * 2 * (int64_t)k : nullptr;
  uint32_t* idx_a = a.ws_idx ? a.ws_idx + row * 2 * (int64_t)k : nullptr;
  int64_t* oidx = a.out_idx + row * (int64_t)k;
  uint32_t placed = 0;     // taken so far
  uint32_t eq_seen = 0;    // keys equal to the cut seen so far
#pragma unroll 1
  for (int base = 0; base < n && placed < k; base += kExactThreads) {
    const int i = base + (int)tid;
    const uint64_t key = i < n ? key_at<kF64>(rbase, i) : 0ull;
    const uint32_t gt = (i < n && key > cut) ? 1u : 0u;
    const uint32_t eq = (i < n && key == cut) ? 1u : 0u;
    uint32_t packed_total;
    const uint32_t packed = block_excl_scan<kExactWaves>((eq << 16) | gt, sh.wsum[(base / kExactThreads) & 1],
                                                         packed_total);
    const uint32_t ties_left = ties > eq_seen ? ties - eq_seen : 0u;
    const uint32_t eq_before = packed >> 16;
    const uint32_t take = gt | (eq & (eq_before < ties_left ? 1u : 0u));
    if (take) {
      const uint32_t pos = placed + (packed & 0xffffu) + min(eq_before, ties_left);
      if (pos < k) {  // always true for consistent counts
        if (key_a) {
          key_a[pos] = key;
          idx_a[pos] = (uint32_t)i;
        } else {
          oidx[pos] = i;
          if (a.out_val) put_value<kF64>(a.out_val, row * (int64_t)k + pos, rbase, i);
        }
      }
    }
    placed += (packed_total & 0xffffu) + min(packed_total >> 16, ties_left);
    eq_seen += packed_total >> 16;
  }
  if (!key_a) return;

  // ---- sort: stable LSD radix sort of the k pairs by descending key
  __syncthreads();  // the gather's global writes are read back below by other threads
  __threadfence_block();
  uint64_t* src_k = key_a;
  uint32_t* src_i = idx_a;
  uint64_t* dst_k = key_a + k;
  uint32_t* dst_i = idx_a + k;
  const uint64_t lanes_lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll 1
  for (int pass = 0; pass < kPasses; ++pass) {
    const int shift = (kF64 ? 0 : 32) + 8 * pass;
    if (tid < (uint32_t)kDigits) sh.hist[tid] = 0u;
    __syncthreads();
    for (uint32_t j = tid; j < k; j += kExactThreads)
      __hip_atomic_fetch_add(&sh.hist[(uint32_t)(~src_k[j] >> shift) & 0xffu], 1u, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_WORKGROUP);
    __syncthreads();
    if (wave == 0) {  // exclusive scan of the 256 digit counts, 4 per lane
      uint32_t c[4];
      uint32_t sum = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        c[q] = sh.hist[4 * lane + q];
        sum += c[q];
      }
      uint32_t run = wave_incl_scan(sum) - sum;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        sh.base[4 * lane + q] = run;
        run += c[q];
      }
    }
    __syncthreads();
#pragma unroll 1
    for (uint32_t cbase = 0; cbase < k; cbase += kExactThreads) {
      const uint32_t j = cbase + tid;
      const bool valid = j < k;
      const uint64_t key = valid ? src_k[j] : 0ull;
      const uint32_t idx = valid ? src_i[j] : 0u;
      const uint32_t d = (uint32_t)(~key >> shift) & 0xffu;
      // Lanes of this wave with the same digit, by eight ballots on its bits.
      uint64_t same = __ballot(valid);
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const uint64_t ones = __ballot((d >> b) & 1u);
        same &= ((d >> b) & 1u) ? ones : ~ones;
      }
      for (uint32_t e = tid; e < (uint32_t)(kExactWaves * kDigits); e += kExactThreads)
        (&sh.wave_count[0][0])[e] = 0u;
      __syncthreads();
      if (valid && (same & lanes_lt) == 0ull) sh.wave_count[wave][d] = (uint32_t)__popcll(same);
      __syncthreads();
      if (tid < (uint32_t)kDigits) {  // per digit: exclusive prefix over the waves
        uint32_t run = 0;
        for (int w = 0; w < kExactWaves; ++w) {
          const uint32_t c = sh.wave_count[w][tid];
          sh.wave_count[w][tid] = run;
          run += c;
        }
        sh.chunk_total[tid] = run;
      }
      __syncthreads();
      if (valid) {
        const uint32_t pos = sh.base[d] + sh.wave_count[wave][d] + (uint32_t)__popcll(same & lanes_lt);
        if (pos < k) {  // always true for consistent counts
          dst_k[pos] = key;
          dst_i[pos] = idx;
        }
      }
      __syncthreads();
      if (tid < (uint32_t)kDigits) sh.base[tid] += sh.chunk_total[tid];
      __syncthreads();
    }
    __threadfence_block();
    uint64_t* tk = src_k;
    src_k = dst_k;
    dst_k = tk;
    uint32_t* ti = src_i;
    src_i = dst_i;
    dst_i = ti;
    __syncthreads();
  }
  for (uint32_t j = tid; j < k; j += kExactThreads) {
    oidx[j] = (int64_t)src_i[j];
    if (a.out_val) put_value<kF64>(a.out_val, row * (int64_t)k + j, rbase, src_i[j]);
  }
}

}  // namespace
}  // namespace dsa

using namespace dsa;

extern "C" int64_t dsa_topk_exact_workspace_bytes(int64_t rows, int64_t k, int32_t sorted) {
  if (rows <= 0 || k <= 0 || !sorted) return 0;
  return rows * 2 * k * (int64_t)(sizeof(uint64_t) + sizeof(uint32_t));
}

extern "C" int dsa_topk_exact(const void* values, int32_t value_dtype, int64_t rows, int64_t length,
                              int64_t row_stride, int64_t k, int32_t sorted, int64_t* out_indices,
                              void* out_values, void* workspace, int64_t workspace_bytes, void* stream) {
  DSA_REQUIRE(values && out_indices, "null pointer argument");
  DSA_REQUIRE(value_dtype == DSA_DTYPE_F64 || value_dtype == DSA_DTYPE_F32, "values must be float64 or float32");
  DSA_REQUIRE(rows > 0 && rows <= 0x7fffffff, "rows %lld out of range", (long long)rows);
  DSA_REQUIRE(length > 0 && length <= 0x7fffffff, "length %lld out of range", (long long)length);
  DSA_REQUIRE(row_stride >= length, "row_stride < length");
  DSA_REQUIRE(k > 0 && k <= length, "k=%lld outside [1, length]", (long long)k);
  DSA_REQUIRE(k <= (int64_t(1) << 30), "k=%lld too large", (long long)k);
  const int64_t need = dsa_topk_exact_workspace_bytes(rows, k, sorted);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(DSA_STATUS_WORKSPACE_TOO_SMALL, "sorted output needs %lld workspace bytes", (long long)need);
  DSA_REQUIRE(!workspace || reinterpret_cast<uintptr_t>(workspace) % 16 == 0, "workspace must be 16-byte aligned");
  ExactArgs a;
  a.values = values;
  a.row_stride = row_stride;
  a.length = (int32_t)length;
  a.k = (int32_t)k;
  a.sorted = sorted;
  a.out_idx = out_indices;
  a.out_val = out_values;
  a.ws_key = sorted ? static_cast<uint64_t*>(workspace) : nullptr;
  a.ws_idx = sorted ? reinterpret_cast<uint32_t*>(static_cast<uint64_t*>(workspace) + rows * 2 * k) : nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (value_dtype == DSA_DTYPE_F64)
    hipLaunchKernelGGL(topk_exact_kernel<true>, dim3((unsigned)rows), dim3(kExactThreads), 0, s, a);
  else
    hipLaunchKernelGGL(topk_exact_kernel<false>, dim3((unsigned)rows), dim3(kExactThreads), 0, s, a);
  return check_launch("topk_exact_kernel");
}
