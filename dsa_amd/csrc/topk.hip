// Exact top-k with stable_topk semantics (reference metrics.py:9-22): the k
// largest values, ties at the cut-off go to the lower index.
//
// One 1024-thread workgroup per (virtual) row.  Thread t owns the contiguous
// slice [t * EPT, t * EPT + EPT) of the row in registers, so a single
// exclusive scan over threads enumerates elements in index order.  Selection is
// a 3-pass MSD radix select (11 + 11 + 10 bits) over order-preserving uint32
// keys with a 2048-bin LDS histogram per pass; it yields the exact k-th value
// v* and the number of elements equal to v* that still have to be taken.  The
// chosen elements are then written in index order, or bitonic-sorted in LDS by
// (value desc, index asc) when a sorted result is requested.
#include "common.hpp"
#include "status.hpp"

namespace dsa {
namespace {

constexpr int kTopkThreads = 1024;
constexpr int kTopkWaves = kTopkThreads / kWave;
constexpr int kMaxK = 4096;
constexpr int kBins = 2048;

struct TopkArgs {
  const float* scores;
  const int64_t* in_idx;
  int64_t row_stride;
  const int32_t* row_lengths;
  int32_t length;
  int32_t chunks;     // virtual rows per row
  int32_t chunk_len;  // elements per virtual row
  int32_t k;
  int32_t sorted;
  int64_t* out_idx;
  float* out_val;
};

struct TopkShared {
  uint32_t hist[kBins];
  uint32_t wave_sums[kTopkWaves];
  uint32_t digit;
  uint32_t krem;
  uint64_t sort_keys[kMaxK];
};

// Exclusive prefix sum over the workgroup in thread order; returns the total
// through `total`.  Contains two barriers.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* wave_sums,
                                                         uint32_t& total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t y = __shfl_up(x, off, kWave);
    if (lane >= off) x += y;
  }
  if (lane == 63) wave_sums[wave] = x;
  __syncthreads();
  uint32_t before = 0;
  uint32_t all = 0;
#pragma unroll
  for (int i = 0; i < kTopkWaves; ++i) {
    const uint32_t s = wave_sums[i];
    before += i < wave ? s : 0u;
    all += s;
  }
  __syncthreads();
  total = all;
  return before + x - v;
}

template <int EPT>
__global__ __launch_bounds__(kTopkThreads) void topk_kernel(TopkArgs a) {
  __shared__ TopkShared sh;
  const int tid = threadIdx.x;
  const int64_t v = blockIdx.x;
  const int64_t row = v / a.chunks;
  const int chunk = (int)(v % a.chunks);
  int row_len = a.length;
  if (a.row_lengths) row_len = min(row_len, max(0, a.row_lengths[row]));
  const int start = chunk * a.chunk_len;
  const int n = max(0, min(a.chunk_len, row_len - start));
  const int64_t base = row * a.row_stride + start;
  const int k = a.k;
  const int64_t out_base = v * (int64_t)k;

  // Load this thread's slice as ordered keys; 0 marks an invalid slot.
  uint32_t key[EPT];
  const int e0 = tid * EPT;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const int pos = e0 + e;
    uint32_t kv = 0;
    if (pos < n) {
      bool ok = true;
      if (a.in_idx) ok = a.in_idx[base + pos] >= 0;
      if (ok) kv = float_to_ordered(a.scores[base + pos]);
    }
    key[e] = kv;
  }

  // Chosen: key > threshold, or key == threshold within the first krem ties.
  // With threshold 1 and unlimited krem every valid slot is chosen (n <= k).
  uint32_t threshold = 1;
  uint32_t krem = 0xffffffffu;
  if (n > k) {
    uint32_t prefix = 0;
    uint32_t prefix_mask = 0;
    uint32_t want = (uint32_t)k;
#pragma unroll 1
    for (int pass = 0; pass < 3; ++pass) {
      const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
      const uint32_t dmask = pass == 2 ? 0x3ffu : 0x7ffu;
      for (int i = tid; i < kBins; i += kTopkThreads) sh.hist[i] = 0;
      if (tid == 0) {
        sh.digit = 0;
        sh.krem = 1;
      }
      __syncthreads();
#pragma unroll
      for (int e = 0; e < EPT; ++e)
        if (key[e] != 0 && (key[e] & prefix_mask) == prefix)
          atomicAdd(&sh.hist[(key[e] >> shift) & dmask], 1u);
      __syncthreads();
      // Thread t owns bins 2t and 2t+1; find the digit holding the want-th
      // largest via a suffix count (total minus inclusive prefix).
      const uint32_t c0 = sh.hist[2 * tid];
      const uint32_t c1 = sh.hist[2 * tid + 1];
      uint32_t total;
      const uint32_t before = block_exclusive_scan(c0 + c1, sh.wave_sums, total);
      const uint32_t above1 = total - before - c0 - c1;  // count in bins > 2t+1
      const uint32_t above0 = above1 + c1;               // count in bins > 2t
      if (c1 && above1 < want && want <= above1 + c1) {
        sh.digit = 2 * tid + 1;
        sh.krem = want - above1;
      }
      if (c0 && above0 < want && want <= above0 + c0) {
        sh.digit = 2 * tid;
        sh.krem = want - above0;
      }
      __syncthreads();
      prefix |= sh.digit << shift;
      prefix_mask |= dmask << shift;
      want = sh.krem;
      __syncthreads();
    }
    threshold = prefix;  // exact key of the k-th largest
    krem = want;         // elements equal to it that are taken (lowest index first)
  }

  // Selection in index order: rank the ties, count the chosen elements per
  // thread, then walk the slice again placing (key, ~position) of each chosen
  // element at its rank in LDS.  threshold >= 1, so invalid slots (key 0) are
  // never chosen.
  uint32_t n_eq = 0;
#pragma unroll
  for (int e = 0; e < EPT; ++e) n_eq += key[e] == threshold ? 1u : 0u;
  uint32_t eq_total;
  const uint32_t eq_rank0 = block_exclusive_scan(n_eq, sh.wave_sums, eq_total);
  uint32_t n_sel = 0;
  {
    uint32_t eq_rank = eq_rank0;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const bool eq = key[e] == threshold;
      n_sel += (key[e] > threshold || (eq && eq_rank < krem)) ? 1u : 0u;
      eq_rank += eq ? 1u : 0u;
    }
  }
  uint32_t sel_total;
  const uint32_t pos0 = block_exclusive_scan(n_sel, sh.wave_sums, sel_total);
  // The selection yields exactly min(n, k) elements; the clamp only guards the
  // buffers should that invariant ever break.
  sel_total = min(sel_total, (uint32_t)k);
  {
    uint32_t eq_rank = eq_rank0;
    uint32_t p = pos0;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const bool eq = key[e] == threshold;
      if (key[e] > threshold || (eq && eq_rank < krem)) {
        if (p < sel_total) sh.sort_keys[p] = (uint64_t(key[e]) << 32) | (uint64_t)(~(uint32_t)(e0 + e));
        ++p;
      }
      eq_rank += eq ? 1u : 0u;
    }
  }
  __syncthreads();

  if (a.sorted) {
    int width = 1;
    while (width < (int)sel_total) width <<= 1;
    for (int i = (int)sel_total + tid; i < width; i += kTopkThreads) sh.sort_keys[i] = 0;
    __syncthreads();
    // Bitonic sort, descending on (key, ~position).
    for (int size = 2; size <= width; size <<= 1) {
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int i = tid; i < (width >> 1); i += kTopkThreads) {
          const int lo = 2 * i - (i & (stride - 1));
          const int hi = lo + stride;
          const uint64_t x = sh.sort_keys[lo];
          const uint64_t y = sh.sort_keys[hi];
          const bool desc = (lo & size) == 0;
          if (desc ? (x < y) : (x > y)) {
            sh.sort_keys[lo] = y;
            sh.sort_keys[hi] = x;
          }
        }
        __syncthreads();
      }
    }
  }
  for (int i = tid; i < (int)sel_total; i += kTopkThreads) {
    const uint32_t pos = ~(uint32_t)(sh.sort_keys[i] & 0xffffffffu);
    if (a.out_idx) a.out_idx[out_base + i] = a.in_idx ? a.in_idx[base + pos] : (int64_t)(start + pos);
    if (a.out_val) a.out_val[out_base + i] = a.scores[base + pos];
  }
  // Padding when fewer than k valid entries exist.
  for (int i = (int)sel_total + tid; i < k; i += kTopkThreads) {
    if (a.out_idx) a.out_idx[out_base + i] = -1;
    if (a.out_val) a.out_val[out_base + i] = -__builtin_inff();
  }
}

int launch_topk(const TopkArgs& a, int64_t virtual_rows, hipStream_t stream) {
  const int n = a.chunk_len;
  const dim3 grid((unsigned)virtual_rows);
  const dim3 block(kTopkThreads);
  if (n <= kTopkThreads * 4) hipLaunchKernelGGL(topk_kernel<4>, grid, block, 0, stream, a);
  else if (n <= kTopkThreads * 8) hipLaunchKernelGGL(topk_kernel<8>, grid, block, 0, stream, a);
  else if (n <= kTopkThreads * 16) hipLaunchKernelGGL(topk_kernel<16>, grid, block, 0, stream, a);
  else hipLaunchKernelGGL(topk_kernel<32>, grid, block, 0, stream, a);
  return check_launch("topk_kernel");
}

constexpr int64_t kMaxRowLen = int64_t(kTopkThreads) * 32;
constexpr int64_t kLongChunk = 32768;

}  // namespace
}  // namespace dsa

using namespace dsa;

extern "C" int dsa_topk(const float* scores, const int64_t* in_indices, int64_t rows,
                        int64_t length, int64_t row_stride, const int32_t* row_lengths, int64_t k,
                        int32_t sorted, int64_t* out_indices, float* out_values, void* stream) {
  DSA_REQUIRE(scores, "scores must be non-null");
  DSA_REQUIRE(rows > 0 && rows < (int64_t(1) << 31), "rows %lld out of range", (long long)rows);
  DSA_REQUIRE(length > 0 && length <= kMaxRowLen, "length %lld outside [1, %lld]",
              (long long)length, (long long)kMaxRowLen);
  DSA_REQUIRE(row_stride >= length, "row_stride %lld < length %lld", (long long)row_stride,
              (long long)length);
  DSA_REQUIRE(k > 0 && k <= kMaxK, "k=%lld outside [1, %d]", (long long)k, kMaxK);
  TopkArgs a;
  a.scores = scores;
  a.in_idx = in_indices;
  a.row_stride = row_stride;
  a.row_lengths = row_lengths;
  a.length = (int32_t)length;
  a.chunks = 1;
  a.chunk_len = (int32_t)length;
  a.k = (int32_t)k;
  a.sorted = sorted ? 1 : 0;
  a.out_idx = out_indices;
  a.out_val = out_values;
  return launch_topk(a, rows, static_cast<hipStream_t>(stream));
}

extern "C" int64_t dsa_topk_long_workspace_bytes(int64_t rows, int64_t length, int64_t k) {
  if (rows <= 0 || length <= 0 || k <= 0) return 0;
  const int64_t chunks = (length + kLongChunk - 1) / kLongChunk;
  return rows * chunks * k * (int64_t)(sizeof(int64_t) + sizeof(float));
}

extern "C" int dsa_topk_long(const float* scores, int64_t rows, int64_t length, int64_t k,
                             int32_t sorted, int64_t* out_indices, float* out_values,
                             void* workspace, int64_t workspace_bytes, void* stream) {
  DSA_REQUIRE(scores, "scores must be non-null");
  DSA_REQUIRE(rows > 0 && rows < (int64_t(1) << 31), "rows %lld out of range", (long long)rows);
  DSA_REQUIRE(length > 0 && length < (int64_t(1) << 31), "length %lld out of range",
              (long long)length);
  DSA_REQUIRE(k > 0 && k <= kMaxK, "k=%lld outside [1, %d]", (long long)k, kMaxK);
  const int64_t chunks = (length + kLongChunk - 1) / kLongChunk;
  DSA_REQUIRE(chunks * k <= kMaxRowLen, "length %lld too long for k=%lld", (long long)length,
              (long long)k);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (chunks == 1) return dsa_topk(scores, nullptr, rows, length, length, nullptr, k, sorted,
                                   out_indices, out_values, stream);
  const int64_t need = dsa_topk_long_workspace_bytes(rows, length, k);
  if (!workspace || workspace_bytes < need)
    return fail(DSA_STATUS_WORKSPACE_TOO_SMALL, "topk_long needs %lld workspace bytes",
                (long long)need);
  int64_t* cand_idx = static_cast<int64_t*>(workspace);
  float* cand_val = reinterpret_cast<float*>(cand_idx + rows * chunks * k);
  // Stage 1: every chunk's local top-k, in index order, padded with -1.
  TopkArgs a;
  a.scores = scores;
  a.in_idx = nullptr;
  a.row_stride = length;
  a.row_lengths = nullptr;
  a.length = (int32_t)length;
  a.chunks = (int32_t)chunks;
  a.chunk_len = (int32_t)kLongChunk;
  a.k = (int32_t)k;
  a.sorted = 0;
  a.out_idx = cand_idx;
  a.out_val = cand_val;
  if (int st = launch_topk(a, rows * chunks, s)) return st;
  // Stage 2: exact merge of the candidates (ties break on the global index).
  return dsa_topk(cand_val, cand_idx, rows, chunks * k, chunks * k, nullptr, k, sorted,
                  out_indices, out_values, stream);
}
