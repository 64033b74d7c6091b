// Exact top-k with stable_topk semantics (reference metrics.py:9-22): the k
// largest values, ties at the cut-off go to the lower index.
//
// One workgroup per (virtual) row: 1024 threads, or 256 when many short rows
// (at most 4096 entries) make throughput matter more than latency.  Thread t owns the contiguous
// slice [t * ept, t * ept + ept) of the row in registers (ept <= EPT, sized to
// the row's length), so a single exclusive scan over threads enumerates
// elements in index order.  The k-th
// largest (value, index) pair is found by a value-linear bucket select whose
// crowded-bucket or degenerate cases fall back to an exact radix select; the
// chosen elements are written in index order, or bitonic-sorted in LDS by
// (value desc, index asc) when a sorted result is requested.
#include "common.hpp"
#include "select.hpp"
#include "status.hpp"

namespace dsa {
namespace {

constexpr int kTopkThreads = 1024;  // widest workgroup (long rows)
constexpr int kMaxK = 4096;
constexpr int kSmallCap = 1024;  // candidate buffer of the short-row kernel
constexpr int kBins = 2048;

#ifdef DSA_PHASE_TRACE
// Per workgroup (by blockIdx.x): 0 start, 1 row loaded, 2 range known,
// 3 cut located, 4 cut resolved, 5 output slots scanned, 6 written.
__device__ uint64_t g_trace_topk[kTraceWgs * kTraceMarks];
#endif

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
  const uint32_t* skip;  // [rows] or null: rows with a nonzero flag are left as they are
};

template <int THREADS, int CAP>
struct TopkShared {
  static constexpr int kWaves = THREADS / kWave;
  uint32_t hist[kBins];
  uint32_t wave_sums[kWaves];
  uint32_t wave_valid[kWaves];
  float wave_lo[kWaves];
  float wave_hi[kWaves];
  uint32_t digit;
  uint32_t krem;
  uint64_t cstar;
  uint64_t sort_keys[CAP + 1];  // slot CAP is a write sink for unchosen lanes
};

// Exclusive prefix sum over the workgroup in thread order; returns the total
// through `total`.  Contains two barriers.
template <int WAVES>
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* wave_sums,
                                                         uint32_t& total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t y = __shfl_up(x, off, kWave);
    x += lane >= off ? y : 0u;
  }
  if (lane == 63) wave_sums[wave] = x;
  __syncthreads();
  uint32_t before = 0;
  uint32_t all = 0;
#pragma unroll
  for (int i = 0; i < WAVES; ++i) {
    const uint32_t s = wave_sums[i];
    before += i < wave ? s : 0u;
    all += s;
  }
  __syncthreads();
  total = all;
  return before + x - v;
}

// Bitonic sort of keys[0, width) in descending order (width a power of two).
template <int THREADS>
__device__ __forceinline__ void bitonic_sort_desc(uint64_t* keys, int width) {
  const int tid = threadIdx.x;
  for (int size = 2; size <= width; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = tid; i < (width >> 1); i += THREADS) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const uint64_t x = keys[lo];
        const uint64_t y = keys[hi];
        const bool desc = (lo & size) == 0;
        const bool swap = desc ? (x < y) : (x > y);
        keys[lo] = swap ? y : x;
        keys[hi] = swap ? x : y;
      }
      __syncthreads();
    }
  }
}

__device__ __forceinline__ void lds_add(uint32_t* p, uint32_t v) {
  __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Rank key of an element: (ordered value, ~position).  Larger is better; all
// composites of a row are distinct.
__device__ __forceinline__ uint64_t composite(uint32_t key, int pos) {
  return (uint64_t(key) << 32) | (uint64_t)(~(uint32_t)pos);
}

// Value-linear bucket of an ordered key: monotone non-decreasing in the value
// (the subtraction, the positive scaling and the truncation are all monotone
// in IEEE arithmetic), so equal values share a bucket and a larger bucket
// always holds strictly larger values.
__device__ __forceinline__ int value_bucket(uint32_t key, float lo, float scale) {
  const float f = ordered_to_float(key);
  const float x = (f - lo) * scale;  // -inf -> -inf, finite >= 0
  return (int)fminf(fmaxf(x, 0.f), (float)(kBins - 1));
}

// Finds the bin holding the want-th largest element of the histogram in
// sh.hist; leaves it in sh.digit and the remaining rank inside it in sh.krem.
// Thread t scans bins [t * B, t * B + B), B = kBins / THREADS.
template <int THREADS, int CAP>
__device__ __forceinline__ void locate_bin(TopkShared<THREADS, CAP>& sh, uint32_t want) {
  constexpr int B = kBins / THREADS;
  const int tid = threadIdx.x;
  uint32_t c[B];
  uint32_t mine = 0;
#pragma unroll
  for (int i = 0; i < B; ++i) {
    c[i] = sh.hist[B * tid + i];
    mine += c[i];
  }
  uint32_t total;
  const uint32_t before = block_exclusive_scan<THREADS / kWave>(mine, sh.wave_sums, total);
  uint32_t above = total - before - mine;  // elements in bins above this thread's
#pragma unroll
  for (int i = B - 1; i >= 0; --i) {
    if (c[i] && above < want && want <= above + c[i]) {
      sh.digit = B * tid + i;
      sh.krem = want - above;
    }
    above += c[i];
  }
  __syncthreads();
}

// The k largest of a row, ties at the cut-off to the lower position.  Every
// element is ranked by its composite; the chosen set is exactly the composites
// >= cstar, the k-th largest composite, which is found by
//   1. a bucket select: value-linear buckets between the row's finite min and
//      max; the bucket T holding the k-th largest is read off a histogram, its
//      (few) candidates are sorted in LDS and cstar is the need-th of them; or
//   2. when the row has no finite spread or bucket T is too crowded: an
//      11+11+10-bit radix select over the ordered keys for the k-th value,
//      whose ties are ranked by position with a prefix scan.
// All per-element work is branch-free (predicated adds and sink-slot writes).
template <int THREADS, int EPT, int CAP>
__global__ __launch_bounds__(THREADS) void topk_kernel(TopkArgs a) {
  constexpr int kWaves = THREADS / kWave;
  __shared__ TopkShared<THREADS, CAP> sh;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // Last virtual rows first: under causal row lengths they are the longest.
  const int64_t v = (int64_t)gridDim.x - 1 - blockIdx.x;
  const int64_t row = v / a.chunks;
  const int chunk = (int)(v % a.chunks);
  if (a.skip && a.skip[row]) return;
  int row_len = a.length;
  if (a.row_lengths) row_len = min(row_len, max(0, a.row_lengths[row]));
  const int start = chunk * a.chunk_len;
  const int n = max(0, min(a.chunk_len, row_len - start));
  const int64_t base = row * a.row_stride + start;
  const int k = a.k;
  const int64_t out_base = v * (int64_t)k;
  DSA_TRACE_MARK(g_trace_topk, blockIdx.x, 0);

  // Load this thread's slice as ordered keys; 0 marks an invalid slot.  The
  // buffer bounds check turns reads past n into zeros, which are masked.
  // Each thread owns ept <= EPT contiguous slots, ept a multiple of 4 just
  // large enough for the row's n entries, so short rows cost little: every
  // per-slot loop stops at ept (a workgroup-uniform bound).
  uint32_t key[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) key[e] = 0u;
  const int ept = min(EPT, (n + 4 * THREADS - 1) / (4 * THREADS) * 4);
  const int e0 = tid * ept;
  {
    const BufferRsrc rsrc = make_buffer(a.scores + base, (uint32_t)n * 4u);
#pragma unroll
    for (int c = 0; c < EPT / 4; ++c) {
      if (4 * c >= ept) break;
      const uint4 raw = buffer_load_16(rsrc, (uint32_t)(e0 + 4 * c) * 4u);
      const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int i = 0; i < 4; ++i)
        key[4 * c + i] = e0 + 4 * c + i < n ? float_to_ordered(__uint_as_float(w4[i])) : 0u;
    }
    if (a.in_idx) {
      const int64_t* ids = a.in_idx + base;
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        if (e >= ept) break;
        if (e0 + e < n && ids[e0 + e] < 0) key[e] = 0;
      }
    }
  }

  // cstar = composite of the k-th largest; with at most k valid slots every
  // valid slot (key >= 1) is chosen.
  uint64_t cstar = uint64_t(1) << 32;
  uint32_t n_valid = 0;
  float lo = __builtin_inff();
  float hi = -__builtin_inff();
#ifdef DSA_PHASE_TRACE
  {  // wait for the row (trace builds only) so that the mark times its arrival
    uint32_t dep = 0;
#pragma unroll
    for (int e = 0; e < EPT; ++e) dep ^= key[e];
    asm volatile("" ::"v"(dep));
  }
#endif
  DSA_TRACE_MARK(g_trace_topk, blockIdx.x, 1);
  if (n > k) {
    // Valid count and finite range of the row in one pass and one barrier;
    // the histogram is cleared in the same phase.
    uint32_t mine = 0;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      if (e >= ept) break;
      const float f = ordered_to_float(key[e]);
      const bool fin = key[e] != 0 && __builtin_isfinite(f);
      mine += key[e] != 0 ? 1u : 0u;
      lo = fminf(lo, fin ? f : __builtin_inff());
      hi = fmaxf(hi, fin ? f : -__builtin_inff());
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      mine += __shfl_xor(mine, off, kWave);
      lo = fminf(lo, __shfl_xor(lo, off, kWave));
      hi = fmaxf(hi, __shfl_xor(hi, off, kWave));
    }
    if (lane == 0) {
      sh.wave_valid[wave] = mine;
      sh.wave_lo[wave] = lo;
      sh.wave_hi[wave] = hi;
    }
    for (int i = tid; i < kBins; i += THREADS) sh.hist[i] = 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
      n_valid += sh.wave_valid[i];
      lo = fminf(lo, sh.wave_lo[i]);
      hi = fmaxf(hi, sh.wave_hi[i]);
    }
  }
  DSA_TRACE_MARK(g_trace_topk, blockIdx.x, 2);
  if (n_valid > (uint32_t)k) {
    bool resolved = false;
    const float scale = (float)kBins / (hi - lo);
    if (lo < hi && __builtin_isfinite(scale) && scale > 0.f) {
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        if (e >= ept) break;
        lds_add(&sh.hist[value_bucket(key[e], lo, scale)], key[e] != 0 ? 1u : 0u);
      }
      __syncthreads();
      locate_bin(sh, (uint32_t)k);
      DSA_TRACE_MARK(g_trace_topk, blockIdx.x, 3);
      const int bucket = (int)sh.digit;
      const uint32_t need = sh.krem;
      const uint32_t crowd = sh.hist[bucket];
      if (crowd <= (uint32_t)CAP) {
        // Gather bucket T's composites at scan-assigned slots, sort them and
        // read the need-th largest.
        uint32_t mine = 0;
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
          if (e >= ept) break;
          mine += (key[e] != 0 && value_bucket(key[e], lo, scale) == bucket) ? 1u : 0u;
        }
        uint32_t total;
        uint32_t slot = block_exclusive_scan<kWaves>(mine, sh.wave_sums, total);
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
          if (e >= ept) break;
          const bool in_t = key[e] != 0 && value_bucket(key[e], lo, scale) == bucket;
          sh.sort_keys[in_t ? slot : CAP] = composite(key[e], e0 + e);
          slot += in_t ? 1u : 0u;
        }
        if (crowd <= (uint32_t)kWave) {
          // Few candidates: the one with need - 1 larger composites is cstar
          // (composites are distinct).
          __syncthreads();
          if (tid < (int)crowd) {
            const uint64_t c = sh.sort_keys[tid];
            uint32_t larger = 0;
            for (int j = 0; j < (int)crowd; ++j) larger += sh.sort_keys[j] > c ? 1u : 0u;
            if (larger + 1 == need) sh.cstar = c;
          }
          __syncthreads();
          cstar = sh.cstar;
        } else {
          int width = 1;
          while (width < (int)crowd) width <<= 1;
          for (int i = (int)crowd + tid; i < width; i += THREADS) sh.sort_keys[i] = 0;
          __syncthreads();
          bitonic_sort_desc<THREADS>(sh.sort_keys, width);
          cstar = sh.sort_keys[need - 1];
        }
        resolved = true;
      }
    }
    if (!resolved) {
      // Radix select of the k-th value, then the krem-th tie in index order.
      uint32_t prefix = 0;
      uint32_t prefix_mask = 0;
      uint32_t want = (uint32_t)k;
#pragma unroll 1
      for (int pass = 0; pass < 3; ++pass) {
        const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
        const uint32_t dmask = pass == 2 ? 0x3ffu : 0x7ffu;
        __syncthreads();
        for (int i = tid; i < kBins; i += THREADS) sh.hist[i] = 0;
        __syncthreads();
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
          if (e >= ept) break;
          lds_add(&sh.hist[(key[e] >> shift) & dmask],
                  (key[e] != 0 && (key[e] & prefix_mask) == prefix) ? 1u : 0u);
        }
        __syncthreads();
        locate_bin(sh, want);
        prefix |= sh.digit << shift;
        prefix_mask |= dmask << shift;
        want = sh.krem;
      }
      const uint32_t threshold = prefix;
      uint32_t mine = 0;
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        if (e >= ept) break;
        mine += key[e] == threshold ? 1u : 0u;
      }
      uint32_t ties;
      uint32_t rank = block_exclusive_scan<kWaves>(mine, sh.wave_sums, ties);
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        if (e >= ept) break;
        const bool tie = key[e] == threshold;
        if (tie && rank + 1 == want) sh.cstar = composite(threshold, e0 + e);
        rank += tie ? 1u : 0u;
      }
      __syncthreads();
      cstar = sh.cstar;
    }
    __syncthreads();
  }

  DSA_TRACE_MARK(g_trace_topk, blockIdx.x, 4);
  // Chosen elements (composite >= cstar) in index order: thread slices are
  // contiguous, so the exclusive scan of the per-thread counts is each
  // element's output slot.
  uint32_t n_sel = 0;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    if (e >= ept) break;
    n_sel += composite(key[e], e0 + e) >= cstar ? 1u : 0u;
  }
  uint32_t sel_total;
  uint32_t p = block_exclusive_scan<kWaves>(n_sel, sh.wave_sums, sel_total);
  DSA_TRACE_MARK(g_trace_topk, blockIdx.x, 5);
  // Exactly min(valid, k) elements are chosen; the clamp only guards buffers.
  sel_total = min(sel_total, (uint32_t)k);
  if (a.sorted) {
    // Stage the chosen composites (at most k <= CAP) and sort them by (value desc, index asc).
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      if (e >= ept) break;
      const uint64_t c = composite(key[e], e0 + e);
      const bool chosen = c >= cstar;
      sh.sort_keys[(chosen && p < sel_total) ? p : CAP] = c;
      p += chosen ? 1u : 0u;
    }
    __syncthreads();
    int width = 1;
    while (width < (int)sel_total) width <<= 1;
    for (int i = (int)sel_total + tid; i < width; i += THREADS) sh.sort_keys[i] = 0;
    __syncthreads();
    bitonic_sort_desc<THREADS>(sh.sort_keys, width);
    for (int i = tid; i < (int)sel_total; i += THREADS) {
      const uint32_t pos = ~(uint32_t)(sh.sort_keys[i] & 0xffffffffu);
      if (a.out_idx) a.out_idx[out_base + i] = a.in_idx ? a.in_idx[base + pos] : (int64_t)(start + pos);
      if (a.out_val) a.out_val[out_base + i] = a.scores[base + pos];
    }
  } else {
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      if (e >= ept) break;
      const bool chosen = composite(key[e], e0 + e) >= cstar && p < sel_total;
      if (chosen) {
        const int pos = e0 + e;
        if (a.out_idx) a.out_idx[out_base + p] = a.in_idx ? a.in_idx[base + pos] : (int64_t)(start + pos);
        if (a.out_val) a.out_val[out_base + p] = a.scores[base + pos];
      }
      p += chosen ? 1u : 0u;
    }
  }
  // Padding when fewer than k valid entries exist.
  for (int i = (int)sel_total + tid; i < k; i += THREADS) {
    if (a.out_idx) a.out_idx[out_base + i] = -1;
    if (a.out_val) a.out_val[out_base + i] = -__builtin_inff();
  }
  DSA_TRACE_MARK(g_trace_topk, blockIdx.x, 6);
}

int launch_topk(const TopkArgs& a, int64_t virtual_rows, hipStream_t stream) {
  const int n = a.chunk_len;
  const dim3 grid((unsigned)virtual_rows);
  if (virtual_rows >= 1024 && n <= 256 * 16 && (!a.sorted || a.k <= kSmallCap)) {
    // Many short rows: 256-thread workgroups with a small candidate buffer
    // (about 17 KB of LDS), eight per CU.
    const dim3 block(256);
    if (n <= 256 * 4) hipLaunchKernelGGL((topk_kernel<256, 4, kSmallCap>), grid, block, 0, stream, a);
    else if (n <= 256 * 8) hipLaunchKernelGGL((topk_kernel<256, 8, kSmallCap>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((topk_kernel<256, 16, kSmallCap>), grid, block, 0, stream, a);
    return check_launch("topk_kernel");
  }
  const dim3 block(kTopkThreads);
  if (n <= kTopkThreads * 4) hipLaunchKernelGGL((topk_kernel<kTopkThreads, 4, kMaxK>), grid, block, 0, stream, a);
  else if (n <= kTopkThreads * 8) hipLaunchKernelGGL((topk_kernel<kTopkThreads, 8, kMaxK>), grid, block, 0, stream, a);
  else if (n <= kTopkThreads * 16) hipLaunchKernelGGL((topk_kernel<kTopkThreads, 16, kMaxK>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((topk_kernel<kTopkThreads, 32, kMaxK>), grid, block, 0, stream, a);
  return check_launch("topk_kernel");
}

constexpr int64_t kMaxRowLen = int64_t(kTopkThreads) * 32;
constexpr int64_t kLongChunk = 32768;
static_assert(kMaxRowLen == kTopkRowsMaxLength, "one-workgroup rows");

}  // namespace

int launch_topk_rows(const float* scores, int64_t rows, int64_t length, int64_t k, int64_t* out_idx,
                     const uint32_t* skip, hipStream_t stream) {
  DSA_REQUIRE(length > 0 && length <= kMaxRowLen && k > 0 && k <= kMaxK, "rows of %lld for k=%lld",
              (long long)length, (long long)k);
  TopkArgs a;
  a.scores = scores;
  a.in_idx = nullptr;
  a.row_stride = length;
  a.row_lengths = nullptr;
  a.length = (int32_t)length;
  a.chunks = 1;
  a.chunk_len = (int32_t)length;
  a.k = (int32_t)k;
  a.sorted = 0;
  a.out_idx = out_idx;
  a.out_val = nullptr;
  a.skip = skip;
  return launch_topk(a, rows, stream);
}

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
  a.skip = nullptr;
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
  a.skip = nullptr;
  if (int st = launch_topk(a, rows * chunks, s)) return st;
  // Stage 2: exact merge of the candidates (ties break on the global index).
  return dsa_topk(cand_val, cand_idx, rows, chunks * k, chunks * k, nullptr, k, sorted,
                  out_indices, out_values, stream);
}

#ifdef DSA_PHASE_TRACE
// The per-row top-k kernel's phase log (trace builds only).
extern "C" int dsa_trace_topk(uint64_t* host, int64_t n, int32_t clear) {
  DSA_REQUIRE(host && n >= 0 && n <= int64_t(kTraceWgs) * kTraceMarks, "bad trace read");
  if (int st = check_hip(hipMemcpyFromSymbol(host, HIP_SYMBOL(g_trace_topk), (size_t)n * 8), "trace read"))
    return st;
  if (clear) {
    static const uint64_t zeros[kTraceWgs * kTraceMarks] = {};
    return check_hip(hipMemcpyToSymbol(HIP_SYMBOL(g_trace_topk), zeros, sizeof(zeros)), "trace clear");
  }
  return DSA_STATUS_OK;
}
#endif
