// Exact top-k for the batched decode step (scores + selection).
//
// The scoring kernel, run with a histogram workspace, also counts every score
// of a row into 4096 bins given by the top 12 bits of its order-preserving key
// (a bin's values are all larger than every value of a lower bin).  The k
// largest per row are then selected with the stable_topk rule (ties at the
// cut-off to the lower index, reference metrics.py:9-22), indices written in
// ascending order, by two launches over the whole GPU, one 256-thread
// workgroup per 2048-score chunk of a row:
//   gather:  locate the bin T holding the k-th largest score, count the
//            chunk's scores above T, and write the chunk's scores inside T
//            (as composites key << 32 | ~index) to the chunk's candidate slice;
//   resolve: fetch the row's counts and candidates in one round trip,
//            radix-select the exact cut among the candidates, derive the
//            chunk's output offset, write its chosen indices, and clear the
//            chunk's share of the histogram for the next call.
// The kernel boundary is the only synchronisation between workgroups.
#include "common.hpp"
#include "select.hpp"
#include "waveops.hpp"
#include "status.hpp"


namespace dsa {
namespace {

constexpr int kSelThreads = 256;
constexpr int kSelWaves = kSelThreads / kWave;
constexpr int kSelEpt = kSelectChunk / kSelThreads;  // 8 scores per thread
constexpr int kDigitBins = 2048;
constexpr int kCandCapacity = 4096;  // row candidates staged in LDS (else read in place)
constexpr int kSpecSlots = 1024;     // candidate slots fetched with the counts

struct SelectArgs {
  const float* scores;  // [rows, length]
  int32_t rows;
  int32_t length;
  int32_t chunks;
  int32_t k;
  SelectWorkspace ws;
  int64_t* out_idx;  // [rows, k]
  float* out_val;    // [rows, k] or null
  const uint32_t* skip;  // [rows] or null: rows with a nonzero flag are not selected
};

__device__ __forceinline__ uint64_t composite(uint32_t key, int pos) { return select_composite(key, (uint32_t)pos); }

#ifdef DSA_PHASE_TRACE
// The list select, per workgroup (by blockIdx.x): 0 start, 1 entries counted
// and the cut's bin located, 2 cut resolved, 3 earlier lists' chosen counted,
// 4 written; 5, 6, 7: the radix cut's passes 0, 1, 2 counted.
__device__ uint64_t g_trace_select[kTraceWgs * kTraceMarks];
#endif

// Radix select of the want-th largest composite among the n entries at(i)
// whose top 12 bits equal `bin`: 11-bit digits of bits 51..41, then the
// score key's last 9 bits (40..32); then the position part, 11, 11 and 10
// bits.  All waves count a digit, wave 0 locates the digit holding the cut
// while the other waves clear the other counter buffer, and a digit with a
// single entry ends the search (that entry was recorded while counting).
// With kOrdered (the entries at(0..n) in ascending position order), once the
// score key is fixed the cut is the rem-th entry carrying it in that order,
// found by one counting pass and a block scan instead of three position
// digits: tied scores are common where scores are quantised.
// digits[0] must be zero on entry; both buffers are left dirty.
struct RadixShared {
  uint64_t last[kDigitBins];  // an entry of each digit (the only one when its count is 1)
  __align__(16) uint32_t wsum[kSelWaves];  // the tie scan's wave sums (read as uint4)
  uint32_t digit, rem, count;
  uint64_t tie;
};

template <bool kOrdered, class At>
__device__ __forceinline__ uint64_t radix_cut(uint32_t bin, uint32_t want, uint32_t n, At at,
                                              uint32_t (*digits)[kDigitBins], RadixShared& rs) {
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = lane_id();
  const uint32_t wave = tid / kWave;
  uint64_t prefix = uint64_t(bin) << 52;
  uint64_t mask = uint64_t(0xfff) << 52;
  uint32_t rem = want;
#pragma unroll 1
  for (int pass = 0; pass < 5; ++pass) {
    if (kOrdered && pass == 2) {
      // The score key is fixed: the rem-th entry carrying it, by position.
      const uint32_t per = (n + kSelThreads - 1) / kSelThreads;
      const uint32_t i0 = min(n, tid * per);
      const uint32_t i1 = min(n, i0 + per);
      uint32_t ties = 0;
      for (uint32_t i = i0; i < i1; ++i) ties += (at(i) & mask) == prefix ? 1u : 0u;
      uint32_t total;
      uint32_t before = block_excl_scan<kSelWaves>(ties, rs.wsum, total);
      if (before < rem && rem <= before + ties) {
        for (uint32_t i = i0; i < i1; ++i) {
          const uint64_t x = at(i);
          if ((x & mask) == prefix && ++before == rem) rs.tie = x;
        }
      }
      __syncthreads();
      return rs.tie;
    }
    // Digits: bits 51..41, 40..32, 31..21, 20..10, 9..0 (selects, not a
    // table: a table would be a scalar load at every pass).
    const int shift = pass == 0 ? 41 : pass == 1 ? 32 : pass == 2 ? 21 : pass == 3 ? 10 : 0;
    const uint32_t dmask = pass == 1 ? 0x1ffu : pass == 4 ? 0x3ffu : 0x7ffu;
    uint32_t* dig = digits[pass & 1];
    // Eight entries per thread are read before any is counted, so that the
    // reads are in flight together (the counts and the recorded entries
    // would otherwise order every read behind the previous entry's writes).
    constexpr int kBatch = 8;
    for (uint32_t i0 = tid; i0 < n; i0 += kBatch * kSelThreads) {
      uint64_t x[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const uint32_t i = i0 + u * kSelThreads;
        x[u] = i < n ? at(i) : 0u;
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        if (i0 + u * kSelThreads < n && (x[u] & mask) == prefix) {
          const uint32_t d = (uint32_t)(x[u] >> shift) & dmask;
          __hip_atomic_fetch_add(&dig[d], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
          rs.last[d] = x[u];
        }
      }
    }
    __syncthreads();
    if (pass < 3) DSA_TRACE_MARK(g_trace_select, blockIdx.x, 5 + pass);
    if (wave == 0) {
      const Locate t = wave_locate<kDigitBins / kWave>(dig, rem, false);
      if (lane == 0) {
        rs.digit = t.digit;
        rs.rem = t.rem;
        rs.count = t.count;
      }
    } else {
      uint32_t* next = digits[(pass + 1) & 1];
      for (uint32_t i = tid - kWave; i < (uint32_t)kDigitBins; i += kSelThreads - kWave) next[i] = 0;
    }
    __syncthreads();
    if (rs.digit == kNoBin) break;  // unreachable for consistent counts
    prefix |= uint64_t(rs.digit) << shift;
    mask |= uint64_t(dmask) << shift;
    rem = rs.rem;
    if (rs.count == 1) return rs.last[rs.digit];  // the one entry carrying the prefix
    // rs is rewritten only after the next pass's first barrier, which every
    // thread reaches after reading it here.
  }
  return prefix;  // all 64 bits fixed
}

// ---------------------------------------------------------------------------
// gather: one workgroup per (row, chunk).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kSelThreads) void select_gather_kernel(SelectArgs a) {
  __shared__ __align__(16) uint32_t hist[kSelectBins];
  __shared__ __align__(16) uint32_t wsum[kSelWaves];
  __shared__ uint32_t s_bin, s_want, s_total;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = lane_id();
  const uint32_t wave = tid / kWave;
  const uint32_t chunks = (uint32_t)a.chunks;
  const uint32_t logical = logical_block();
  const uint32_t row = logical / chunks;
  const uint32_t c = logical % chunks;
  if (a.skip && a.skip[row]) return;
  const uint32_t n = (uint32_t)a.length;
  const uint32_t kk = (uint32_t)a.k;
  const uint32_t p0 = c * kSelectChunk + tid * kSelEpt;

  // This thread's 8 scores and 16 bins of the row's histogram, issued together.
  const BufferRsrc srs = make_buffer(a.scores + (size_t)row * n, n * 4u);
  const uint4 s0 = buffer_load_16(srs, p0 * 4u);
  const uint4 s1 = buffer_load_16(srs, (p0 + 4u) * 4u);
  {
    const BufferRsrc hr = make_buffer(a.ws.hist + (size_t)row * kSelectBins, kSelectBins * 4u);
#pragma unroll
    for (int q = 0; q < kSelectBins / (4 * kSelThreads); ++q)
      reinterpret_cast<uint4*>(hist)[tid + q * kSelThreads] = buffer_load_16(hr, (tid + q * kSelThreads) * 16u);
  }
  __syncthreads();
  if (wave == 0) {
    const Locate t = wave_locate<kSelectBins / kWave>(hist, kk, true);
    if (lane == 0) {
      s_bin = t.digit;
      s_want = t.rem;
      s_total = t.total;
    }
  }
  __syncthreads();
  const uint32_t bin = s_bin;

  uint32_t key[kSelEpt];
  {
    const uint32_t w8[kSelEpt] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
    for (int i = 0; i < kSelEpt; ++i) key[i] = p0 + i < n ? float_to_ordered(__uint_as_float(w8[i])) : 0u;
  }
  uint32_t n_above = 0;
  uint32_t n_cand = 0;
#pragma unroll
  for (int i = 0; i < kSelEpt; ++i) {
    const uint32_t kb = key[i] >> 20;
    n_above += (key[i] != 0 && (bin == kNoBin || kb > bin)) ? 1u : 0u;
    n_cand += (key[i] != 0 && bin != kNoBin && kb == bin) ? 1u : 0u;
  }
  uint32_t packed_total;
  const uint32_t packed = block_excl_scan<kSelWaves>((n_cand << 16) | n_above, wsum, packed_total);
  if (n_cand) {
    uint64_t* slice = a.ws.cand + (size_t)row * n + (size_t)c * kSelectChunk;
    uint32_t slot = packed >> 16;
#pragma unroll
    for (int i = 0; i < kSelEpt; ++i)
      if (key[i] != 0 && (key[i] >> 20) == bin) slice[slot++] = composite(key[i], (int)(p0 + i));
  }
  if (tid == 0) {
    a.ws.above[(size_t)row * chunks + c] = packed_total & 0xffffu;
    a.ws.cand_count[(size_t)row * chunks + c] = packed_total >> 16;
    if (c == 0) {
      a.ws.meta[row * 4 + 0] = bin;
      a.ws.meta[row * 4 + 1] = s_want;
      a.ws.meta[row * 4 + 2] = s_total;
    }
  }
}

// ---------------------------------------------------------------------------
// resolve: one workgroup per (row, chunk).
//
// One round trip fetches this chunk's scores, the row's meta, the per-chunk
// counts (wave 0 scans them) and the first slots of every chunk's candidate
// slice; the candidates are staged in LDS.  The exact cut is a radix select
// over (key, ~position) composites (radix_cut).  The candidates of the
// earlier chunks at or above the cut and this chunk's chosen scores share one
// block scan.  Five barriers in the common case.
// ---------------------------------------------------------------------------
struct ResolveShared {
  uint64_t cands[kCandCapacity];
  RadixShared radix;
  uint32_t digits[2][kDigitBins];
  uint32_t base[kMaxSelectChunks + 1];  // candidate prefix over the row's chunks
  uint32_t wsum[2][kSelWaves];
  uint32_t offset, crowd, overflow;
};

__global__ __launch_bounds__(kSelThreads) void select_resolve_kernel(SelectArgs a) {
  __shared__ ResolveShared sh;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = lane_id();
  const uint32_t wave = tid / kWave;
  const uint32_t chunks = (uint32_t)a.chunks;
  const uint32_t logical = logical_block();
  const uint32_t row = logical / chunks;
  const uint32_t c = logical % chunks;
  if (a.skip && a.skip[row]) return;
  const uint32_t n = (uint32_t)a.length;
  const uint32_t kk = (uint32_t)a.k;
  const uint32_t p0 = c * kSelectChunk + tid * kSelEpt;
  const uint64_t* row_cands = a.ws.cand + (size_t)row * n;

  // One round trip: this chunk's scores, the row's meta, the per-chunk counts
  // (wave 0, up to 4 chunks per lane) and the first `spec` candidate slots of
  // every chunk (valid below a chunk's count, stale above it).
  const BufferRsrc srs = make_buffer(a.scores + (size_t)row * n, n * 4u);
  const uint4 s0 = buffer_load_16(srs, p0 * 4u);
  const uint4 s1 = buffer_load_16(srs, (p0 + 4u) * 4u);
  const uint32_t bin = a.ws.meta[row * 4 + 0];
  const uint32_t want = a.ws.meta[row * 4 + 1];
  const uint32_t total = a.ws.meta[row * 4 + 2];
  constexpr int kPerLane = kMaxSelectChunks / kWave;  // 4
  uint32_t above_q[kPerLane];
  uint32_t cand_q[kPerLane];
  if (wave == 0) {
#pragma unroll
    for (int q = 0; q < kPerLane; ++q) {
      const uint32_t j = lane * kPerLane + q;
      above_q[q] = j < chunks ? a.ws.above[(size_t)row * chunks + j] : 0u;
      cand_q[q] = j < chunks ? a.ws.cand_count[(size_t)row * chunks + j] : 0u;
    }
  }
  const uint32_t spec = kSpecSlots / chunks;  // >= 4
  uint64_t pre[kSpecSlots / kSelThreads];
  if (bin != kNoBin) {
#pragma unroll
    for (int i = 0; i < kSpecSlots / kSelThreads; ++i) {
      const uint32_t p = tid + i * kSelThreads;
      const uint32_t j = p / spec;
      const uint32_t at = j * kSelectChunk + p % spec;  // stays inside the row's candidate area
      pre[i] = (j < chunks && at < n) ? row_cands[at] : 0u;
    }
  }
  if (wave == 0) {
    // Exclusive prefix of both counts over the chunks, lane-major.
    uint32_t a_sum = 0;
    uint32_t c_sum = 0;
    uint32_t widest = 0;
#pragma unroll
    for (int q = 0; q < kPerLane; ++q) {
      a_sum += above_q[q];
      c_sum += cand_q[q];
      widest = max(widest, cand_q[q]);
    }
    const uint32_t a_incl = wave_incl_scan(a_sum);
    const uint32_t c_incl = wave_incl_scan(c_sum);
    uint32_t a_run = a_incl - a_sum;
    uint32_t c_run = c_incl - c_sum;
#pragma unroll
    for (int q = 0; q < kPerLane; ++q) {
      const uint32_t j = lane * kPerLane + q;
      if (j < chunks) sh.base[j] = c_run;
      if (j == c) sh.offset = a_run;  // chosen scores above the bin in earlier chunks
      a_run += above_q[q];
      c_run += cand_q[q];
    }
    const bool overflow = __ballot(widest > spec) != 0;
    if (lane == kWave - 1) {
      sh.base[chunks] = c_incl;
      sh.crowd = c_incl;
      sh.overflow = overflow ? 1u : 0u;
    }
  } else {
    for (uint32_t i = tid - kWave; i < 2u * kDigitBins; i += kSelThreads - kWave) (&sh.digits[0][0])[i] = 0;
  }
  __syncthreads();
  const uint32_t crowd = sh.crowd;
  const bool in_lds = crowd <= (uint32_t)kCandCapacity;
  auto chunk_of = [&](uint32_t i) -> uint32_t {  // last chunk whose base is <= i
    uint32_t lo = 0;
    uint32_t hi = chunks - 1;
    while (lo < hi) {
      const uint32_t mid = (lo + hi + 1) >> 1;
      if (sh.base[mid] <= i) lo = mid; else hi = mid - 1;
    }
    return lo;
  };
  auto cand_at = [&](uint32_t i) -> uint64_t {
    if (in_lds) return sh.cands[i];
    const uint32_t j = chunk_of(i);
    return row_cands[(size_t)j * kSelectChunk + (i - sh.base[j])];
  };

  uint64_t cstar = uint64_t(1) << 32;  // every valid score when the row has <= k
  if (bin != kNoBin) {
    if (in_lds) {
#pragma unroll
      for (int i = 0; i < kSpecSlots / kSelThreads; ++i) {
        const uint32_t p = tid + i * kSelThreads;
        const uint32_t j = p / spec;
        const uint32_t s = p % spec;
        if (j < chunks && sh.base[j] + s < sh.base[j + 1]) sh.cands[sh.base[j] + s] = pre[i];
      }
      if (sh.overflow) {
        // Some chunk holds more candidates than its prefetched slots: the rest.
        for (uint32_t i = tid; i < crowd; i += kSelThreads) {
          const uint32_t j = chunk_of(i);
          const uint32_t s = i - sh.base[j];
          if (s >= spec) sh.cands[i] = row_cands[(size_t)j * kSelectChunk + s];
        }
      }
      __syncthreads();
    }
    cstar = radix_cut<false>(bin, want, crowd, cand_at, sh.digits, sh.radix);
  }

  // This chunk's chosen scores in index order, after the chosen scores of the
  // earlier chunks: those above the bin (sh.offset) and the candidates at or
  // above the cut, counted here and summed by the same block scan.
  uint32_t key[kSelEpt];
  {
    const uint32_t w8[kSelEpt] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
    for (int i = 0; i < kSelEpt; ++i) key[i] = p0 + i < n ? float_to_ordered(__uint_as_float(w8[i])) : 0u;
  }
  uint32_t mine = 0;
#pragma unroll
  for (int i = 0; i < kSelEpt; ++i) mine += composite(key[i], (int)(p0 + i)) >= cstar ? 1u : 0u;
  uint32_t before = 0;
  if (bin != kNoBin)
    for (uint32_t i = tid; i < sh.base[c]; i += kSelThreads) before += cand_at(i) >= cstar ? 1u : 0u;
  const uint32_t offset = sh.offset;
  uint32_t slot;
  if (crowd < 65536u) {
    uint32_t packed_total;
    const uint32_t packed = block_excl_scan<kSelWaves>((before << 16) | mine, sh.wsum[0], packed_total);
    slot = offset + (packed_total >> 16) + (packed & 0xffffu);
  } else {
    uint32_t before_all;
    block_excl_scan<kSelWaves>(before, sh.wsum[0], before_all);
    uint32_t chunk_total;
    slot = offset + before_all + block_excl_scan<kSelWaves>(mine, sh.wsum[1], chunk_total);
  }
  int64_t* oidx = a.out_idx + (size_t)row * kk;
  float* oval = a.out_val ? a.out_val + (size_t)row * kk : nullptr;
  if (mine) {
#pragma unroll
    for (int i = 0; i < kSelEpt; ++i) {
      if (composite(key[i], (int)(p0 + i)) >= cstar) {
        if (slot < kk) {  // always true for consistent counts; keeps writes in the row
          oidx[slot] = (int64_t)(p0 + i);
          if (oval) oval[slot] = ordered_to_float(key[i]);
        }
        ++slot;
      }
    }
  }
  if (c == 0) {
    for (uint32_t i = min(total, kk) + tid; i < kk; i += kSelThreads) {
      oidx[i] = -1;
      if (oval) oval[i] = -__builtin_inff();
    }
  }
  // No reader of the row's histogram is left: clear this chunk's share.
  {
    uint32_t* hrow = a.ws.hist + (size_t)row * kSelectBins;
    const uint32_t per = (kSelectBins + chunks - 1) / chunks;
    for (uint32_t i = tid; i < per; i += kSelThreads)
      if (c * per + i < (uint32_t)kSelectBins) hrow[c * per + i] = 0;
  }
}

// ---------------------------------------------------------------------------
// list select: one workgroup per (row, candidate list) of the decode step,
// after a scoring kernel that wrote candidate lists (no histogram pass).
//
// List j holds, in index order, every key of the row's chunk j (keys
// [j * chunk_keys, ...)) whose 12-bit bin is at least b_j.  Every workgroup of
// a row reads all of the row's lists (staged in LDS when they fit), counts
// their bins and locates the bin B of the k-th largest listed key.  The lists
// hold every key at or above the cut when each b_j <= B: the cut among the
// listed keys is then the row's cut, because the row's k-th largest is at
// least the listed k-th largest.  A list with b_j > B may miss keys; its
// chunk's raw scores replace it and the workgroup counts again.  The second
// round always holds: B can only rise, and raw chunks miss nothing.  The
// entries of bin B are compacted and radix_cut finds the cut among them; the
// workgroup then writes its own list's chosen keys after the chosen keys of
// the lists before it.
//
// Each list is read by threads_per_list consecutive threads (entry s by
// thread s mod threads_per_list), whose first kListSpec entries are fetched
// with the lists' lengths, in one round trip.
// ---------------------------------------------------------------------------
constexpr int kListSpec = 24;

struct ListArgs {
  const float* scores;      // [rows, length]
  const uint64_t* lists;    // [rows, length]: list j at j * chunk_keys
  const uint32_t* meta;     // [rows][kMaxListChunks][2]: length, lowest bin listed
  int32_t length;
  int32_t chunks;           // lists per row
  int32_t chunk_keys;
  int32_t k;
  uint32_t total_wgs;       // rows * chunks (the grid is padded to a multiple of 8)
  int64_t* out_idx;         // [rows, k]
  float* out_val;           // [rows, k] or null
  const uint32_t* count_parts;  // [rows * chunks] or null: per-chunk counts (bits 0-30) summed into count_out,
                                // bit 31 a per-chunk flag counted into flag_out
  int32_t* count_out;           // [rows]
  int32_t* flag_out;            // [rows] or null
};

struct ListShared {
  uint64_t stage[kListStageCapacity];  // the row's entries, list j at base[j]
  uint64_t cands[kCandCapacity];       // the entries of the cut's bin
  RadixShared radix;
  uint32_t hist[kSelectBins];  // bins of the entries; then the radix digit counters
  uint32_t base[kMaxListChunks + 1];  // entry prefix over the row's sources
  uint32_t raw[kMaxListChunks];       // 1: the source is the chunk's raw scores
  uint32_t wsum[2][kSelWaves];
  uint32_t bin, want, miss, crowd;
};

__global__ __launch_bounds__(kSelThreads) void select_lists_kernel(ListArgs a) {
  __shared__ ListShared sh;
  args_in_sgprs(a.scores, a.lists, a.meta, a.length, a.chunks, a.chunk_keys, a.k, a.total_wgs, a.out_idx,
                a.out_val);
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = lane_id();
  const uint32_t wave = tid / kWave;
  const uint32_t logical = logical_block();
  if (logical >= a.total_wgs) return;
  const uint32_t chunks = (uint32_t)a.chunks;
  const uint32_t row = logical / chunks;
  const uint32_t c = logical % chunks;
  const uint32_t n = (uint32_t)a.length;
  const uint32_t ck = (uint32_t)a.chunk_keys;
  const uint32_t kk = (uint32_t)a.k;
  const float* srow = a.scores + (size_t)row * n;
  const uint64_t* lrow = a.lists + (size_t)row * n;
  DSA_TRACE_MARK(g_trace_select, blockIdx.x, 0);
  if (a.count_parts && c == 0 && wave == 0) {
    uint32_t sum = 0;
    uint32_t flags = 0;
    for (uint32_t j = lane; j < chunks; j += kWave) {
      const uint32_t part = a.count_parts[(size_t)row * chunks + j];
      sum += part & 0x7fffffffu;
      flags += part >> 31;
    }
    for (int off = 32; off > 0; off >>= 1) {
      sum += (uint32_t)__shfl_xor((int)sum, off, kWave);
      flags += (uint32_t)__shfl_xor((int)flags, off, kWave);
    }
    if (lane == 0) {
      a.count_out[row] = (int32_t)sum;
      if (a.flag_out) a.flag_out[row] = (int32_t)flags;
    }
  }

  // This thread's list j and its place r among the list's threads.
  const uint32_t tpl = chunks >= (uint32_t)kSelThreads ? 1u : (uint32_t)kSelThreads / chunks;
  const uint32_t j = tid / tpl;
  const uint32_t r = tid % tpl;
  const bool has_list = j < chunks;
  const uint32_t chunk_len = has_list ? min(ck, n - j * ck) : 0u;
  uint32_t list_len = 0;
  uint32_t list_bin = 0;
  uint64_t pre[kListSpec] = {};
  if (has_list) {
    const uint32_t* m = a.meta + 2 * ((size_t)row * kMaxListChunks + j);
    list_len = min(m[0], chunk_len);  // (keeps every read inside the row whatever the workspace holds)
    list_bin = m[1];
#pragma unroll
    for (int q = 0; q < kListSpec; ++q) {
      const uint32_t s = r + tpl * q;
      pre[q] = s < chunk_len ? lrow[j * ck + s] : 0u;
    }
  }
  bool raw = false;
  auto load_entry = [&](uint32_t s) -> uint64_t {  // entry s of this thread's source
    const uint32_t pos = j * ck + s;
    return raw ? select_composite(float_to_ordered(srow[pos]), pos) : lrow[pos];
  };

  uint32_t entries = 0;
  uint32_t src_len = 0;
  uint32_t src_base = 0;
  bool staged = false;
#pragma unroll 1
  for (int round = 0; round < 2; ++round) {
#pragma unroll
    for (int q = 0; q < kSelectBins / kSelThreads; ++q) sh.hist[tid + kSelThreads * q] = 0;
    src_len = has_list ? (raw ? chunk_len : list_len) : 0u;
    const uint32_t before = block_excl_scan<kSelWaves>(r == 0 ? src_len : 0u, sh.wsum[round], entries);
    if (has_list && r == 0) {
      sh.base[j] = before;
      sh.raw[j] = raw ? 1u : 0u;
    }
    if (tid == 0) {
      sh.base[chunks] = entries;
      sh.miss = 0;
      sh.crowd = 0;
    }
    __syncthreads();
    src_base = has_list ? sh.base[j] : 0u;
    staged = entries <= (uint32_t)kListStageCapacity;
    // Count every entry's bin; stage the entries when they fit.
    auto take = [&](uint32_t s, uint64_t x) {
      __hip_atomic_fetch_add(&sh.hist[(uint32_t)(x >> 52)], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      if (staged) sh.stage[src_base + s] = x;
    };
    if (!raw) {
#pragma unroll
      for (int q = 0; q < kListSpec; ++q)
        if (r + tpl * q < src_len) take(r + tpl * q, pre[q]);
    }
    for (uint32_t s = r + (raw ? 0u : tpl * kListSpec); s < src_len; s += tpl) take(s, load_entry(s));
    __syncthreads();
    if (wave == 0) {
      const Locate t = wave_locate<kSelectBins / kWave>(sh.hist, kk, true);
      if (lane == 0) {
        sh.bin = t.digit;
        sh.want = t.rem;
      }
    }
    __syncthreads();
    // A list misses keys of the cut's bin or above when it stops above that
    // bin (or, when every entry is chosen, when it is not its whole chunk).
    const uint32_t bin = sh.bin;
    const bool miss = has_list && !raw && (bin == kNoBin ? list_bin != 0u : list_bin > bin);
    if (miss) sh.miss = 1;
    __syncthreads();
    if (!sh.miss) break;
    raw = raw || miss;
    __syncthreads();  // every thread has read sh.miss before the next round clears it
  }

  DSA_TRACE_MARK(g_trace_select, blockIdx.x, 1);
  const uint32_t bin = sh.bin;
  auto raw_of = [&](uint32_t list) { return sh.raw[list] != 0u; };
  auto entry_of = [&](uint32_t s) -> uint64_t {  // entry s of this thread's source
    return staged ? sh.stage[src_base + s] : load_entry(s);
  };
  // Entries of the sources before this chunk's: those above the cut's bin
  // are chosen; those inside it are compacted with the rest of the bin.
  // (With at most k entries, every entry of the earlier sources is chosen.)
  uint32_t before = (bin == kNoBin && tid == 0) ? sh.base[c] : 0u;
  uint64_t cstar = uint64_t(1) << 32;  // every listed key when they number at most k
  if (bin != kNoBin && staged) {
    // Staged entries: the radix cut runs over the whole stage, counting only
    // the cut bin's entries (its prefix), with no compaction of the bin
    // first (a count, a scan and a placement, 0.6 us at C2); then the chosen
    // entries of the earlier lists are counted off the stage.
    uint32_t (*digits)[kDigitBins] = reinterpret_cast<uint32_t (*)[kDigitBins]>(sh.hist);
    for (uint32_t i = tid; i < (uint32_t)kDigitBins; i += kSelThreads) digits[0][i] = 0;
    __syncthreads();
    cstar = radix_cut<true>(bin, sh.want, entries, [&](uint32_t i) { return sh.stage[i]; }, digits, sh.radix);
    DSA_TRACE_MARK(g_trace_select, blockIdx.x, 2);
    before = 0;
    for (uint32_t i = tid; i < sh.base[c]; i += kSelThreads) before += sh.stage[i] >= cstar ? 1u : 0u;
  } else if (bin != kNoBin) {
    // Entries read in place (raw rounds past the stage): count, scan, then
    // place the entries of the cut's bin, from the registers that fetched
    // them where they still hold them, else from memory.
    const bool in_regs = !raw;
    const uint32_t spec_end = in_regs ? min(src_len, tpl * kListSpec) : 0u;
    uint32_t n_cand = 0;
#pragma unroll
    for (int q = 0; q < kListSpec; ++q) {
      const uint32_t s = r + tpl * q;
      const uint32_t b = (uint32_t)(pre[q] >> 52);
      n_cand += (s < spec_end && b == bin) ? 1u : 0u;
      before += (s < spec_end && b > bin && j < c) ? 1u : 0u;
    }
    const uint32_t tail0 = in_regs ? r + tpl * kListSpec : r;
    for (uint32_t s = tail0; s < src_len; s += tpl) {
      const uint32_t b = (uint32_t)(entry_of(s) >> 52);
      n_cand += b == bin ? 1u : 0u;
      before += (b > bin && j < c) ? 1u : 0u;
    }
    uint32_t crowd_total;
    uint32_t slot = block_excl_scan<kSelWaves>(n_cand, sh.wsum[0], crowd_total);
    if (n_cand) {
#pragma unroll
      for (int q = 0; q < kListSpec; ++q) {
        const uint32_t s = r + tpl * q;
        if (s < spec_end && (uint32_t)(pre[q] >> 52) == bin) {
          if (slot < (uint32_t)kCandCapacity) sh.cands[slot] = pre[q];
          ++slot;
        }
      }
      for (uint32_t s = tail0; s < src_len; s += tpl) {
        const uint64_t x = entry_of(s);
        if ((uint32_t)(x >> 52) == bin) {
          if (slot < (uint32_t)kCandCapacity) sh.cands[slot] = x;
          ++slot;
        }
      }
    }
    if (tid == 0) sh.crowd = crowd_total;
    // The bin counters are dead: they become the radix digit counters.
    uint32_t (*digits)[kDigitBins] = reinterpret_cast<uint32_t (*)[kDigitBins]>(sh.hist);
    for (uint32_t i = tid; i < (uint32_t)kDigitBins; i += kSelThreads) digits[0][i] = 0;
    __syncthreads();
    const uint32_t crowd = sh.crowd;
    if (crowd <= (uint32_t)kCandCapacity) {
      cstar = radix_cut<false>(bin, sh.want, crowd, [&](uint32_t i) { return sh.cands[i]; }, digits, sh.radix);
      // The chosen entries of the cut's bin in the lists before this chunk's.
      for (uint32_t i = tid; i < crowd; i += kSelThreads) {
        const uint64_t x = sh.cands[i];
        before += (x >= cstar && (~(uint32_t)x) / ck < c) ? 1u : 0u;
      }
    } else {
      // Too many to compact (heavy ties): cut over every entry in place, then
      // recount the chosen entries of the earlier lists.
      auto entry_at = [&](uint32_t i) -> uint64_t {
        if (staged) return sh.stage[i];
        uint32_t lo = 0;
        uint32_t hi = chunks - 1;
        while (lo < hi) {
          const uint32_t mid = (lo + hi + 1) >> 1;
          if (sh.base[mid] <= i) lo = mid; else hi = mid - 1;
        }
        const uint32_t pos = lo * ck + (i - sh.base[lo]);
        return raw_of(lo) ? select_composite(float_to_ordered(srow[pos]), pos) : lrow[pos];
      };
      cstar = radix_cut<true>(bin, sh.want, entries, entry_at, digits, sh.radix);
      before = 0;
      for (uint32_t i = tid; i < sh.base[c]; i += kSelThreads) before += entry_at(i) >= cstar ? 1u : 0u;
    }
  }

  DSA_TRACE_MARK(g_trace_select, blockIdx.x, 3);
  // This chunk's own source, a contiguous run per thread, in index order.
  const uint32_t own0 = sh.base[c];
  const uint32_t own_n = sh.base[c + 1] - own0;
  const uint32_t per = (own_n + kSelThreads - 1) / kSelThreads;
  const uint32_t first = min(own_n, tid * per);
  const uint32_t last = min(own_n, first + per);
  auto own_at = [&](uint32_t s) -> uint64_t {
    if (staged) return sh.stage[own0 + s];
    const uint32_t pos = c * ck + s;
    return raw_of(c) ? select_composite(float_to_ordered(srow[pos]), pos) : lrow[pos];
  };
  uint32_t mine = 0;
  for (uint32_t i = first; i < last; ++i) mine += own_at(i) >= cstar ? 1u : 0u;
  uint32_t slot;
  if (kk < 65536u) {
    uint32_t packed_total;
    const uint32_t packed = block_excl_scan<kSelWaves>((before << 16) | mine, sh.wsum[0], packed_total);
    slot = (packed_total >> 16) + (packed & 0xffffu);
  } else {
    uint32_t before_all;
    block_excl_scan<kSelWaves>(before, sh.wsum[0], before_all);
    uint32_t own_total;
    slot = before_all + block_excl_scan<kSelWaves>(mine, sh.wsum[1], own_total);
  }
  int64_t* oidx = a.out_idx + (size_t)row * kk;
  float* oval = a.out_val ? a.out_val + (size_t)row * kk : nullptr;
  for (uint32_t i = first; i < last && mine; ++i) {
    const uint64_t x = own_at(i);
    if (x >= cstar) {
      if (slot < kk) {  // always true for consistent counts; keeps writes in the row
        oidx[slot] = (int64_t)(~(uint32_t)x);
        if (oval) oval[slot] = ordered_to_float((uint32_t)(x >> 32));
      }
      ++slot;
      --mine;
    }
  }
  if (c == 0) {
    for (uint32_t i = min(n, kk) + tid; i < kk; i += kSelThreads) {
      oidx[i] = -1;
      if (oval) oval[i] = -__builtin_inff();
    }
  }
  DSA_TRACE_MARK(g_trace_select, blockIdx.x, 4);
}

// ---------------------------------------------------------------------------
// histogram of arbitrary score rows: one workgroup per (row, chunk); every
// entry is counted (-inf in its own bin), so a row's total is its length.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kSelThreads) void select_hist_kernel(SelectArgs a) {
  __shared__ __align__(16) uint32_t hist[kSelectBins];
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = lane_id();
  const uint32_t chunks = (uint32_t)a.chunks;
  const uint32_t logical = logical_block();
  const uint32_t row = logical / chunks;
  const uint32_t c = logical % chunks;
  const uint32_t n = (uint32_t)a.length;
  for (uint32_t i = tid; i < (uint32_t)kSelectBins; i += kSelThreads) hist[i] = 0;
  __syncthreads();
  const uint32_t p0 = c * kSelectChunk + tid * kSelEpt;
  const BufferRsrc srs = make_buffer(a.scores + (size_t)row * n, n * 4u);
  const uint4 s0 = buffer_load_16(srs, p0 * 4u);
  const uint4 s1 = buffer_load_16(srs, (p0 + 4u) * 4u);
  const uint32_t w8[kSelEpt] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
  const uint32_t neg_inf_bin = float_to_ordered(-__builtin_inff()) >> 20;
  uint32_t neg_inf = 0;  // counted per wave: a sparse row is mostly -inf
#pragma unroll
  for (int i = 0; i < kSelEpt; ++i) {
    if (p0 + i >= n) continue;
    const uint32_t bin = float_to_ordered(__uint_as_float(w8[i])) >> 20;
    if (bin == neg_inf_bin)
      ++neg_inf;
    else
      __hip_atomic_fetch_add(&hist[bin], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  for (int off = 32; off > 0; off >>= 1) neg_inf += (uint32_t)__shfl_xor((int)neg_inf, off, kWave);
  if (lane == 0 && neg_inf)
    __hip_atomic_fetch_add(&hist[neg_inf_bin], neg_inf, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  __syncthreads();
  uint32_t* ghist = a.ws.hist + (size_t)row * kSelectBins;
  for (uint32_t i = tid; i < (uint32_t)kSelectBins; i += kSelThreads) {
    const uint32_t v = hist[i];
    if (v) __hip_atomic_fetch_add(&ghist[i], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace

SelectWorkspace select_workspace_layout(void* base, int64_t rows, int64_t length) {
  const int64_t chunks = (length + kSelectChunk - 1) / kSelectChunk;
  auto round = [](int64_t bytes) { return (bytes + 255) / 256 * 256; };
  const int64_t hist_off = 0;
  const int64_t count_off = hist_off + round(rows * kSelectBins * 4);
  const int64_t meta_off = count_off + round(rows * chunks * 4);
  const int64_t above_off = meta_off + round(rows * 16);
  const int64_t list_off = above_off + round(rows * chunks * 4);
  const int64_t cand_off = list_off + round(rows * kMaxListChunks * 8);
  SelectWorkspace ws;
  ws.bytes = cand_off + rows * length * 8;
  const uintptr_t p = reinterpret_cast<uintptr_t>(base);
  ws.hist = base ? reinterpret_cast<uint32_t*>(p + hist_off) : nullptr;
  ws.cand_count = base ? reinterpret_cast<uint32_t*>(p + count_off) : nullptr;
  ws.meta = base ? reinterpret_cast<uint32_t*>(p + meta_off) : nullptr;
  ws.above = base ? reinterpret_cast<uint32_t*>(p + above_off) : nullptr;
  ws.cand = base ? reinterpret_cast<uint64_t*>(p + cand_off) : nullptr;
  ws.list_meta = base ? reinterpret_cast<uint32_t*>(p + list_off) : nullptr;
  return ws;
}

int launch_select(const float* scores, int64_t rows, int64_t length, int64_t k,
                  const SelectWorkspace& ws, int64_t* out_idx, float* out_val,
                  hipStream_t stream, hipEvent_t start, hipEvent_t stop, const uint32_t* skip) {
  SelectArgs a;
  a.skip = skip;
  a.scores = scores;
  a.rows = (int32_t)rows;
  a.length = (int32_t)length;
  a.chunks = (int32_t)((length + kSelectChunk - 1) / kSelectChunk);
  a.k = (int32_t)k;
  a.ws = ws;
  a.out_idx = out_idx;
  a.out_val = out_val;
  const dim3 grid((unsigned)(rows * a.chunks));
  launch_timed(select_gather_kernel, grid, dim3(kSelThreads), 0, stream, start, nullptr, a);
  if (int st = check_launch("select_gather_kernel")) return st;
  launch_timed(select_resolve_kernel, grid, dim3(kSelThreads), 0, stream, nullptr, stop, a);
  return check_launch("select_resolve_kernel");
}

int launch_select_lists(const float* scores, int64_t rows, int64_t length, int64_t k,
                        const ListPlan& plan, const SelectWorkspace& ws, int64_t* out_idx,
                        float* out_val, hipStream_t stream, hipEvent_t start, hipEvent_t stop,
                        const uint32_t* count_parts, int32_t* count_out, int32_t* flag_out) {
  ListArgs a;
  a.count_parts = count_parts;
  a.count_out = count_out;
  a.flag_out = flag_out;
  a.scores = scores;
  a.lists = ws.cand;
  a.meta = ws.list_meta;
  a.length = (int32_t)length;
  a.chunks = plan.chunks;
  a.chunk_keys = plan.chunk_keys;
  a.k = (int32_t)k;
  a.total_wgs = (uint32_t)(rows * plan.chunks);
  a.out_idx = out_idx;
  a.out_val = out_val;
  // Padded to a multiple of 8 so that logical_block maps workgroup (row, j)
  // to the XCD whose L2 holds the list that scoring workgroup wrote.
  const int64_t grid = (rows * plan.chunks + 7) / 8 * 8;
  launch_timed(select_lists_kernel, dim3((unsigned)grid), dim3(kSelThreads), 0, stream, start, stop, a);
  return check_launch("select_lists_kernel");
}

int launch_select_scores(const float* scores, int64_t rows, int64_t length, int64_t k,
                         const SelectWorkspace& ws, int64_t* out_idx, float* out_val, hipStream_t stream) {
  SelectArgs a;
  a.skip = nullptr;
  a.scores = scores;
  a.rows = (int32_t)rows;
  a.length = (int32_t)length;
  a.chunks = (int32_t)((length + kSelectChunk - 1) / kSelectChunk);
  a.k = (int32_t)k;
  a.ws = ws;
  a.out_idx = out_idx;
  a.out_val = out_val;
  hipLaunchKernelGGL(select_hist_kernel, dim3((unsigned)(rows * a.chunks)), dim3(kSelThreads), 0, stream, a);
  if (int st = check_launch("select_hist_kernel")) return st;
  return launch_select(scores, rows, length, k, ws, out_idx, out_val, stream);
}

}  // namespace dsa

using namespace dsa;

extern "C" int dsa_topk_distributed(const float* scores, int64_t rows, int64_t length, int64_t k,
                                    int64_t* out_indices, float* out_values, void* workspace,
                                    int64_t workspace_bytes, void* stream) {
  DSA_REQUIRE(scores && out_indices, "null pointer argument");
  DSA_REQUIRE(rows > 0 && rows <= 65535, "rows %lld out of range", (long long)rows);
  DSA_REQUIRE(length > 0 && length <= int64_t(kSelectChunk) * kMaxSelectChunks,
              "length %lld outside [1, %d]", (long long)length, kSelectChunk * kMaxSelectChunks);
  DSA_REQUIRE(k > 0 && k <= (int64_t(1) << 27), "k=%lld out of range", (long long)k);
  DSA_REQUIRE(reinterpret_cast<uintptr_t>(scores) % 16 == 0 && reinterpret_cast<uintptr_t>(workspace) % 256 == 0,
              "scores (16 B) and workspace (256 B) must be aligned");
  const SelectWorkspace ws = select_workspace_layout(workspace, rows, length);
  if (!workspace || workspace_bytes < ws.bytes)
    return fail(DSA_STATUS_WORKSPACE_TOO_SMALL, "the distributed top-k needs %lld workspace bytes",
                (long long)ws.bytes);
  return launch_select_scores(scores, rows, length, k, ws, out_indices, out_values,
                              static_cast<hipStream_t>(stream));
}

static int select_topk(const float* scores, int64_t batch, int64_t length, int64_t k, int64_t* out_indices,
                       float* out_values, void* workspace, int64_t workspace_bytes, void* stream,
                       hipEvent_t start, hipEvent_t stop) {
  DSA_REQUIRE(scores && out_indices, "null pointer argument");
  DSA_REQUIRE(batch > 0 && batch <= 65535, "batch %lld out of range", (long long)batch);
  DSA_REQUIRE(length > 0 && length <= int64_t(kSelectChunk) * kMaxSelectChunks,
              "length %lld outside [1, %d]", (long long)length, kSelectChunk * kMaxSelectChunks);
  DSA_REQUIRE(k > 0 && k <= (int64_t(1) << 27), "k=%lld out of range", (long long)k);
  DSA_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, "workspace must be 256-byte aligned");
  const SelectWorkspace ws = select_workspace_layout(workspace, batch, length);
  if (!workspace || workspace_bytes < ws.bytes)
    return fail(DSA_STATUS_WORKSPACE_TOO_SMALL, "the decode step needs %lld workspace bytes",
                (long long)ws.bytes);
  const ListPlan plan = list_plan(batch, length, k);
  if (plan.on)
    return launch_select_lists(scores, batch, length, k, plan, ws, out_indices, out_values,
                               static_cast<hipStream_t>(stream), start, stop);
  return launch_select(scores, batch, length, k, ws, out_indices, out_values,
                       static_cast<hipStream_t>(stream), start, stop);
}

extern "C" int dsa_select_topk(const float* scores, int64_t batch, int64_t length, int64_t k,
                               int64_t* out_indices, float* out_values, void* workspace,
                               int64_t workspace_bytes, void* stream) {
  return select_topk(scores, batch, length, k, out_indices, out_values, workspace, workspace_bytes, stream,
                     nullptr, nullptr);
}

extern "C" int dsa_select_topk_timed(const float* scores, int64_t batch, int64_t length, int64_t k,
                                     int64_t* out_indices, float* out_values, void* workspace,
                                     int64_t workspace_bytes, void* stream, void* start_event,
                                     void* stop_event) {
  return select_topk(scores, batch, length, k, out_indices, out_values, workspace, workspace_bytes, stream,
                     static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(stop_event));
}

#ifdef DSA_PHASE_TRACE
// The list select's phase log (trace builds only).
extern "C" int dsa_trace_select_lists(uint64_t* host, int64_t n, int32_t clear) {
  using namespace dsa;
  DSA_REQUIRE(host && n >= 0 && n <= int64_t(kTraceWgs) * kTraceMarks, "bad trace read");
  if (int st = check_hip(hipMemcpyFromSymbol(host, HIP_SYMBOL(g_trace_select), (size_t)n * 8), "trace read"))
    return st;
  if (clear) {
    static const uint64_t zeros[kTraceWgs * kTraceMarks] = {};
    return check_hip(hipMemcpyToSymbol(HIP_SYMBOL(g_trace_select), zeros, sizeof(zeros)), "trace clear");
  }
  return DSA_STATUS_OK;
}
#endif
