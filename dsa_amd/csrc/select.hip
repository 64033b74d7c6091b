// Distributed exact top-k for the batched decode step (scores + selection).
//
// The scoring kernel, run with a histogram workspace, also counts every score
// of a row into 4096 bins given by the top 12 bits of its order-preserving key
// (a bin's values are all larger than every value of a lower bin).  Two
// kernels then select the k largest per row with the stable_topk rule (ties at
// the cut-off to the lower index, reference metrics.py:9-22), each spread over
// ceil(L / 2048) workgroups per row:
//   gather:  find the bin T holding the k-th largest, count each chunk's
//            elements in bins above T, and append T's elements (as composites
//            (key << 32 | ~index)) to the row's candidate list;
//   resolve: radix-select the exact cut-off composite among the candidates,
//            derive every chunk's output offset, write the chosen indices of
//            the chunk in ascending index order, and clear the histogram.
// Kernel boundaries order the phases, so no workgroup ever waits on another.
#include "common.hpp"
#include "select.hpp"
#include "status.hpp"

namespace dsa {
namespace {

constexpr int kSelThreads = 256;
constexpr int kSelWaves = kSelThreads / kWave;
constexpr int kSelEpt = kSelectChunk / kSelThreads;  // 8
constexpr int kDigitBins = 2048;
constexpr int kCandCapacity = 4096;  // candidates staged in LDS (else read in place)
constexpr uint32_t kNoBin = 0xffffffffu;
// Buffer stores aimed here fall outside every descriptor's range and are
// dropped; small enough that offset + size cannot wrap.
constexpr uint32_t kSinkOffset = 0x7ffffff0u;
constexpr uint32_t kSinkSlot = 0x0ffffffeu;  // * 8 stays below 2^31

struct SelectArgs {
  const float* scores;  // [rows, length]
  int32_t rows;
  int32_t length;
  int32_t chunks;
  int32_t k;
  SelectWorkspace ws;
  int64_t* out_idx;  // [rows, k]
  float* out_val;    // [rows, k] or null
};

__device__ __forceinline__ uint64_t composite(uint32_t key, int pos) {
  return (uint64_t(key) << 32) | (uint64_t)(~(uint32_t)pos);
}

// Exclusive scan over the 256 threads; two barriers.
__device__ __forceinline__ uint32_t sel_scan(uint32_t v, uint32_t* wave_sums, uint32_t& total) {
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
  for (int i = 0; i < kSelWaves; ++i) {
    const uint32_t s = wave_sums[i];
    before += i < wave ? s : 0u;
    all += s;
  }
  __syncthreads();
  total = all;
  return before + x - v;
}

// Loads this thread's 8 ordered keys of chunk c (0 = past the row end).
__device__ __forceinline__ void load_chunk(const float* row_scores, int length, int c,
                                           uint32_t (&key)[kSelEpt], int& e0) {
  e0 = c * kSelectChunk + threadIdx.x * kSelEpt;
  const BufferRsrc rsrc = make_buffer(row_scores, (uint32_t)length * 4u);
#pragma unroll
  for (int h = 0; h < kSelEpt / 4; ++h) {
    const uint4 raw = buffer_load_16(rsrc, (uint32_t)(e0 + 4 * h) * 4u);
    const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      key[4 * h + i] = e0 + 4 * h + i < length ? float_to_ordered(__uint_as_float(w4[i])) : 0u;
  }
}

__global__ __launch_bounds__(kSelThreads) void select_gather_kernel(SelectArgs a) {
  __shared__ uint32_t wave_sums[kSelWaves];
  __shared__ uint32_t s_bin;
  __shared__ uint32_t s_need;
  const int tid = threadIdx.x;
  const int row = blockIdx.x / a.chunks;
  const int c = blockIdx.x % a.chunks;

  // Issue the chunk's scores and the row histogram together.
  uint32_t key[kSelEpt];
  int e0;
  load_chunk(a.scores + (size_t)row * a.length, a.length, c, key, e0);
  uint32_t h[16];  // thread t owns bins [16t, 16t + 16)
  {
    const uint4* p = reinterpret_cast<const uint4*>(a.ws.hist + (size_t)row * kSelectBins + tid * 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 v = p[i];
      h[4 * i] = v.x;
      h[4 * i + 1] = v.y;
      h[4 * i + 2] = v.z;
      h[4 * i + 3] = v.w;
    }
  }
  uint32_t mine = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) mine += h[i];
  if (tid == 0) {
    s_bin = kNoBin;
    s_need = 0;
  }
  uint32_t total;
  const uint32_t before = sel_scan(mine, wave_sums, total);
  const uint32_t want = (uint32_t)a.k;
  uint32_t above = total - before - mine;  // elements in bins past this thread's
#pragma unroll
  for (int i = 15; i >= 0; --i) {
    if (total > want && h[i] && above < want && want <= above + h[i]) {
      s_bin = tid * 16 + i;
      s_need = want - above;
    }
    above += h[i];
  }
  __syncthreads();
  const uint32_t bin = s_bin;
  if (c == 0 && tid == 0) {
    uint32_t* meta = a.ws.meta + (size_t)row * 4;
    meta[0] = bin;
    meta[1] = s_need;
    meta[2] = total;
  }

  // This chunk: elements above T are chosen outright, T's are candidates and
  // go to the chunk's own slice of the candidate buffer.
  uint32_t n_above = 0;
  uint32_t n_cand = 0;
#pragma unroll
  for (int e = 0; e < kSelEpt; ++e) {
    const uint32_t b = key[e] >> 20;
    const bool valid = key[e] != 0;
    n_above += (valid && (bin == kNoBin || b > bin)) ? 1u : 0u;
    n_cand += (valid && bin != kNoBin && b == bin) ? 1u : 0u;
  }
  uint32_t above_total;
  sel_scan(n_above, wave_sums, above_total);
  uint32_t cand_total;
  uint32_t rank = sel_scan(n_cand, wave_sums, cand_total);
  if (tid == 0) {
    a.ws.above[(size_t)row * a.chunks + c] = above_total;
    a.ws.cand_count[(size_t)row * a.chunks + c] = cand_total;
  }
  const BufferRsrc cand = make_buffer(a.ws.cand + (size_t)row * a.length + (size_t)c * kSelectChunk,
                                      kSelectChunk * 8u);
#pragma unroll
  for (int e = 0; e < kSelEpt; ++e) {
    const bool is_cand = key[e] != 0 && bin != kNoBin && (key[e] >> 20) == bin;
    buffer_store_u64(cand, is_cand ? rank * 8u : kSinkOffset, composite(key[e], e0 + e));
    rank += is_cand ? 1u : 0u;
  }
}

__global__ __launch_bounds__(kSelThreads) void select_resolve_kernel(SelectArgs a) {
  __shared__ uint32_t wave_sums[kSelWaves];
  __shared__ uint32_t hist[kDigitBins];
  __shared__ uint32_t chunk_above[kMaxSelectChunks];
  __shared__ uint32_t chunk_count[kMaxSelectChunks];
  __shared__ uint32_t chunk_first[kMaxSelectChunks + 1];
  __shared__ uint32_t chunk_chosen[kMaxSelectChunks];
  __shared__ uint64_t cands[kCandCapacity];
  __shared__ uint32_t s_digit;
  __shared__ uint32_t s_krem;
  __shared__ uint64_t s_cstar;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int row = blockIdx.x / a.chunks;
  const int c = blockIdx.x % a.chunks;
  const int chunks = a.chunks;

  // Issue this chunk's scores, the row's meta and per-chunk counts together.
  uint32_t key[kSelEpt];
  int e0;
  load_chunk(a.scores + (size_t)row * a.length, a.length, c, key, e0);
  const uint32_t* meta = a.ws.meta + (size_t)row * 4;
  const uint32_t bin = meta[0];
  const uint32_t need = meta[1];
  const uint32_t total = meta[2];
  for (int j = tid; j < chunks; j += kSelThreads) {
    chunk_above[j] = a.ws.above[(size_t)row * chunks + j];
    chunk_count[j] = a.ws.cand_count[(size_t)row * chunks + j];
    chunk_chosen[j] = 0;
  }
  __syncthreads();
  if (tid < kWave) {  // exclusive prefix of the candidate counts
    uint32_t carry = 0;
    for (int j0 = 0; j0 < chunks; j0 += kWave) {
      const int j = j0 + lane;
      const uint32_t v = j < chunks ? chunk_count[j] : 0u;
      uint32_t x = v;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(x, off, kWave);
        x += lane >= off ? y : 0u;
      }
      if (j < chunks) chunk_first[j] = carry + x - v;
      carry += __shfl(x, 63, kWave);
    }
    if (lane == 0) chunk_first[chunks] = carry;
  }
  __syncthreads();
  const uint32_t crowd = chunk_first[chunks];
  const bool in_lds = crowd <= (uint32_t)kCandCapacity;
  const uint64_t* row_cands = a.ws.cand + (size_t)row * a.length;

  // Cut-off composite: with no threshold bin every valid element is chosen.
  uint64_t cstar = uint64_t(1) << 32;
  if (bin != kNoBin) {
    // Candidate i of the row in chunk-major order lives in the slice of the
    // chunk j with chunk_first[j] <= i < chunk_first[j + 1].
    auto cand_global = [&](uint32_t i) -> uint64_t {
      int lo = 0;
      int hi = chunks - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (chunk_first[mid] <= i) lo = mid;
        else hi = mid - 1;
      }
      return row_cands[(size_t)lo * kSelectChunk + (i - chunk_first[lo])];
    };
    if (in_lds) {
      for (uint32_t i = tid; i < crowd; i += kSelThreads) cands[i] = cand_global(i);
      __syncthreads();
    }
    auto cand_at = [&](uint32_t i) -> uint64_t { return in_lds ? cands[i] : cand_global(i); };
    // Radix select of the need-th largest composite below the 12 bits the
    // candidates share; stops as soon as the cut-off digit holds one of them.
    uint64_t prefix = uint64_t(bin) << 52;
    uint64_t mask = uint64_t(0xfff) << 52;
    uint32_t want = need;
    bool done = false;
#pragma unroll 1
    for (int shift = 41; shift > -11 && !done; shift -= 11) {
      const int sh = shift < 0 ? 0 : shift;
      const uint32_t width = shift < 0 ? (uint32_t)(11 + shift) : 11u;
      const uint64_t dmask = (uint64_t(1) << width) - 1;
      __syncthreads();
      for (int i = tid; i < kDigitBins; i += kSelThreads) hist[i] = 0;
      if (tid == 0) {
        s_digit = 0;
        s_krem = 1;
      }
      __syncthreads();
      for (uint32_t i = tid; i < crowd; i += kSelThreads) {
        const uint64_t x = cand_at(i);
        __hip_atomic_fetch_add(&hist[(x >> sh) & dmask], (x & mask) == prefix ? 1u : 0u,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
      __syncthreads();
      // Thread t owns digits [8t, 8t + 8).
      uint32_t hv[8];
      uint32_t mine = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        hv[i] = hist[tid * 8 + i];
        mine += hv[i];
      }
      uint32_t all;
      const uint32_t before = sel_scan(mine, wave_sums, all);
      uint32_t above = all - before - mine;
#pragma unroll
      for (int i = 7; i >= 0; --i) {
        if (hv[i] && above < want && want <= above + hv[i]) {
          s_digit = tid * 8 + i;
          s_krem = want - above;
        }
        above += hv[i];
      }
      __syncthreads();
      const uint32_t digit = s_digit;
      prefix |= uint64_t(digit) << sh;
      mask |= dmask << sh;
      want = s_krem;
      done = hist[digit] == 1 || sh == 0;
    }
    // The unique candidate matching the prefix is the cut-off.
    for (uint32_t i = tid; i < crowd; i += kSelThreads) {
      const uint64_t x = cand_at(i);
      if ((x & mask) == prefix) s_cstar = x;
    }
    __syncthreads();
    cstar = s_cstar;
    // Chosen candidates per chunk (a candidate's chunk follows from its index).
    for (uint32_t i = tid; i < crowd; i += kSelThreads) {
      const uint64_t x = cand_at(i);
      const uint32_t pos = ~(uint32_t)(x & 0xffffffffu);
      __hip_atomic_fetch_add(&chunk_chosen[pos / kSelectChunk], x >= cstar ? 1u : 0u,
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }
  __syncthreads();
  // Output offset of this chunk: everything chosen in the chunks before it.
  uint32_t offset = 0;
  for (int j = 0; j < c; ++j) offset += chunk_above[j] + chunk_chosen[j];

  uint32_t n_sel = 0;
#pragma unroll
  for (int e = 0; e < kSelEpt; ++e) n_sel += composite(key[e], e0 + e) >= cstar ? 1u : 0u;
  uint32_t sel_total;
  uint32_t rank = offset + sel_scan(n_sel, wave_sums, sel_total);
  const uint32_t kk = (uint32_t)a.k;
  const BufferRsrc oidx = make_buffer(a.out_idx + (size_t)row * kk, kk * 8u);
  const BufferRsrc oval = make_buffer(a.out_val ? a.out_val + (size_t)row * kk : nullptr,
                                      a.out_val ? kk * 4u : 0u);
#pragma unroll
  for (int e = 0; e < kSelEpt; ++e) {
    const bool chosen = composite(key[e], e0 + e) >= cstar;
    const uint32_t slot = chosen ? rank : kSinkSlot;  // dropped past the row
    buffer_store_u64(oidx, slot * 8u, (uint64_t)(int64_t)(e0 + e));
    if (a.out_val)
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(ordered_to_float(key[e])), oval,
                                            (int)(slot * 4u), 0, 0);
    rank += chosen ? 1u : 0u;
  }
  // Rows with fewer than k scores: pad with index -1 / value -inf.
  if (c == 0) {
    for (uint32_t i = min(total, kk) + tid; i < kk; i += kSelThreads) {
      a.out_idx[(size_t)row * kk + i] = -1;
      if (a.out_val) a.out_val[(size_t)row * kk + i] = -__builtin_inff();
    }
  }
  // Leave the histogram zeroed for the next call (its readers are done).
  const int per = (kSelectBins + chunks - 1) / chunks;
  uint32_t* hrow = a.ws.hist + (size_t)row * kSelectBins;
  for (int i = c * per + tid; i < min(kSelectBins, (c + 1) * per); i += kSelThreads) hrow[i] = 0;
}

// Rows of up to 32768 scores with k <= 4096: one 1024-thread workgroup per
// row.  Wave w holds positions [2048w, 2048w + 2048) in registers, lane l the
// eight 4-position groups 2048w + 256g + 4l (g = 0..7), so that a wave's
// positions in (g, lane, i) order are in index order.  Wave 0 alone locates
// the threshold bin in the histogram the scoring kernel built, and later the
// radix digits; the bin's keys are compacted into LDS with ballots, the exact
// k-th key is radix-selected among them (bits 19..9, then 8..0), ties at that
// key are ranked by position, and the chosen positions are staged in LDS in
// index order and written out coalesced.  The kernel runs once per row, so
// its time is set by latency: it avoids block-wide scans on the common path
// (one barrier per phase, wave-level ballot and DPP scans otherwise).
constexpr int kRowThreads = 1024;
constexpr int kRowWaves = kRowThreads / kWave;
constexpr int kRowLength = 32768;
constexpr int kRowGroups = 8;      // 4-position groups per lane
constexpr int kRowMaxK = 4096;
constexpr int kRowCand = 4096;     // threshold-bin keys compacted into LDS
constexpr int kRowDigits1 = 2048;  // bits 19..9
constexpr int kRowDigits2 = 512;   // bits 8..0

__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x & (kWave - 1); }

// Inclusive scan over the 64 lanes: DPP row shifts within 16-lane rows, then
// the row totals read off lanes 15, 31 and 47.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
  const uint32_t lane = lane_id();
  x += __builtin_amdgcn_update_dpp(0u, x, 0x111, 0xf, 0xf, true);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0u, x, 0x112, 0xf, 0xf, true);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0u, x, 0x114, 0xf, 0xf, true);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0u, x, 0x118, 0xf, 0xf, true);  // row_shr:8
  const uint32_t r0 = __builtin_amdgcn_readlane(x, 15);
  const uint32_t r1 = __builtin_amdgcn_readlane(x, 31);
  const uint32_t r2 = __builtin_amdgcn_readlane(x, 47);
  return x + (lane >= 16 ? r0 : 0u) + (lane >= 32 ? r1 : 0u) + (lane >= 48 ? r2 : 0u);
}

// Exclusive scan over the workgroup: one barrier; `ws` (16 words) must not be
// rewritten until every thread has passed a later barrier.
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* ws, uint32_t& total) {
  const uint32_t lane = lane_id();
  const uint32_t wave = threadIdx.x / kWave;
  const uint32_t incl = wave_incl_scan(v);
  if (lane == kWave - 1) ws[wave] = incl;
  __syncthreads();
  uint32_t before = 0;
  uint32_t all = 0;
#pragma unroll
  for (int q = 0; q < kRowWaves / 4; ++q) {
    const uint4 s4 = reinterpret_cast<const uint4*>(ws)[q];
    const uint32_t sv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      before += (uint32_t)(4 * q + j) < wave ? sv[j] : 0u;
      all += sv[j];
    }
  }
  total = all;
  return before + incl - v;
}

__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

struct Locate {
  uint32_t digit;  // kNoBin when the want-th largest is not in these bins
  uint32_t rem;    // its rank among the keys of that digit (1-based)
  uint32_t count;  // keys in that digit
};

// One wave finds the bin holding the want-th largest key among 64*N LDS
// counters (higher bin = larger keys) in two levels: lane l sums bins
// [N*l, N*l + N), a scan over the lane sums names the lane, then that lane's
// N bins, one per lane, are scanned again.  With `none_if_fits`, a total of
// at most `want` keys returns kNoBin (every key is selected).
template <int N>
__device__ __forceinline__ Locate wave_locate(const uint32_t* bins, uint32_t want, bool none_if_fits) {
  static_assert(N % 4 == 0 && N <= kWave, "bins per lane");
  const uint32_t lane = lane_id();
  const uint4* b4 = reinterpret_cast<const uint4*>(bins);
  uint32_t sum = 0;
#pragma unroll
  for (int q = 0; q < N / 4; ++q) {
    // Rotated so that 8 consecutive lanes read 8 distinct 16-byte bank groups.
    const uint4 v = b4[(N / 4) * lane + ((q + lane) % (N / 4))];
    sum += v.x + v.y + v.z + v.w;
  }
  const uint32_t incl = wave_incl_scan(sum);
  const uint32_t total = __builtin_amdgcn_readlane(incl, kWave - 1);
  const uint32_t above = total - incl;  // keys in the bins of higher lanes
  const uint64_t m = __ballot(above < want && want <= above + sum);
  if (m == 0 || (none_if_fits && total <= want)) return Locate{kNoBin, 0u, 0u};
  const uint32_t owner = (uint32_t)__builtin_ctzll(m);
  const uint32_t above_owner = __builtin_amdgcn_readlane(above, owner);
  const uint32_t c = lane < (uint32_t)N ? bins[N * owner + lane] : 0u;
  const uint32_t incl2 = wave_incl_scan(c);
  const uint32_t above2 = above_owner + __builtin_amdgcn_readlane(incl2, kWave - 1) - incl2;
  const uint64_t m2 = __ballot(above2 < want && want <= above2 + c);
  const uint32_t j = (uint32_t)__builtin_ctzll(m2);
  return Locate{N * owner + j, want - (uint32_t)__builtin_amdgcn_readlane(above2, j),
                (uint32_t)__builtin_amdgcn_readlane(c, j)};
}

__global__ __launch_bounds__(kRowThreads) void select_row_kernel(SelectArgs a) {
  __shared__ uint32_t cand[kRowCand];       // bin keys (low 20 bits), then staged positions
  __shared__ uint32_t stage_key[kRowMaxK];  // staged keys
  __shared__ __align__(16) uint32_t hist[kSelectBins];
  __shared__ __align__(16) uint32_t digits1[kRowDigits1];
  __shared__ __align__(16) uint32_t digits2[kRowDigits2];
  __shared__ __align__(16) uint32_t wsum[2][kRowWaves];
  __shared__ uint32_t s_bin, s_want, s_crowd, s_fill, s_d1, s_cpos;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = lane_id();
  const uint32_t wave = tid / kWave;
  const int row = blockIdx.x;
  const int n = a.length;
  const uint32_t kk = (uint32_t)a.k;

  // The row's histogram (4 bins per thread) is issued first, then the scores
  // of this lane's 32 positions.
  const BufferRsrc hr = make_buffer(a.ws.hist + (size_t)row * kSelectBins, kSelectBins * 4u);
  const uint4 hv = buffer_load_16(hr, tid * 16u);
  const uint32_t base = wave * 2048u + 4u * lane;
  uint4 raw[kRowGroups];
  {
    const BufferRsrc rsrc = make_buffer(a.scores + (size_t)row * n, (uint32_t)n * 4u);
#pragma unroll
    for (int g = 0; g < kRowGroups; ++g) raw[g] = buffer_load_16(rsrc, (base + 256u * g) * 4u);
  }
  for (uint32_t i = tid; i < (uint32_t)kRowDigits1; i += kRowThreads) digits1[i] = 0;
  if (tid < (uint32_t)kRowDigits2) digits2[tid] = 0;
  reinterpret_cast<uint4*>(hist)[tid] = hv;
  // This workgroup is the histogram's only reader: clear it for the next call.
  buffer_store_16(hr, tid * 16u, make_uint4(0u, 0u, 0u, 0u));
  __syncthreads();
  if (wave == 0) {
    const Locate t = wave_locate<kSelectBins / kWave>(hist, kk, true);
    if (lane == 0) {
      s_bin = t.digit;
      s_want = t.rem;
      s_crowd = t.count;
      s_fill = 0;
    }
  }
  uint32_t key[4 * kRowGroups];
#pragma unroll
  for (int g = 0; g < kRowGroups; ++g) {
    const uint32_t w4[4] = {raw[g].x, raw[g].y, raw[g].z, raw[g].w};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      key[4 * g + i] = (int)(base + 256u * g + i) < n ? float_to_ordered(__uint_as_float(w4[i])) : 0u;
  }
  __syncthreads();
  const uint32_t bin = s_bin;
  const uint32_t crowd = s_crowd;
  uint32_t want = s_want;

  // The selection is every key above (ckey, cpos) in (key desc, index asc)
  // order; with total <= k that is every valid key (key >= 1).
  uint32_t ckey = 1;
  uint32_t cpos = 0xffffffffu;
  if (bin != kNoBin) {
    uint32_t d1;
    uint32_t low;
    uint32_t ties;
    if (crowd <= (uint32_t)kRowCand) {
      // Compact the bin's keys (low 20 bits) into LDS.
      uint32_t wcount = 0;
#pragma unroll
      for (int e = 0; e < 4 * kRowGroups; ++e)
        wcount += __popcll(__ballot(key[e] != 0 && (key[e] >> 20) == bin));
      uint32_t at = 0;
      if (lane == 0 && wcount) at = __hip_atomic_fetch_add(&s_fill, wcount, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      at = __builtin_amdgcn_readfirstlane(at);
#pragma unroll
      for (int e = 0; e < 4 * kRowGroups; ++e) {
        const bool in = key[e] != 0 && (key[e] >> 20) == bin;
        const uint64_t m = __ballot(in);
        if (in) cand[at + lanes_below(m)] = key[e] & 0xfffffu;
        at += __popcll(m);
      }
      __syncthreads();
      for (uint32_t i = tid; i < crowd; i += kRowThreads)
        __hip_atomic_fetch_add(&digits1[cand[i] >> 9], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      __syncthreads();
      if (wave == 0) {
        const Locate t = wave_locate<kRowDigits1 / kWave>(digits1, want, false);
        if (lane == 0) {
          s_d1 = t.digit;
          s_want = t.rem;
        }
      }
      __syncthreads();
      d1 = s_d1;
      want = s_want;
      for (uint32_t i = tid; i < crowd; i += kRowThreads) {
        const uint32_t v = cand[i];
        if ((v >> 9) == d1)
          __hip_atomic_fetch_add(&digits2[v & 0x1ffu], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    } else {
      // A crowded bin (many equal or near-equal scores): count in place.
#pragma unroll
      for (int e = 0; e < 4 * kRowGroups; ++e)
        if (key[e] != 0 && (key[e] >> 20) == bin)
          __hip_atomic_fetch_add(&digits1[(key[e] >> 9) & 0x7ffu], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      __syncthreads();
      if (wave == 0) {
        const Locate t = wave_locate<kRowDigits1 / kWave>(digits1, want, false);
        if (lane == 0) {
          s_d1 = t.digit;
          s_want = t.rem;
        }
      }
      __syncthreads();
      d1 = s_d1;
      want = s_want;
#pragma unroll
      for (int e = 0; e < 4 * kRowGroups; ++e)
        if (key[e] != 0 && (key[e] >> 9) == ((bin << 11) | d1))
          __hip_atomic_fetch_add(&digits2[key[e] & 0x1ffu], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    __syncthreads();
    if (wave == 0) {
      const Locate t = wave_locate<kRowDigits2 / kWave>(digits2, want, false);
      if (lane == 0) {
        s_d1 = t.digit;
        s_want = t.rem;
        s_crowd = t.count;
      }
    }
    __syncthreads();
    low = (d1 << 9) | s_d1;
    want = s_want;
    ties = s_crowd;
    ckey = (bin << 20) | low;
    if (want < ties) {
      // Only the first `want` keys equal to ckey (in index order) are chosen:
      // rank the ties in (wave, g, lane, i) order, which is index order.
      uint32_t wrun = 0;
      uint32_t off[kRowGroups];
#pragma unroll
      for (int g = 0; g < kRowGroups; ++g) {
        uint32_t t = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) t += key[4 * g + i] == ckey ? 1u : 0u;
        const uint32_t incl = wave_incl_scan(t);
        off[g] = wrun + incl - t;
        wrun += __builtin_amdgcn_readlane(incl, kWave - 1);
      }
      uint32_t all_t;
      const uint32_t wbase = block_excl_scan(lane == 0 ? wrun : 0u, wsum[0], all_t);
      const uint32_t first = __builtin_amdgcn_readfirstlane(wbase);
#pragma unroll
      for (int g = 0; g < kRowGroups; ++g) {
        uint32_t r = first + off[g];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool tie = key[4 * g + i] == ckey;
          if (tie && r + 1 == want) s_cpos = base + 256u * g + i;
          r += tie ? 1u : 0u;
        }
      }
      __syncthreads();
      cpos = s_cpos;
    }
  }

  // Chosen positions in index order: per-wave offsets from DPP scans, wave
  // bases from one exchange, staged in LDS, then written out coalesced.
  uint32_t wrun = 0;
  uint32_t off[kRowGroups];
#pragma unroll
  for (int g = 0; g < kRowGroups; ++g) {
    uint32_t t = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t v = key[4 * g + i];
      t += (v > ckey || (v == ckey && base + 256u * g + i <= cpos)) ? 1u : 0u;
    }
    const uint32_t incl = wave_incl_scan(t);
    off[g] = wrun + incl - t;
    wrun += __builtin_amdgcn_readlane(incl, kWave - 1);
  }
  if (lane == 0) wsum[1][wave] = wrun;
  __syncthreads();
  uint32_t wbase = 0;
  uint32_t sel_total = 0;
#pragma unroll
  for (int q = 0; q < kRowWaves / 4; ++q) {
    const uint4 s4 = reinterpret_cast<const uint4*>(wsum[1])[q];
    const uint32_t sv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      wbase += (uint32_t)(4 * q + j) < wave ? sv[j] : 0u;
      sel_total += sv[j];
    }
  }
#pragma unroll
  for (int g = 0; g < kRowGroups; ++g) {
    uint32_t slot = wbase + off[g];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t v = key[4 * g + i];
      const uint32_t p = base + 256u * g + i;
      if (v > ckey || (v == ckey && p <= cpos)) {
        cand[slot] = p;
        stage_key[slot] = v;
        ++slot;
      }
    }
  }
  __syncthreads();
  int64_t* oidx = a.out_idx + (size_t)row * kk;
  float* oval = a.out_val ? a.out_val + (size_t)row * kk : nullptr;
  for (uint32_t i = tid; i < kk; i += kRowThreads) {
    const bool live = i < sel_total;
    oidx[i] = live ? (int64_t)cand[i] : int64_t(-1);
    if (oval) oval[i] = live ? ordered_to_float(stage_key[i]) : -__builtin_inff();
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
  const int64_t cand_off = above_off + round(rows * chunks * 4);
  SelectWorkspace ws;
  ws.bytes = cand_off + rows * length * 8;
  const uintptr_t p = reinterpret_cast<uintptr_t>(base);
  ws.hist = base ? reinterpret_cast<uint32_t*>(p + hist_off) : nullptr;
  ws.cand_count = base ? reinterpret_cast<uint32_t*>(p + count_off) : nullptr;
  ws.meta = base ? reinterpret_cast<uint32_t*>(p + meta_off) : nullptr;
  ws.above = base ? reinterpret_cast<uint32_t*>(p + above_off) : nullptr;
  ws.cand = base ? reinterpret_cast<uint64_t*>(p + cand_off) : nullptr;
  return ws;
}

int launch_select(const float* scores, int64_t rows, int64_t length, int64_t k,
                  const SelectWorkspace& ws, int64_t* out_idx, float* out_val,
                  hipStream_t stream) {
  SelectArgs a;
  a.scores = scores;
  a.rows = (int32_t)rows;
  a.length = (int32_t)length;
  a.chunks = (int32_t)((length + kSelectChunk - 1) / kSelectChunk);
  a.k = (int32_t)k;
  a.ws = ws;
  a.out_idx = out_idx;
  a.out_val = out_val;
  if (length <= kRowLength && k <= kRowMaxK) {
    hipLaunchKernelGGL(select_row_kernel, dim3((unsigned)rows), dim3(kRowThreads), 0, stream, a);
    return check_launch("select_row_kernel");
  }
  const dim3 grid((unsigned)(rows * a.chunks));
  hipLaunchKernelGGL(select_gather_kernel, grid, dim3(kSelThreads), 0, stream, a);
  if (int st = check_launch("select_gather_kernel")) return st;
  hipLaunchKernelGGL(select_resolve_kernel, grid, dim3(kSelThreads), 0, stream, a);
  return check_launch("select_resolve_kernel");
}

}  // namespace dsa

using namespace dsa;

extern "C" int dsa_select_topk(const float* scores, int64_t batch, int64_t length, int64_t k,
                               int64_t* out_indices, float* out_values, void* workspace,
                               int64_t workspace_bytes, void* stream) {
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
  return launch_select(scores, batch, length, k, ws, out_indices, out_values,
                       static_cast<hipStream_t>(stream));
}
