// Temporal pruning of one decode step: a seeded, bounded block scan.
//
// The previous step's top-k keys (the seeds) are scored first; their minimum
// is the seed threshold tau.  Every key block b gets the upper bound
// U_b = previous block max + gamma (blocks holding keys the previous step did
// not have are never pruned).  Blocks are visited in a scan order (address;
// previous-hot first, then larger U, then address; or larger U, then
// address) and pruned iff U_b < tau; kept blocks are scored in full.  With
// wave W > 0 the threshold is refreshed after every W blocks of the scan to
// the k-th largest score evaluated so far (W = 1 is the reference's dynamic
// filter, replay.py:172-222); with W = 0 it stays at the seed threshold (the
// reference's static filter).  The result is the scores of the evaluated keys
// (-inf elsewhere), which blocks were kept, the number of keys scored and the
// stable top-k among the evaluated keys.
//
// The same scan runs the own-trajectory policy (approx.py:129-364): per-block
// metadata kept on the device gives each block a risk (stale block max, or
// EMA plus volatility, plus gamma and an age slope) that plays the bound's
// part, some blocks are forced, and after the step the metadata of refreshed
// blocks is advanced in place while skipped blocks keep stale values.
//
// Keys are scored with the tile code of the dense kernel (indexer.hpp), so
// an evaluated key's score equals the dense score bit for bit, and pruned
// blocks load no key bytes.
#include "temporal.hpp"

#include <cstdlib>
#include <cstring>

#include "status.hpp"

namespace dsa {
namespace {

// Scan orders ranked by rank_blocks (every sorted order but the
// policy's buckets, which the prep kernel sorts itself).
__host__ __device__ inline bool ranked_order(const TemporalArgs& a) {
  const bool policy = a.policy_mode != 0;
  const bool sorted = policy ? a.ap.p.order != DSA_ORDER_ADDRESS : a.scan_order != 0;
  return sorted && !(policy && a.ap.p.order == DSA_ORDER_BUCKET);
}

constexpr int kPrepClearKeys = 16384;  // scores each clearing workgroup of the prep sets to -inf

// Bounds, scan order and a clean slate for one row (one workgroup per row).
// Replay filter: U_b = prev max + gamma, +inf for blocks with new keys, order
// (previous-hot first,) larger U, lower address.  Policy: U_b = risk, or +inf
// for a forced block, order by risk (approx.py:93-109: address, larger risk
// then lower address, or buckets of that rank in address order).
__global__ __launch_bounds__(1024) void temporal_prep_kernel(TemporalArgs a) {
  __shared__ uint64_t xh[kSortN];
  __shared__ uint32_t xl[kSortN];
  __shared__ uint8_t hot[kMaxTemporalBlocks];
  __shared__ double s_upper[kMaxTemporalBlocks];
  __shared__ double s_rank[kMaxTemporalBlocks];
  __shared__ uint32_t s_exact;
  const int tid = threadIdx.x;
  const int L = a.length;
  if ((int)blockIdx.x >= a.rows) {
    // The workgroups past the rows clear the scores rows, kPrepClearKeys keys
    // each, beside the row workgroups' work.
    const int c = (int)blockIdx.x - a.rows;
    const int parts = (L + kPrepClearKeys - 1) / kPrepClearKeys;
    float* srow = a.scores + (size_t)(c / parts) * L;
    const int k1 = min(L, (c % parts + 1) * kPrepClearKeys);
    for (int i = (c % parts) * kPrepClearKeys + tid; i < k1; i += 1024) srow[i] = -__builtin_inff();
    return;
  }
  const int row = blockIdx.x;
  const int nb = a.blocks;
  const int bs = a.block_size;
  const int words = (L + 31) / 32;
  for (int i = tid; i < words; i += 1024) a.ws.seed_mask[(size_t)row * words + i] = 0;
  for (int i = tid; i < nb; i += 1024) a.evaluated[(size_t)row * nb + i] = 0;
  if (tid < kMaxRounds) a.ws.list_total[(size_t)row * kMaxRounds + tid] = 0;
  for (int i = tid; i < kSelectBins; i += 1024) a.ws.select.hist[(size_t)row * kSelectBins + i] = 0;
  if (tid == 0) {
    a.ws.tau[row] = 0xffffffffu;
    a.ws.floor[row] = 0xffffffffu;
    a.ws.done[row] = 0u;
    a.ws.loaded[row] = 0;
    a.qk_scored[row] = 0;
    if (a.waits_given_up) a.waits_given_up[row] = 0;  // only the fused static step waits
    s_exact = 0;
  }
  const int first_new = a.prev_length / bs;
  const bool grown = a.prev_length < L;
  const bool policy = a.policy_mode != 0;
  const bool sorted = policy ? a.ap.p.order != DSA_ORDER_ADDRESS : a.scan_order != 0;
  const bool hot_first = !policy && a.scan_order == 1;
  if (hot_first) {
    for (int b = tid; b < nb; b += 1024) hot[b] = 0;
    __syncthreads();
    for (int i = tid; i < a.k; i += 1024) {
      const int64_t key = a.seeds[(size_t)row * a.k + i];
      if (key >= 0 && key < L) hot[key / bs] = 1;
    }
    __syncthreads();
  }
  // Thread t owns blocks 2t and 2t + 1 (nb <= kSortN); entries past nb are
  // padding that sorts last.
  uint64_t h[2] = {~0ull, ~0ull};
  uint32_t l[2] = {0xffffffffu, 0xffffffffu};
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int b = 2 * tid + j;
    if (b >= nb) continue;
    double upper, rank_value;
    uint32_t group = 0;
    if (policy) {
      const dsa_approx_policy& p = a.ap.p;
      const double gamma = a.ap.gamma_rows ? a.ap.gamma_rows[row] : p.gamma;
      const size_t at = (size_t)row * a.ap.stride + b;
      const bool stored = b < a.prev_blocks;
      const float last = stored ? a.ap.last_max[at] : -__builtin_inff();
      const float ema = stored ? a.ap.ema[at] : -__builtin_inff();
      const float vol = stored ? a.ap.vol[at] : 0.f;
      const int age = stored ? a.ap.age[at] : 0;
      const int cold = stored ? a.ap.cold[at] : 1;
      const int recent_first = p.recent_window > 0 ? max(0, L - p.recent_window) / bs : nb;
      rank_value = policy_risk(p, gamma, last, ema, vol, age);
      const double risk = rank_value;
      if (p.order == DSA_ORDER_CURRENT_MAX) rank_value = (double)a.order_key[(size_t)row * nb + b];
      const bool forced = p.full_refresh || (grown && b >= first_new) || b >= recent_first ||
                          (p.age_cap >= 0 && age >= p.age_cap) || cold < p.cold_streak;
      upper = forced ? HUGE_VAL : risk;
    } else {
      const bool fresh = grown && b >= first_new;
      const float pm = b < a.prev_blocks ? a.prev_max[(size_t)row * a.prev_blocks + b] : -__builtin_inff();
      const double margin = a.margins ? a.margins[(size_t)row * a.prev_blocks + min(b, a.prev_blocks - 1)]
                                      : (a.gamma_d ? a.gamma_d[row] : (double)a.gamma[row]);
      upper = fresh ? HUGE_VAL : (double)pm + margin;
      rank_value = a.scan_order == 3 ? (double)a.order_key[(size_t)row * nb + b] : upper;
      group = hot_first && !hot[b] ? 0x80000000u : 0u;
    }
    a.ws.upper[(size_t)row * nb + b] = upper;
    s_upper[b] = upper;
    s_rank[b] = rank_value;
    h[j] = ~double_to_ordered(rank_value);
    l[j] = group | (uint32_t)b;
    if (ranked_order(a)) {
      a.ws.sort_hi[(size_t)row * nb + b] = h[j];
      a.ws.sort_lo[(size_t)row * nb + b] = l[j];
    }
  }
  if (ranked_order(a)) return;  // rank_blocks orders the blocks
  if (!sorted) {
    for (int b = tid; b < nb; b += 1024) {
      a.ws.order[(size_t)row * nb + b] = b;
      if (a.order_out) a.order_out[(size_t)row * nb + b] = b;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
      if (2 * tid + j < nb) a.ws.upper_pos[(size_t)row * nb + 2 * tid + j] = s_upper[2 * tid + j];
    return;
  }
  int n = 2;
  while (n < nb) n <<= 1;
  // Fast sort of (group, rank value rounded to float, larger first, block)
  // packed in 64 bits.  The rounding is monotone, so only blocks whose rank
  // values round to one float can come out of the float64 order; when two
  // such values differ the exact sort (float64 key, then group | block) runs.
  uint64_t v[2] = {~0ull, ~0ull};
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int b = 2 * tid + j;
    if (b >= nb) continue;
    const double d = __builtin_isnan(s_rank[b]) ? -HUGE_VAL : s_rank[b];
    const uint32_t fkey = float_to_ordered((float)d);
    v[j] = ((uint64_t)(l[j] >> 31) << 63) | ((uint64_t)~fkey << 12) | (uint64_t)b;
  }
  uint64_t* xk = xh;
  block_sort64(v, xk, n);
#pragma unroll
  for (int j = 0; j < 2; ++j) xk[2 * tid + j] = v[j];
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int pos = 2 * tid + j;
    if (pos == 0 || pos >= nb) continue;
    const uint64_t prev = xk[pos - 1];
    if ((prev >> 12) == (v[j] >> 12) &&
        double_to_ordered(s_rank[prev & 0xfffu]) != double_to_ordered(s_rank[v[j] & 0xfffu]))
      s_exact = 1;
  }
  __syncthreads();
  if (s_exact) {  // uniform
    block_sort(h, l, xh, xl, n);
#pragma unroll
    for (int j = 0; j < 2; ++j)
      if (2 * tid + j < nb) v[j] = l[j] & 0x7fffffffu;
  }
  if (policy && a.ap.p.order == DSA_ORDER_BUCKET) {
    // Rank r in the risk order -> bucket min(N - 1, r * N / nb); then address
    // order within each bucket.
    const int64_t buckets = a.ap.p.buckets;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int r = 2 * tid + j;
      if (r < nb) v[j] = ((uint64_t)min<int64_t>(buckets - 1, (int64_t)r * buckets / nb) << 12) | (v[j] & 0xfffu);
    }
    __syncthreads();  // xk is reused
    block_sort64(v, xk, n);
  }
  __syncthreads();  // s_upper of every block, for the bound at each position
#pragma unroll
  for (int j = 0; j < 2; ++j)
    if (2 * tid + j < nb) {
      const uint32_t blk = (uint32_t)(v[j] & 0xfffu);
      a.ws.order[(size_t)row * nb + 2 * tid + j] = blk;
      a.ws.upper_pos[(size_t)row * nb + 2 * tid + j] = s_upper[blk];
      if (a.order_out) a.order_out[(size_t)row * nb + 2 * tid + j] = (int32_t)blk;
    }
}


// The scan order by ranks: block t's position is the number of blocks whose
// (group, sort key, block) entry sorts before its own.  One workgroup per 16
// blocks of a row, 16 threads per block each counting over a sixteenth of
// the row's entries (in LDS), so the ranking of a row spreads over
// ceil(blocks / 16) CUs instead of one CU sorting.
constexpr int kRankTargets = 16;
constexpr int kRankParts = 16;

__device__ __forceinline__ void rank_blocks(const TemporalArgs& a, int block) {
  __shared__ uint64_t s_hi[kMaxTemporalBlocks];
  __shared__ uint32_t s_lo[kMaxTemporalBlocks];
  __shared__ uint32_t s_part[kRankParts][kRankTargets];
  const int tid = threadIdx.x;
  const int nb = a.blocks;
  const int per_row = (nb + kRankTargets - 1) / kRankTargets;
  const int row = block / per_row;
  const int target = (block % per_row) * kRankTargets + tid % kRankTargets;
  const int part = tid / kRankTargets;
  for (int i = tid; i < nb; i += kRankTargets * kRankParts) {
    s_hi[i] = a.ws.sort_hi[(size_t)row * nb + i];
    s_lo[i] = a.ws.sort_lo[(size_t)row * nb + i];
  }
  __syncthreads();
  uint32_t count = 0;
  if (target < nb) {
    const uint64_t th = s_hi[target];
    const uint32_t tl = s_lo[target];
    for (int b = part; b < nb; b += kRankParts) count += sorts_before(s_hi[b], s_lo[b], th, tl) ? 1u : 0u;
  }
  s_part[part][tid % kRankTargets] = count;
  __syncthreads();
  if (tid < kRankTargets && target < nb) {
    uint32_t rank = 0;
#pragma unroll
    for (int p = 0; p < kRankParts; ++p) rank += s_part[p][tid];
    a.ws.order[(size_t)row * nb + rank] = (uint32_t)target;
    a.ws.upper_pos[(size_t)row * nb + rank] = a.ws.upper[(size_t)row * nb + target];
    if (a.order_out) a.order_out[(size_t)row * nb + rank] = target;
  }
}

// The seeds: 64 per wave, gathered by index (block: the seed workgroup).
template <class Tag, class KF>
__device__ __forceinline__ void score_seeds(const TemporalArgs& a, int block) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15;
  const int g = lane >> 4;
  const int per_row = (a.k + 255) / 256;
  const int row = block / per_row;
  const int base = (block % per_row) * 256 + wave * 64;
  if (base >= a.k) return;
  const int64_t* seeds = a.seeds + (size_t)row * a.k;
  int tile_key[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int i = base + 16 * t + r;
    const int64_t key = i < a.k ? seeds[i] : -1;
    tile_key[t] = (key >= 0 && key < a.length) ? (int)key : (int)kFarKey;
  }
  const int i = base + lane;
  float v;
  if (a.source) {  // recorded scores: lane l reads its own seed's
    const int64_t key = i < a.k ? seeds[i] : -1;
    v = (key >= 0 && key < a.length) ? a.source[(size_t)row * a.source_stride + key] : 0.f;
  } else {
    v = score_unit<Tag, KF>(a, row, tile_key, r, g);
  }
  uint32_t least = 0xffffffffu;  // this lane's seed key (none: neutral for the min)
  uint32_t lowest = 0xffffffffu;  // this lane's entry of run (the floor of the running k largest)
  const uint64_t loads = __ballot(i < a.k && !a.source && seeds[i] >= 0 && seeds[i] < a.length);
  if (lane == 0 && loads)
    __hip_atomic_fetch_add(a.ws.loaded + row, (uint32_t)__builtin_popcountll(loads), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  if (i < a.k) {
    const int64_t key = seeds[i];
    if (key < 0 || key >= a.length) {
      a.ws.run[(size_t)row * a.k + i] = 0;  // below every score
      a.ws.run_idx[(size_t)row * a.k + i] = 0xffffffffu;
      lowest = 0;
    } else {
      if constexpr (KF::kScaled)
        if (!a.source) v *= a.scales[(size_t)row * ((a.key_stride + 127) / 128) + (key >> 7)];
      a.scores[(size_t)row * a.length + key] = v;
      const int words = (a.length + 31) / 32;
      __hip_atomic_fetch_or(a.ws.seed_mask + (size_t)row * words + (key >> 5), 1u << (key & 31),
                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      least = float_to_ordered(v);
      lowest = least;
      a.ws.run[(size_t)row * a.k + i] = least;
      a.ws.run_idx[(size_t)row * a.k + i] = (uint32_t)key;
    }
  }
  // One atomic per wave and value: the minimum of its 64 seeds.
  for (int off = 32; off > 0; off >>= 1) {
    least = min(least, (uint32_t)__shfl_xor((int)least, off, kWave));
    lowest = min(lowest, (uint32_t)__shfl_xor((int)lowest, off, kWave));
  }
  if (lane == 0 && least != 0xffffffffu)
    __hip_atomic_fetch_min(a.ws.tau + row, least, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (lane == 0 && lowest != 0xffffffffu)
    __hip_atomic_fetch_min(a.ws.floor + row, lowest, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <class Tag, class KF>
__global__ __launch_bounds__(256) void temporal_seed_kernel(TemporalArgs a) {
  score_seeds<Tag, KF>(a, blockIdx.x);
}

// The seeds and the ranked scan order in one launch: they are independent
// (the ranks read the prep's sort keys; the seeds score the previous top-k
// into the cleared scores row), so the seeds' gathers run beside the ranking
// instead of after it.  Workgroups [0, seed_wgs) score seeds, the rest rank.
static_assert(kRankTargets * kRankParts == 256, "rank and seed workgroups share one shape");
template <class Tag, class KF>
__global__ __launch_bounds__(256) void temporal_seed_rank_kernel(TemporalArgs a, int32_t seed_wgs) {
  if ((int)blockIdx.x < seed_wgs)
    score_seeds<Tag, KF>(a, blockIdx.x);
  else
    rank_blocks(a, (int)blockIdx.x - seed_wgs);
}

// One block per wave: scan positions [wave_start, wave_start + wave_len) of
// every row; prune against the threshold in force, score the kept blocks.
template <class Tag, class KF>
__global__ __launch_bounds__(256) void temporal_block_kernel(TemporalArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15;
  const int g = lane >> 4;
  const int per_row = (a.wave_len + 3) / 4;
  const int row = blockIdx.x / per_row;
  const int pos = a.wave_start + (blockIdx.x % per_row) * 4 + wave;
  if (pos >= a.blocks || pos >= a.wave_start + a.wave_len) return;
  const int nb = a.blocks;
  const int blk = (int)a.ws.order[(size_t)row * nb + pos];
  const double tau = (double)ordered_to_float(a.ws.tau[row]);
  const bool keep = !(a.ws.upper[(size_t)row * nb + blk] < tau);
  if (lane == 0) a.evaluated[(size_t)row * nb + blk] = keep ? 1 : 0;
  if (!keep) return;
  const int first = blk * a.block_size;
  const int end = min(a.length, first + a.block_size);
  for (int u = first >> 6; u * 64 < end; ++u) {
    int tile_key[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int tile = u * 64 + 16 * t;  // blocks are whole 16-key tiles
      tile_key[t] = (tile >= first && tile < first + a.block_size) ? tile + r : (int)kFarKey;
    }
    const int key = u * 64 + lane;
    float v;
    if (a.source)  // recorded scores: lane l reads key u * 64 + l
      v = (key >= first && key < end) ? a.source[(size_t)row * a.source_stride + key] : 0.f;
    else
      v = score_unit<Tag, KF>(a, row, tile_key, r, g);
    if (key >= first && key < end) {
      if constexpr (KF::kScaled)
        if (!a.source) v *= a.scales[(size_t)row * ((a.key_stride + 127) / 128) + (key >> 7)];
      a.scores[(size_t)row * a.length + key] = v;
    }
  }
}

// After a wave: tau = the k-th largest score evaluated so far (one workgroup
// per row merges the running k largest with the wave's new, non-seed keys).
__global__ __launch_bounds__(1024) void temporal_refresh_kernel(TemporalArgs a) {
  __shared__ uint32_t vals[kMaxMerge];
  __shared__ __align__(16) uint32_t digits[kDigitBinsT];
  __shared__ uint32_t s_fill, s_digit, s_rem, s_above;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int row = blockIdx.x;
  const int k = a.k;
  const int nb = a.blocks;
  const int bs = a.block_size;
  const int words = (a.length + 31) / 32;
  uint32_t* run = a.ws.run + (size_t)row * k;
  for (int i = tid; i < k; i += 1024) vals[i] = run[i];
  if (tid == 0) {
    s_fill = k;
    s_above = 0;
  }
  __syncthreads();
  const int span = a.wave_len * bs;
  for (int e = tid; e < span; e += 1024) {
    const int pos = a.wave_start + e / bs;
    if (pos >= nb) continue;
    const int blk = (int)a.ws.order[(size_t)row * nb + pos];
    if (!a.evaluated[(size_t)row * nb + blk]) continue;
    const int key = blk * bs + e % bs;
    if (key >= a.length) continue;
    if ((a.ws.seed_mask[(size_t)row * words + (key >> 5)] >> (key & 31)) & 1u) continue;
    const uint32_t slot = __hip_atomic_fetch_add(&s_fill, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    vals[slot] = float_to_ordered(a.scores[(size_t)row * a.length + key]);
  }
  __syncthreads();
  const uint32_t n = s_fill;
  // Radix select of the k-th largest value: bits 31..21, 20..10, 9..0.
  uint32_t prefix = 0;
  uint32_t mask = 0;
  uint32_t want = (uint32_t)k;
#pragma unroll 1
  for (int pass = 0; pass < 3; ++pass) {
    const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
    const uint32_t dmask = pass < 2 ? 0x7ffu : 0x3ffu;
    for (int i = tid; i < kDigitBinsT; i += 1024) digits[i] = 0;
    __syncthreads();
    for (uint32_t i = tid; i < n; i += 1024) {
      const uint32_t v = vals[i];
      if ((v & mask) == prefix)
        __hip_atomic_fetch_add(&digits[(v >> shift) & dmask], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    __syncthreads();
    if (wave == 0) {
      const Locate t = wave_locate<kDigitBinsT / kWave>(digits, want, false);
      if (lane == 0) {
        s_digit = t.digit;
        s_rem = t.rem;
      }
    }
    __syncthreads();
    prefix |= s_digit << shift;
    mask |= dmask << shift;
    want = s_rem;
  }
  // prefix is the k-th largest; `want` of its copies belong to the k largest.
  const uint32_t above = (uint32_t)k - want;
  for (uint32_t i = tid; i < n; i += 1024) {
    const uint32_t v = vals[i];
    if (v > prefix) run[__hip_atomic_fetch_add(&s_above, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)] = v;
  }
  for (uint32_t j = tid; j < want; j += 1024) run[above + j] = prefix;
  if (tid == 0) a.ws.tau[row] = prefix;
}

// The dynamic scan of one row in one workgroup: for each wave of W scan
// positions, every block of the wave is pruned or kept against the threshold
// in force at the wave's start (one block per wave of threads), kept blocks
// are scored, and the wave's new (non-seed) scores join the running k largest
// in LDS; a radix select then names the k-th largest, the next threshold.
// The running k largest never leave LDS and the row needs no relaunch between
// waves.  Every loop bound is uniform over the workgroup.
constexpr int kScanThreads = 512;
constexpr int kScanWaves = kScanThreads / kWave;
constexpr int kMaxRun = 4096;  // k
constexpr int kScanTiles = 6;  // 16-key tiles in flight per wave
// Keys per row: the persistent scan keeps the row's seed mask (one bit per
// key, 16 KiB at this length) in LDS; block counts are capped separately by
// kMaxTemporalBlocks (131072 keys in blocks of 64 or more).
constexpr int kMaxTemporalLength = 131072;
// Above this many waves of scan positions a step runs the persistent
// per-row scan: one launch per wave costs a launch, a grid drain and a refresh
// launch (~11 us at C3), against ~4.4 us per wave in LDS but with one CU per
// row scoring (~185 us for a C3 row's 4 MB of keys).  Rows of more key bytes
// than kPersistentRowBytes stay on the launch path, whose block launches
// spread the scoring over the whole GPU (C5, 16 MB of fp8 keys per row, 22
// waves: 435 us per step against 717 us in the persistent scan).
constexpr int kPersistentScanWaves = 16;
constexpr int64_t kPersistentRowBytes = int64_t(8) << 20;

template <class Tag, class KF>
__global__ __launch_bounds__(kScanThreads) void temporal_scan_kernel(TemporalArgs a, int32_t wave_blocks) {
  __shared__ uint32_t vals[kMaxMerge];  // [0, k): the running k largest; then the wave's new keys
  __shared__ uint32_t kept[kMaxRun];    // the next running k largest, before it moves back to vals
  __shared__ __align__(16) uint32_t digits[kDigitBinsT];
  __shared__ uint32_t s_fill, s_digit, s_rem, s_above, s_floor, s_kept;
  __shared__ int klist[kMaxMerge / 16];  // kept blocks of the current wave
  __shared__ uint32_t order[kMaxTemporalBlocks];        // block at each scan position
  __shared__ double upper[kMaxTemporalBlocks];          // its bound
  __shared__ uint32_t seed_mask[kMaxTemporalLength / 32];  // keys scored as seeds
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15;
  const int g = lane >> 4;
  const int row = blockIdx.x;
  const int k = a.k;
  const int nb = a.blocks;
  const int bs = a.block_size;
  const int tiles_per_block = bs / 16;
  const int words = (a.length + 31) / 32;
  float* srow = a.scores + (size_t)row * a.length;
  // The row's scan order, bounds and seed mask stay in LDS for the whole scan.
  for (int i = tid; i < nb; i += kScanThreads) {
    const uint32_t blk = a.ws.order[(size_t)row * nb + i];
    order[i] = blk;
    upper[i] = a.ws.upper[(size_t)row * nb + blk];  // the bound of the block at scan position i
  }
  for (int i = tid; i < words; i += kScanThreads) seed_mask[i] = a.ws.seed_mask[(size_t)row * words + i];
  // The query tiles of the row stay in registers for the whole scan.
  uint4 qa[4][4] = {};
  float wr[4][4] = {};
  if (!a.source)
    load_dense_head_tiles<4, KF::kNaturalK>(a.q + (size_t)row * kHeads * kHeadDim, a.w + (size_t)row * kHeads, r, g,
                                            qa, wr);
  // recorded scores: an empty key buffer (every load reads 0 without touching memory)
  const BufferRsrc keys = make_buffer(a.source ? nullptr : a.keys + (size_t)row * a.key_stride * KF::kRowBytes,
                                      a.source ? 0u : (uint32_t)a.length * KF::kRowBytes);
  if (tid == 0) {
    s_fill = (uint32_t)k;
    s_floor = 0xffffffffu;
  }
  __syncthreads();
  uint32_t least = 0xffffffffu;
  for (int i = tid; i < k; i += kScanThreads) {
    const uint32_t v = a.ws.run[(size_t)row * k + i];
    vals[i] = v;
    least = min(least, v);
  }
  for (int off = 32; off > 0; off >>= 1) least = min(least, (uint32_t)__shfl_xor((int)least, off, kWave));
  if (lane == 0) __hip_atomic_fetch_min(&s_floor, least, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  uint32_t tau = a.ws.tau[row];
  __syncthreads();
  // floor: the k-th largest of the running set (its minimum).  A new key at or
  // below it cannot change the k largest, so only keys above it are merged.
  uint32_t floor_key = s_floor;
  for (int start = 0; start < nb; start += wave_blocks) {
    const int len = min(wave_blocks, nb - start);
    const double bound = (double)ordered_to_float(tau);
    // Decisions for the wave's blocks, kept ones listed in LDS.
    if (tid == 0) s_kept = 0;
    __syncthreads();
    for (int p = tid; p < len; p += kScanThreads) {
      const int blk = (int)order[start + p];
      const bool keep = !(upper[start + p] < bound);
      a.evaluated[(size_t)row * nb + blk] = keep ? 1 : 0;
      if (keep) klist[__hip_atomic_fetch_add(&s_kept, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)] = blk;
    }
    __syncthreads();
    // The kept blocks' 16-key tiles, dealt round-robin to the waves, each wave
    // issuing the loads of all its tiles of a round before using any.
    const int tiles = (int)s_kept * tiles_per_block;
    for (int base = 0; base < tiles; base += kScanWaves * kScanTiles) {
      uint4 buf[kScanTiles][KF::kRaw];
      int tkey[kScanTiles];
#pragma unroll
      for (int i = 0; i < kScanTiles; ++i) {
        const int j = base + wave + kScanWaves * i;
        int key0 = -1;
        if (j < tiles) key0 = klist[j / tiles_per_block] * bs + 16 * (j % tiles_per_block);
        tkey[i] = key0;
        KF::load_buf(keys, (key0 >= 0 && key0 < a.length) ? key0 + r : (int)kFarKey, g, buf[i]);
      }
#pragma unroll
      for (int i = 0; i < kScanTiles; ++i) {
        if (tkey[i] < 0) continue;  // uniform over the wave
        const int key = tkey[i] + r;
        float v = a.source ? (key < a.length ? a.source[(size_t)row * a.source_stride + key] : 0.f)
                           : reduce_lane_groups(tile_contrib<Tag, 4, KF>(qa, wr, buf[i]));
        if (g == 0 && key < a.length) {
          if constexpr (KF::kScaled)
            if (!a.source) v *= a.scales[(size_t)row * ((a.key_stride + 127) / 128) + (key >> 7)];
          srow[key] = v;
          const uint32_t o = float_to_ordered(v);
          if (o > floor_key && !((seed_mask[key >> 5] >> (key & 31)) & 1u))
            vals[__hip_atomic_fetch_add(&s_fill, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)] = o;
        }
      }
    }
    __syncthreads();
    if (start + wave_blocks >= nb) break;  // no refresh after the last wave
    if (s_fill == (uint32_t)k) {
      // nothing above the floor: the k largest are unchanged and the threshold
      // is their minimum
      tau = floor_key;
      continue;
    }
    const uint32_t n = s_fill;
    // Radix select of the k-th largest of vals[0, n): bits 31..21, 20..10, 9..0.
    uint32_t prefix = 0;
    uint32_t mask = 0;
    uint32_t want = (uint32_t)k;
#pragma unroll 1
    for (int pass = 0; pass < 3; ++pass) {
      const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
      const uint32_t dmask = pass < 2 ? 0x7ffu : 0x3ffu;
      for (int i = tid; i < kDigitBinsT; i += kScanThreads) digits[i] = 0;
      __syncthreads();
      for (uint32_t i = tid; i < n; i += kScanThreads) {
        const uint32_t v = vals[i];
        if ((v & mask) == prefix)
          __hip_atomic_fetch_add(&digits[(v >> shift) & dmask], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
      __syncthreads();
      if (wave == 0) {
        const Locate loc = wave_locate<kDigitBinsT / kWave>(digits, want, false);
        if (lane == 0) {
          s_digit = loc.digit;
          s_rem = loc.rem;
        }
      }
      if (tid == 0) s_above = 0;
      __syncthreads();
      prefix |= s_digit << shift;
      mask |= dmask << shift;
      want = s_rem;
    }
    // prefix is the k-th largest; `want` of its copies belong to the k largest.
    const uint32_t above = (uint32_t)k - want;
    for (uint32_t i = tid; i < n; i += kScanThreads) {
      const uint32_t v = vals[i];
      if (v > prefix) kept[__hip_atomic_fetch_add(&s_above, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)] = v;
    }
    for (uint32_t j = tid; j < want; j += kScanThreads) kept[above + j] = prefix;
    __syncthreads();
    for (int i = tid; i < k; i += kScanThreads) vals[i] = kept[i];
    if (tid == 0) s_fill = (uint32_t)k;
    tau = prefix;
    floor_key = prefix;
    __syncthreads();
  }
  if (tid == 0) a.ws.tau[row] = tau;
}

// After the scan: the 4096-bin histogram (top 12 bits of the ordered key)
// of the step's scores for the select kernels, keys never scored (-inf)
// included in their own bin so that the row's count is its length, and the
// number of keys scored (the seeds plus every key of a kept block, each
// counted once).  One workgroup per (row, chunk of kSelectChunk keys).
__global__ __launch_bounds__(256) void temporal_hist_kernel(TemporalArgs a) {
  __shared__ __align__(16) uint32_t hist[kSelectBins];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int L = a.length;
  const int chunks = (L + kSelectChunk - 1) / kSelectChunk;
  const int row = blockIdx.x / chunks;
  const int c = blockIdx.x % chunks;
  if (a.ws.done[row]) return;  // finished by the dynamic rounds' last replay
  for (int i = tid; i < kSelectBins; i += 256) hist[i] = 0;
  __syncthreads();
  const float* srow = a.scores + (size_t)row * L;
  const int p0 = c * kSelectChunk + tid * (kSelectChunk / 256);
  uint32_t unscored = 0;
#pragma unroll
  for (int i = 0; i < kSelectChunk / 256; ++i) {
    const int pos = p0 + i;
    if (pos >= L) break;
    const float v = srow[pos];
    if (v == -__builtin_inff())
      ++unscored;
    else
      __hip_atomic_fetch_add(&hist[float_to_ordered(v) >> 20], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  for (int off = 32; off > 0; off >>= 1) unscored += (uint32_t)__shfl_xor((int)unscored, off, kWave);
  if (lane == 0 && unscored)
    __hip_atomic_fetch_add(&hist[float_to_ordered(-__builtin_inff()) >> 20], unscored, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_WORKGROUP);
  // Keys scored in this chunk: 64 words of 32 keys (wave 0).
  if (tid < 64) {
    const int words = (L + 31) / 32;
    const int wd = c * (kSelectChunk / 32) + tid;
    uint32_t count = 0;
    if (wd < words) {
      uint32_t bits = a.ws.seed_mask[(size_t)row * words + wd];
      for (int sub = 0; sub < 32; sub += 16) {  // blocks are multiples of 16 keys
        const int blk = (wd * 32 + sub) / a.block_size;
        if (blk < a.blocks && a.evaluated[(size_t)row * a.blocks + blk]) bits |= 0xffffu << sub;
      }
      const int valid = min(32, L - wd * 32);
      if (valid < 32) bits &= (1u << valid) - 1u;
      count = __popc(bits);
    }
    for (int off = 32; off > 0; off >>= 1) count += (uint32_t)__shfl_xor((int)count, off, kWave);
    if (tid == 0 && count)
      __hip_atomic_fetch_add(a.qk_scored + row, (int32_t)count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  uint32_t* ghist = a.ws.select.hist + (size_t)row * kSelectBins;
  for (int i = tid; i < kSelectBins; i += 256) {
    const uint32_t n = hist[i];
    if (n) __hip_atomic_fetch_add(&ghist[i], n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

enum StateMode { kStateOwn = 0, kStateInit = 1, kStateTeacher = 2 };

struct StateArgs {
  const float* scores;     // [rows][score_stride]: the step's scores (dense for init / teacher)
  int64_t score_stride;
  const int64_t* topk;     // [rows][k]: the step's top-k (hot blocks)
  const uint8_t* evaluated;  // [rows][blocks]: refreshed blocks (update only)
  const uint8_t* rescued;    // [rows][blocks] or null: blocks a verifier rescued (updated like refreshed ones)
  ApproxDev ap;
  int32_t length, blocks, block_size, k, state_blocks;
};

// kStateInit: initialize_state (approx.py:112-126) from a dense step.
// kStateOwn: the own-mode update after a step (approx.py:253-287): refreshed
// blocks take the block max of the current scores (all of their keys were
// scored), EMA and volatility move by ema_alpha (float64, stored as float32;
// the volatility's second term and sum are float32, as numpy evaluates
// `float * float32 scalar`), every other block keeps stale values and ages.
// kStateTeacher: the teacher-mode update (approx.py:270-274): every block
// takes the dense row's block max as last max and EMA, volatility 0, age 0.
// In both updates the cold streak restarts at blocks holding a key of
// s.topk (the step's own top-k, or the dense top-k for the teacher) and
// grows elsewhere.  In place: each thread reads and writes only its own
// blocks.
template <int kMode>
__global__ __launch_bounds__(1024) void approx_state_kernel(StateArgs s) {
#pragma clang fp contract(off)
  constexpr bool kInit = kMode == kStateInit;
  constexpr bool kTeacher = kMode == kStateTeacher;
  __shared__ uint8_t hot[kMaxTemporalBlocks];
  const int tid = threadIdx.x;
  const int row = blockIdx.x;
  const int nb = s.blocks;
  const int bs = s.block_size;
  // A thread's blocks (at most two: nb <= 2048): their refresh flags and
  // stored state are loaded first, unconditionally (clamped block; the state
  // rows hold at least nb entries), so that their latency overlaps the top-k
  // reads below.
  constexpr int kPer = kMaxTemporalBlocks / 1024;
  bool refreshed[kPer];
  float last_in[kPer], ema_in[kPer], vol_in[kPer];
  int age_in[kPer], cold_in[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int bc = min(tid + 1024 * j, nb - 1);
    const size_t at = (size_t)row * s.ap.stride + bc;
    refreshed[j] = kInit || kTeacher || s.evaluated[(size_t)row * nb + bc] ||
                   (s.rescued && s.rescued[(size_t)row * nb + bc]);
    if constexpr (!kInit) cold_in[j] = s.ap.cold[at];
    if constexpr (!kInit && !kTeacher) {
      last_in[j] = s.ap.last_max[at];
      ema_in[j] = s.ap.ema[at];
      vol_in[j] = s.ap.vol[at];
      age_in[j] = s.ap.age[at];
    }
  }
  for (int b = tid; b < nb; b += 1024) hot[b] = 0;
  __syncthreads();
  for (int i = tid; i < s.k; i += 1024) {
    const int64_t key = s.topk[(size_t)row * s.k + i];
    if (key >= 0 && key < s.length) hot[key / bs] = 1;
  }
  __syncthreads();
  const float* srow = s.scores + (size_t)row * s.score_stride;
  const dsa_approx_policy& p = s.ap.p;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int b = tid + 1024 * j;
    if (b >= nb) break;
    const size_t at = (size_t)row * s.ap.stride + b;
    const bool refresh = refreshed[j];
    float seen = -__builtin_inff();
    if (refresh) {
      const int end = min(s.length, (b + 1) * bs);
      for (int key = b * bs; key < end; ++key) seen = fmaxf(seen, srow[key]);
    }
    if constexpr (kInit) {
      s.ap.last_max[at] = seen;
      s.ap.ema[at] = seen;
      s.ap.vol[at] = 0.f;
      s.ap.age[at] = 0;
      s.ap.cold[at] = hot[b] ? 0 : 1;
    } else if constexpr (kTeacher) {
      const int cold = b < s.state_blocks ? cold_in[j] : 1;
      s.ap.last_max[at] = seen;
      s.ap.ema[at] = seen;
      s.ap.vol[at] = 0.f;
      s.ap.age[at] = 0;
      s.ap.cold[at] = (int16_t)(hot[b] ? 0 : min(cold + 1, 32767));
    } else {
      const bool stored = b < s.state_blocks;
      float last = stored ? last_in[j] : -__builtin_inff();
      float ema = stored ? ema_in[j] : -__builtin_inff();
      float vol = stored ? vol_in[j] : 0.f;
      int age = min((stored ? age_in[j] : 0) + 1, 32767);
      const int cold = stored ? cold_in[j] : 1;
      if (refresh) {
        const double observed = (double)seen;
        const double mean = __builtin_isfinite(ema) ? (double)ema : observed;
        const double alpha = p.ema_alpha;
        last = seen;
        ema = (float)(alpha * observed + (1.0 - alpha) * mean);
        const float carried = (float)(1.0 - alpha) * vol;
        vol = (float)(alpha * fabs(observed - mean)) + carried;
        age = 0;
      }
      s.ap.last_max[at] = last;
      s.ap.ema[at] = ema;
      s.ap.vol[at] = vol;
      s.ap.age[at] = (int16_t)age;
      s.ap.cold[at] = (int16_t)(hot[b] ? 0 : min(cold + 1, 32767));
    }
  }
}

template <class Tag, class KF>
int launch_scan(TemporalArgs& a, int32_t wave, int32_t key_dtype, hipStream_t stream) {
  const int clear_parts = (a.length + kPrepClearKeys - 1) / kPrepClearKeys;
  hipLaunchKernelGGL(temporal_prep_kernel, dim3(a.rows * (1 + clear_parts)), dim3(1024), 0, stream, a);
  if (int st = check_launch("temporal_prep_kernel")) return st;
  const int seed_wgs = a.rows * ((a.k + 255) / 256);
  if (ranked_order(a)) {
    const int per_row = (a.blocks + kRankTargets - 1) / kRankTargets;
    hipLaunchKernelGGL((temporal_seed_rank_kernel<Tag, KF>), dim3((unsigned)(seed_wgs + a.rows * per_row)), dim3(256),
                       0, stream, a, seed_wgs);
    if (int st = check_launch("temporal_seed_rank_kernel")) return st;
  } else {
    hipLaunchKernelGGL((temporal_seed_kernel<Tag, KF>), dim3(seed_wgs), dim3(256), 0, stream, a);
    if (int st = check_launch("temporal_seed_kernel")) return st;
  }
  if (wave > 0 && !legacy_paths_forced()) return temporal_rounds(a, wave, key_dtype, stream);
  const int step = wave > 0 ? wave : a.blocks;
  const int waves = (a.blocks + step - 1) / step;
  const bool light_rows = a.source || int64_t(a.length) * KF::kRowBytes <= kPersistentRowBytes;
  if (wave > 0 && waves > kPersistentScanWaves && light_rows) {
    // many refreshes: the whole scan of a row in one workgroup, no relaunch per wave
    hipLaunchKernelGGL((temporal_scan_kernel<Tag, KF>), dim3(a.rows), dim3(kScanThreads), 0, stream, a, wave);
    return check_launch("temporal_scan_kernel");
  }
  // few refreshes (or none): each wave of scan positions is scored by the
  // whole grid, and a refresh launch merges the running k largest after it
  for (int start = 0; start < a.blocks; start += step) {
    a.wave_start = start;
    a.wave_len = min(step, a.blocks - start);
    hipLaunchKernelGGL((temporal_block_kernel<Tag, KF>), dim3(a.rows * ((a.wave_len + 3) / 4)), dim3(256), 0,
                       stream, a);
    if (int st = check_launch("temporal_block_kernel")) return st;
    if (wave > 0 && start + step < a.blocks) {
      hipLaunchKernelGGL(temporal_refresh_kernel, dim3(a.rows), dim3(1024), 0, stream, a);
      if (int st = check_launch("temporal_refresh_kernel")) return st;
    }
  }
  return DSA_STATUS_OK;
}

int run_step(TemporalArgs& a, int32_t wave, int32_t key_dtype, int64_t* out_topk, void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (wave == 0 && !legacy_paths_forced()) {
    bool ran = false;
    if (int st = temporal_static_fused(a, key_dtype, out_topk, s, ran)) return st;
    if (ran) return DSA_STATUS_OK;
  }
  // Dynamic rounds: the last replay writes the top-k of the rows it can and,
  // for rows a one-workgroup top-k holds, every row's keys scored, so that
  // only that top-k runs after it (on the rows the replay left).
  const bool rounds = wave > 0 && !legacy_paths_forced();
  a.replay_topk = rounds ? out_topk : nullptr;
  a.replay_qk = rounds && a.length <= kTopkRowsMaxLength;
  if (int st = temporal_scan(a, wave, key_dtype, s)) return st;
  if (a.replay_qk) {
    if (int st = launch_topk_rows(a.scores, a.rows, a.length, a.k, out_topk, a.ws.done, s)) return st;
    return policy_state(a, out_topk, nullptr, s);
  }
  return temporal_finish(a, out_topk, nullptr, s);
}

}  // namespace

bool legacy_paths_forced() {
  const char* v = std::getenv("DSA_AMD_TEMPORAL_PATH");
  return v && std::strcmp(v, "launch") == 0;
}

int temporal_scan(TemporalArgs& a, int32_t wave, int32_t key_dtype, hipStream_t stream) {
  switch (key_dtype) {
    case DSA_DTYPE_BF16: return launch_scan<Bf16Tag, KeysB16>(a, wave, key_dtype, stream);
    case DSA_DTYPE_F16: return launch_scan<F16Tag, KeysB16>(a, wave, key_dtype, stream);
    default: return launch_scan<Bf16Tag, KeysFP8>(a, wave, key_dtype, stream);
  }
}

int temporal_finish(TemporalArgs& a, int64_t* out_topk, const uint8_t* rescued, hipStream_t stream) {
  const int chunks = (a.length + kSelectChunk - 1) / kSelectChunk;
  hipLaunchKernelGGL(temporal_hist_kernel, dim3(a.rows * chunks), dim3(256), 0, stream, a);
  if (int st = check_launch("temporal_hist_kernel")) return st;
  // Rows the dynamic rounds' last replay finished (ws.done, cleared by the
  // prep) are skipped by the histogram and the select.
  if (int st = launch_select(a.scores, a.rows, a.length, a.k, a.ws.select, out_topk, nullptr, stream, nullptr,
                             nullptr, a.ws.done))
    return st;
  return policy_state(a, out_topk, rescued, stream);
}

int policy_state(TemporalArgs& a, const int64_t* out_topk, const uint8_t* rescued, hipStream_t stream) {
  if (a.policy_mode == 0) return DSA_STATUS_OK;
  StateArgs s = {};
  s.scores = a.scores;
  s.score_stride = a.length;
  s.topk = out_topk;
  s.evaluated = a.evaluated;
  s.rescued = rescued;
  s.ap = a.ap;
  s.length = a.length;
  s.blocks = a.blocks;
  s.block_size = a.block_size;
  s.k = a.k;
  s.state_blocks = a.prev_blocks;
  if (a.ap.p.history == DSA_HISTORY_TEACHER) {
    // The teacher resets every block from the dense row (the recorded scores).
    s.scores = a.source;
    s.score_stride = a.source_stride;
    s.topk = a.teacher_topk;
    hipLaunchKernelGGL(approx_state_kernel<kStateTeacher>, dim3(a.rows), dim3(1024), 0, stream, s);
  } else {
    hipLaunchKernelGGL(approx_state_kernel<kStateOwn>, dim3(a.rows), dim3(1024), 0, stream, s);
  }
  return check_launch("approx_state_kernel");
}

int check_step(const void* queries, const void* keys, int64_t key_stride, const float* key_scales,
               int64_t prev_length, int64_t batch, int64_t length, int64_t k, int32_t block_size, int32_t wave,
               int32_t key_dtype, const void* workspace) {
  DSA_REQUIRE(batch > 0 && batch <= 65535, "batch %lld out of range", (long long)batch);
  DSA_REQUIRE(block_size == 16 || block_size == 32 || block_size == 64 || block_size == 128,
              "block_size %d not in {16, 32, 64, 128}", block_size);
  DSA_REQUIRE(length > 0 && length <= kMaxTemporalLength, "length %lld outside [1, %d]", (long long)length,
              kMaxTemporalLength);
  DSA_REQUIRE(key_stride >= length, "key_stride < length");
  DSA_REQUIRE(prev_length > 0 && prev_length <= length, "prev_length %lld outside [1, length]",
              (long long)prev_length);
  DSA_REQUIRE(k > 0 && k <= kMaxRun && k <= prev_length, "k=%lld must be in [1, min(4096, prev_length)]",
              (long long)k);
  DSA_REQUIRE(wave >= 0, "wave must be >= 0");
  // The sequential path merges the running k largest with a wave's keys in
  // LDS; the rounds' replay sorts in the workspace past its LDS.
  DSA_REQUIRE(wave == 0 || !legacy_paths_forced() || k + int64_t(wave) * block_size <= kMaxMerge,
              "k + wave * block_size exceeds %d on the sequential path", kMaxMerge);
  DSA_REQUIRE(key_dtype == DSA_DTYPE_BF16 || key_dtype == DSA_DTYPE_F16 || key_dtype == DSA_DTYPE_FP8_E4M3,
              "the temporal step takes fp16/bf16/fp8 keys (got %d)", key_dtype);
  DSA_REQUIRE(key_dtype != DSA_DTYPE_FP8_E4M3 || key_scales, "fp8 keys need key_scales");
  DSA_REQUIRE(reinterpret_cast<uintptr_t>(queries) % 16 == 0 && reinterpret_cast<uintptr_t>(keys) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(workspace) % 256 == 0,
              "queries, keys (16 B) and workspace (256 B) must be aligned");
  const int64_t blocks = (length + block_size - 1) / block_size;
  DSA_REQUIRE(blocks <= kMaxTemporalBlocks, "%lld blocks exceed %d", (long long)blocks, kMaxTemporalBlocks);
  return DSA_STATUS_OK;
}

}  // namespace dsa

using namespace dsa;

extern "C" int64_t dsa_temporal_workspace_bytes(int64_t batch, int64_t length, int64_t k, int32_t block_size) {
  if (batch <= 0 || length <= 0 || k <= 0 || block_size <= 0) return 0;
  return temporal_layout(nullptr, batch, length, k, block_size).bytes;
}

extern "C" int dsa_temporal_keys_loaded(const void* workspace, int64_t batch, int64_t length, int64_t k,
                                        int32_t block_size, int32_t* out, void* stream) {
  using namespace dsa;
  DSA_REQUIRE(workspace && out, "null pointer");
  DSA_REQUIRE(batch > 0 && length > 0 && k > 0 && block_size > 0, "bad shape");
  const TemporalWorkspace ws = temporal_layout(const_cast<void*>(workspace), batch, length, k, block_size);
  return check_hip(hipMemcpyAsync(out, ws.loaded, (size_t)batch * 4, hipMemcpyDeviceToDevice,
                                  static_cast<hipStream_t>(stream)),
                   "keys loaded copy");
}

extern "C" int dsa_temporal_step(const void* queries, const float* weights, const void* keys,
                                 int64_t key_stride, const float* key_scales, const float* prev_block_max,
                                 int64_t prev_length,
                                 const int64_t* prev_topk, const float* gamma, const double* block_margins,
                                 float* scores,
                                 uint8_t* evaluated_blocks, int64_t* out_topk, int32_t* qk_scored,
                                 int32_t* waits_given_up,
                                 int64_t batch, int64_t length, int64_t k, int32_t block_size,
                                 int32_t scan_order, int32_t wave, int32_t key_dtype, void* workspace,
                                 int64_t workspace_bytes, void* stream) {
  DSA_REQUIRE(queries && weights && keys && prev_block_max && prev_topk && (gamma || block_margins) && scores &&
                  evaluated_blocks && out_topk && qk_scored,
              "null pointer argument");
  if (int st = check_step(queries, keys, key_stride, key_scales, prev_length, batch, length, k, block_size, wave,
                          key_dtype, workspace))
    return st;
  DSA_REQUIRE(scan_order >= 0 && scan_order <= 2, "scan_order %d not in {0, 1, 2}", scan_order);
  const int64_t blocks = (length + block_size - 1) / block_size;
  const TemporalWorkspace ws = temporal_layout(workspace, batch, length, k, block_size);
  if (!workspace || workspace_bytes < ws.bytes)
    return fail(DSA_STATUS_WORKSPACE_TOO_SMALL, "the temporal step needs %lld workspace bytes", (long long)ws.bytes);
  TemporalArgs a = {};
  a.q = static_cast<const uint16_t*>(queries);
  a.w = weights;
  a.keys = static_cast<const uint8_t*>(keys);
  a.key_stride = key_stride;
  a.scales = key_scales;
  a.prev_max = prev_block_max;
  a.seeds = prev_topk;
  a.gamma = gamma;
  a.margins = block_margins;
  a.scores = scores;
  a.evaluated = evaluated_blocks;
  a.qk_scored = qk_scored;
  a.waits_given_up = waits_given_up;
  a.rows = (int32_t)batch;
  a.length = (int32_t)length;
  a.k = (int32_t)k;
  a.block_size = block_size;
  a.blocks = (int32_t)blocks;
  a.prev_length = (int32_t)prev_length;
  a.prev_blocks = (int32_t)((prev_length + block_size - 1) / block_size);
  a.scan_order = scan_order;
  a.ws = ws;
  return run_step(a, wave, key_dtype, out_topk, stream);
}

extern "C" int dsa_temporal_replay_step(const float* current_scores, int64_t score_stride,
                                        const float* prev_block_max, int64_t prev_length, const int64_t* prev_topk,
                                        const double* gamma, const float* order_key, float* scores,
                                        uint8_t* evaluated_blocks,
                                        int32_t* scan_order_out, int64_t* out_topk, int32_t* qk_scored, int64_t batch,
                                        int64_t length, int64_t k, int32_t block_size, int32_t scan_order,
                                        int32_t wave, void* workspace, int64_t workspace_bytes, void* stream) {
  DSA_REQUIRE(current_scores && prev_block_max && prev_topk && gamma && scores && evaluated_blocks && out_topk &&
                  qk_scored,
              "null pointer argument");
  DSA_REQUIRE(score_stride == 0 || score_stride >= length, "score_stride must be 0 or >= length");
  if (int st = check_step(nullptr, nullptr, length, nullptr, prev_length, batch, length, k, block_size, wave,
                          DSA_DTYPE_BF16, workspace))
    return st;
  DSA_REQUIRE(scan_order >= 0 && scan_order <= 3, "scan_order %d not in {0, 1, 2, 3}", scan_order);
  DSA_REQUIRE(scan_order != 3 || order_key, "scan order 3 needs order_key");
  const int64_t blocks = (length + block_size - 1) / block_size;
  const TemporalWorkspace ws = temporal_layout(workspace, batch, length, k, block_size);
  if (!workspace || workspace_bytes < ws.bytes)
    return fail(DSA_STATUS_WORKSPACE_TOO_SMALL, "the replay step needs %lld workspace bytes", (long long)ws.bytes);
  TemporalArgs a = {};
  a.source = current_scores;
  a.source_stride = score_stride;
  a.order_out = scan_order_out;
  a.order_key = order_key;
  a.key_stride = length;
  a.prev_max = prev_block_max;
  a.seeds = prev_topk;
  a.gamma_d = gamma;
  a.scores = scores;
  a.evaluated = evaluated_blocks;
  a.qk_scored = qk_scored;
  a.rows = (int32_t)batch;
  a.length = (int32_t)length;
  a.k = (int32_t)k;
  a.block_size = block_size;
  a.blocks = (int32_t)blocks;
  a.prev_length = (int32_t)prev_length;
  a.prev_blocks = (int32_t)((prev_length + block_size - 1) / block_size);
  a.scan_order = scan_order;
  a.ws = ws;
  return run_step(a, wave, DSA_DTYPE_BF16, out_topk, stream);
}

extern "C" int dsa_approx_step(const void* queries, const float* weights, const void* keys, int64_t key_stride,
                               const float* key_scales, const dsa_approx_policy* policy, const double* gamma_rows,
                               int64_t prev_length, const int64_t* prev_topk, float* last_max, float* ema,
                               float* volatility, int16_t* age, int16_t* cold_streak, int64_t state_stride,
                               float* scores, uint8_t* evaluated_blocks, int64_t* out_topk, int32_t* qk_scored,
                               int64_t batch, int64_t length, int64_t k, int32_t block_size, int32_t wave,
                               int32_t key_dtype, void* workspace, int64_t workspace_bytes, void* stream) {
  DSA_REQUIRE(queries && weights && keys && policy && prev_topk && last_max && ema && volatility && age &&
                  cold_streak && scores && evaluated_blocks && out_topk && qk_scored,
              "null pointer argument");
  if (int st = check_step(queries, keys, key_stride, key_scales, prev_length, batch, length, k, block_size, wave,
                          key_dtype, workspace))
    return st;
  DSA_REQUIRE(policy->risk_model == DSA_RISK_LAST_MAX || policy->risk_model == DSA_RISK_EMA,
              "risk_model %d unknown", policy->risk_model);
  DSA_REQUIRE(policy->order >= DSA_ORDER_ADDRESS && policy->order <= DSA_ORDER_BUCKET, "order %d unknown",
              policy->order);
  DSA_REQUIRE(policy->order != DSA_ORDER_BUCKET || policy->buckets >= 1, "bucket order needs buckets >= 1");
  DSA_REQUIRE(policy->recent_window >= 0, "recent_window must be >= 0");
  DSA_REQUIRE(policy->history == DSA_HISTORY_OWN, "a live step runs the own history (the teacher's needs the dense trace)");
  const int64_t blocks = (length + block_size - 1) / block_size;
  DSA_REQUIRE(state_stride >= blocks, "state_stride %lld < %lld blocks", (long long)state_stride, (long long)blocks);
  const TemporalWorkspace ws = temporal_layout(workspace, batch, length, k, block_size);
  if (!workspace || workspace_bytes < ws.bytes)
    return fail(DSA_STATUS_WORKSPACE_TOO_SMALL, "the approximate step needs %lld workspace bytes",
                (long long)ws.bytes);
  TemporalArgs a = {};
  a.q = static_cast<const uint16_t*>(queries);
  a.w = weights;
  a.keys = static_cast<const uint8_t*>(keys);
  a.key_stride = key_stride;
  a.scales = key_scales;
  a.seeds = prev_topk;
  a.scores = scores;
  a.evaluated = evaluated_blocks;
  a.qk_scored = qk_scored;
  a.rows = (int32_t)batch;
  a.length = (int32_t)length;
  a.k = (int32_t)k;
  a.block_size = block_size;
  a.blocks = (int32_t)blocks;
  a.prev_length = (int32_t)prev_length;
  a.prev_blocks = (int32_t)((prev_length + block_size - 1) / block_size);
  a.policy_mode = 1;
  a.ap = ApproxDev{last_max, ema, volatility, age, cold_streak, state_stride, gamma_rows, *policy};
  a.ws = ws;
  return run_step(a, wave, key_dtype, out_topk, stream);
}

extern "C" int dsa_approx_replay_step(const float* current_scores, int64_t score_stride,
                                      const float* current_block_max, const dsa_approx_policy* policy,
                                      const double* gamma_rows, int64_t prev_length,
                                      const int64_t* prev_topk, const int64_t* teacher_topk, float* last_max,
                                      float* ema, float* volatility,
                                      int16_t* age, int16_t* cold_streak, int64_t state_stride, float* scores,
                                      uint8_t* evaluated_blocks, int64_t* out_topk, int32_t* qk_scored,
                                      int64_t batch, int64_t length, int64_t k, int32_t block_size, int32_t wave,
                                      void* workspace, int64_t workspace_bytes, void* stream) {
  DSA_REQUIRE(current_scores && policy && prev_topk && last_max && ema && volatility && age && cold_streak && scores &&
                  evaluated_blocks && out_topk && qk_scored,
              "null pointer argument");
  DSA_REQUIRE(score_stride >= length, "score_stride < length");
  if (int st = check_step(nullptr, nullptr, length, nullptr, prev_length, batch, length, k, block_size, wave,
                          DSA_DTYPE_BF16, workspace))
    return st;
  DSA_REQUIRE(policy->risk_model == DSA_RISK_LAST_MAX || policy->risk_model == DSA_RISK_EMA,
              "risk_model %d unknown", policy->risk_model);
  DSA_REQUIRE(policy->order >= DSA_ORDER_ADDRESS && policy->order <= DSA_ORDER_CURRENT_MAX, "order %d unknown",
              policy->order);
  DSA_REQUIRE(policy->order != DSA_ORDER_CURRENT_MAX || current_block_max,
              "the current-max order needs current_block_max");
  DSA_REQUIRE(policy->order != DSA_ORDER_BUCKET || policy->buckets >= 1, "bucket order needs buckets >= 1");
  DSA_REQUIRE(policy->recent_window >= 0, "recent_window must be >= 0");
  DSA_REQUIRE(policy->history == DSA_HISTORY_OWN || policy->history == DSA_HISTORY_TEACHER, "history %d unknown",
              policy->history);
  DSA_REQUIRE(policy->history != DSA_HISTORY_TEACHER || teacher_topk, "the teacher history needs teacher_topk");
  const int64_t blocks = (length + block_size - 1) / block_size;
  DSA_REQUIRE(state_stride >= blocks, "state_stride %lld < %lld blocks", (long long)state_stride, (long long)blocks);
  const TemporalWorkspace ws = temporal_layout(workspace, batch, length, k, block_size);
  if (!workspace || workspace_bytes < ws.bytes)
    return fail(DSA_STATUS_WORKSPACE_TOO_SMALL, "the approximate replay step needs %lld workspace bytes",
                (long long)ws.bytes);
  TemporalArgs a = {};
  a.source = current_scores;
  a.source_stride = score_stride;
  a.order_key = current_block_max;
  a.key_stride = length;
  a.seeds = prev_topk;
  a.scores = scores;
  a.evaluated = evaluated_blocks;
  a.qk_scored = qk_scored;
  a.rows = (int32_t)batch;
  a.length = (int32_t)length;
  a.k = (int32_t)k;
  a.block_size = block_size;
  a.blocks = (int32_t)blocks;
  a.prev_length = (int32_t)prev_length;
  a.prev_blocks = (int32_t)((prev_length + block_size - 1) / block_size);
  a.policy_mode = 1;
  a.ap = ApproxDev{last_max, ema, volatility, age, cold_streak, state_stride, gamma_rows, *policy};
  a.teacher_topk = teacher_topk;
  a.ws = ws;
  return run_step(a, wave, DSA_DTYPE_BF16, out_topk, stream);
}

extern "C" int dsa_approx_init_state(const float* scores, int64_t score_stride, const int64_t* topk,
                                     float* last_max, float* ema, float* volatility, int16_t* age,
                                     int16_t* cold_streak, int64_t state_stride, int64_t batch, int64_t length,
                                     int64_t k, int32_t block_size, void* stream) {
  DSA_REQUIRE(scores && topk && last_max && ema && volatility && age && cold_streak, "null pointer argument");
  DSA_REQUIRE(batch > 0 && batch <= 65535, "batch %lld out of range", (long long)batch);
  DSA_REQUIRE(length > 0 && score_stride >= length, "length %lld / score_stride %lld invalid", (long long)length,
              (long long)score_stride);
  DSA_REQUIRE(k > 0 && k <= length, "k=%lld outside [1, length]", (long long)k);
  DSA_REQUIRE(block_size > 0, "block_size must be positive");
  const int64_t blocks = (length + block_size - 1) / block_size;
  DSA_REQUIRE(blocks <= kMaxTemporalBlocks, "%lld blocks exceed %d", (long long)blocks, kMaxTemporalBlocks);
  DSA_REQUIRE(state_stride >= blocks, "state_stride %lld < %lld blocks", (long long)state_stride, (long long)blocks);
  StateArgs s = {};
  s.scores = scores;
  s.score_stride = score_stride;
  s.topk = topk;
  s.ap = ApproxDev{last_max, ema, volatility, age, cold_streak, state_stride, nullptr, {}};
  s.length = (int32_t)length;
  s.blocks = (int32_t)blocks;
  s.block_size = block_size;
  s.k = (int32_t)k;
  s.state_blocks = (int32_t)blocks;
  hipLaunchKernelGGL(approx_state_kernel<kStateInit>, dim3(batch), dim3(1024), 0, static_cast<hipStream_t>(stream), s);
  return check_launch("approx_state_kernel");
}
