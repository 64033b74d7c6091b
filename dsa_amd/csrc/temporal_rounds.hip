// The dynamic temporal scan in rounds.
//
// The dynamic filter (replay.py:172-222, the threshold refreshed after every
// group of W scan positions to the k-th largest score evaluated so far) is
// sequential: whether the block at a position is kept depends on every
// decision before its group.  But the threshold never falls inside a scan:
// it is the k-th largest of a set that only grows (the running k largest
// starts as the seeds' scores), so the k-th largest at the start of a range
// of positions bounds every threshold inside that range from below.  A round
// over a range of positions therefore
//
//  1. scores, over the whole GPU, every block of the range whose bound clears
//     that floor -- a superset of the blocks the scan keeps there -- writing
//     their scores and listing each non-seed key above the floor under its
//     threshold group (temporal_round_kernel);
//  2. replays the scan over the range in one workgroup per row, group by
//     group: the group's decisions against the exact threshold, then the
//     listed keys of its kept blocks join the running k largest; scored
//     blocks that the replay prunes get -inf back, seeds excepted
//     (temporal_resolve_kernel).  No threshold of the round exceeds the k-th
//     largest of all the round's keys, and none falls below the one in force,
//     so a run of groups whose every bound lies outside that interval is
//     decided, and joined, in one step of the replay.
//
// The decisions, the evaluated keys and their scores are those of the
// sequential scan (the persistent and per-wave paths of temporal.hip) bit for
// bit.  The blocks scored and then pruned are the price of the parallel
// scoring: the rounds split the scan at group boundaries so that later rounds
// start from a higher floor.
//
// The running k largest in the replay (one wave, no barriers): a count per
// 12-bit bin of the ordered key (E), the bin of the k-th largest (the cut
// bin), the number of keys above that bin, the keys at or above it (V) and the
// keys in it (B).  A bound outside the cut bin is decided by the bins alone;
// one inside it needs the exact k-th largest, a select among B's keys, which
// stays valid until keys join.  When the count above the cut bin reaches k the
// cut moves up and V and B are rebuilt from V.
#include <cstdlib>
#include <mutex>
#include <vector>

#include "status.hpp"
#include "temporal.hpp"

namespace dsa {
namespace {

constexpr int kRoundThreads = 256;
constexpr int kRoundWaves = kRoundThreads / kWave;
constexpr int kRoundParts = 2;            // kRoundKeys spans of positions per wide workgroup
constexpr int64_t kRoundWideSpans = 192;  // spans in a round from which its workgroups are wide
static_assert(kRoundWaves * kRoundWaveKeys == kRoundKeys, "two 64-key units per scoring wave");

#ifdef DSA_PHASE_TRACE
// Per row (trace builds only): wall-clock ticks of the replay's phases and
// event counts: 0 group loop, 1 decisions, 2 exact selects, 3 select count
// (low half) and cut move count (high half), 4 joins, 5 cut moves, 6 listed
// keys (bits 0-23), loop steps (bits 24-47) and rounds that sorted in the
// workspace (high 16), 7 setup
// (kernel start to the group loop).  Accumulated in registers by wave 0 and added to memory once per
// launch, so that the timing itself adds no memory round trip to the loop.
__device__ uint64_t g_trace_resolve[kTraceWgs * kTraceMarks];
#define RESOLVE_T0(v) uint64_t v = wall_clock64()
#define RESOLVE_ADD(i, t0) \
  do {                     \
    trace_acc[i] += wall_clock64() - (t0); \
  } while (0)
#define RESOLVE_COUNT(i, n) \
  do {                      \
    trace_acc[i] += (n);    \
  } while (0)
#else
#define RESOLVE_T0(v) \
  do {                \
  } while (0)
#define RESOLVE_ADD(i, t0) \
  do {                     \
  } while (0)
#define RESOLVE_COUNT(i, n) \
  do {                      \
  } while (0)
#endif

struct RoundPlan {
  int32_t pos_begin, pos_end;  // scan positions of the round (whole groups)
  int32_t per_wg;              // scan positions per scoring workgroup
  int32_t wgs_per_row;
  int32_t group;         // scan positions per threshold group (the wave W)
  int32_t first_round;   // the round's first group is the scan's first (seed threshold)
  int32_t last_round;    // no round follows: the running k largest is not written back
  int32_t round;         // index of the round (its list count)
};

// The key of the largest float at or below a float64 bound: for every float
// t that is not NaN, (bound < t) == (upper_key(bound) < key(t)).  A NaN bound
// (never pruned) maps to the largest key.
__device__ __forceinline__ uint32_t upper_key(double bound) {
  if (__builtin_isnan(bound)) return 0xffffffffu;
  return float_to_ordered(__double2float_rd(bound));
}

// Ordered keys of NaN floats (a threshold that prunes nothing: `U < NaN` is
// false), and the pruning test `U < t` on keys.
__device__ __forceinline__ bool nan_key(uint32_t t) { return t > 0xff800000u || t < 0x007fffffu; }
__device__ __forceinline__ bool prunes(uint32_t bound_key, uint32_t t) { return !nan_key(t) && bound_key < t; }

// The running k largest that round r reads (and round r - 1 wrote): two
// buffers of [rows][k], used alternately; the seed pass writes the first.
__device__ __forceinline__ size_t run_offset(const TemporalArgs& a, int round, int row) {
  return ((size_t)(round & 1) * a.rows + row) * a.k;
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// Calls use(i, load(i)) for i = first, first + stride, ... below n, the loads
// of each batch of kBatch indices issued before any of them is used (a load
// past n re-reads the batch's first index), so that a thread's loads cost one
// memory latency per batch instead of one per index.
template <int kBatch, class Load, class Use>
__device__ __forceinline__ void batched(uint32_t first, uint32_t n, uint32_t stride, Load load, Use use) {
  for (uint32_t i0 = first; i0 < n; i0 += kBatch * stride) {
    decltype(load(i0)) v[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const uint32_t i = i0 + (uint32_t)j * stride;
      v[j] = load(i < n ? i : i0);
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const uint32_t i = i0 + (uint32_t)j * stride;
      if (i < n) use(i, v[j]);
    }
  }
}

// ---------------------------------------------------------------------------
// 1. Scoring.  Workgroup (row, part) covers scan positions
// [pos_begin + part * per_wg, + per_wg) of the round (kParts x kRoundKeys
// keys): the blocks there whose bound clears the row's floor are
// cut into 16-key tiles, which the four waves score four at a time (one MFMA
// unit) with the dense kernel's tile code, each wave's units streamed through
// two register buffers.  Every scored key's score goes to the scores row; a
// non-seed key above the floor is listed, with its group, in the row's list
// of the round (one atomic reservation per wave).
// ---------------------------------------------------------------------------
template <class Tag, class KF, int kParts>
__global__ __launch_bounds__(kRoundThreads) void temporal_round_kernel(TemporalArgs a, RoundPlan rp) {
  constexpr int kRoundTiles = kParts * kRoundKeys / 16;           // 16-key tiles a workgroup scores at most
  constexpr int kRoundWaveUnits = kRoundTiles / 4 / kRoundWaves;  // 64-key units per wave at most
  __shared__ uint32_t s_tile_key[kRoundTiles];
  __shared__ uint16_t s_tile_group[kRoundTiles];
  __shared__ uint16_t s_tile_seeds[kRoundTiles];  // the tile's seeds (scored by the seed pass: not loaded again)
  __shared__ __align__(16) uint32_t s_wsum[kRoundWaves];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15;
  const int g = lane >> 4;
  const int row = blockIdx.x / rp.wgs_per_row;
  const int part = blockIdx.x % rp.wgs_per_row;
  const int p0 = rp.pos_begin + part * rp.per_wg;
  const int p1 = min(p0 + rp.per_wg, rp.pos_end);
  const int nb = a.blocks;
  const int bs = a.block_size;
  const int L = a.length;

  // The query tiles, then the position's block and bound (one position per
  // thread): their loads are in flight together.
  uint4 qa[4][4] = {};
  float wr[4][4] = {};
  if (!a.source)
    load_dense_head_tiles<4, KF::kNaturalK>(a.q + (size_t)row * kHeads * kHeadDim, a.w + (size_t)row * kHeads, r, g,
                                            qa, wr);
  const uint32_t floor_key = a.ws.floor[row];
  int blk = 0;
  uint32_t my_tiles = 0;
  const int p = p0 + tid;
  if (p < p1) {
    blk = (int)a.ws.order[(size_t)row * nb + p];
    const double up = a.ws.upper_pos[(size_t)row * nb + p];
    if (!prunes(upper_key(up), floor_key)) my_tiles = (uint32_t)((min(L, (blk + 1) * bs) - blk * bs + 15) >> 4);
  }
  // The seed-mask words of the block's first eight tiles, read before the
  // scan so that their latency overlaps it (one round trip, not one per tile).
  const uint32_t words = (uint32_t)(L + 31) / 32u;
  const uint32_t* mask = a.ws.seed_mask + (size_t)row * words;
  const uint32_t key_first = (uint32_t)(blk * bs);
  const uint32_t wbase = key_first >> 5;
  const bool odd = (key_first & 16u) != 0u;  // the block starts in a word's upper half
  uint32_t mw[5];
#pragma unroll
  for (int i = 0; i < 5; ++i) mw[i] = my_tiles ? mask[min(wbase + (uint32_t)i, words - 1u)] : 0u;
  uint32_t total = 0;
  const uint32_t first = block_excl_scan<kRoundWaves>(my_tiles, s_wsum, total);
  const uint16_t group = (uint16_t)(p / rp.group);
#pragma unroll
  for (uint32_t j = 0; j < 8u; ++j) {
    if (j >= my_tiles) break;
    const uint32_t key0 = key_first + 16u * j;  // tiles are 16-key aligned
    const uint32_t word = odd ? mw[(j + 1u) >> 1] : mw[j >> 1];
    s_tile_key[first + j] = key0;
    s_tile_group[first + j] = group;
    s_tile_seeds[first + j] = (uint16_t)(word >> (key0 & 16u));
  }
  for (uint32_t j = 8u; j < my_tiles; ++j) {  // blocks of more than 128 keys
    const uint32_t key0 = key_first + 16u * j;
    s_tile_key[first + j] = key0;
    s_tile_group[first + j] = group;
    s_tile_seeds[first + j] = (uint16_t)(mask[key0 >> 5] >> (key0 & 16u));
  }
  __syncthreads();

  // recorded scores: an empty key buffer (every load reads 0 without touching memory)
  const BufferRsrc keys = make_buffer(a.source ? nullptr : a.keys + (size_t)row * a.key_stride * KF::kRowBytes,
                                      a.source ? 0u : (uint32_t)L * KF::kRowBytes);
  const BufferRsrc out = make_buffer(a.scores + (size_t)row * L, (uint32_t)L * 4u);
  if constexpr (kParts == 1) {
    // Two units per wave at most: both loaded before either is scored.
    const int units = (int)(total + 3) >> 2;
    const int t_res = lane >> 4;  // the tile of this lane's result
    // A seed's row is not loaded (its score is the seed pass's, already in
    // the scores row).
    uint4 buf[2][4][KF::kRaw];
    float scale[2] = {1.f, 1.f};
    int key_res[2];
    bool valid[2];
  #pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int u = wave + kRoundWaves * h;
  #pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int ti = 4 * u + t;
        int key = (int)kFarKey;
        if (ti < (int)total && !((s_tile_seeds[ti] >> r) & 1u)) key = (int)s_tile_key[ti] + r;
        KF::load_buf(keys, key < L ? key : (int)kFarKey, g, buf[h][t]);
      }
      const int ti = 4 * u + t_res;
      valid[h] = ti < (int)total && !((s_tile_seeds[ti] >> r) & 1u);
      key_res[h] = valid[h] ? (int)s_tile_key[ti] + r : 0;
      valid[h] = valid[h] && key_res[h] < L;
      if constexpr (KF::kScaled)
        if (valid[h] && !a.source) scale[h] = a.scales[(size_t)row * ((a.key_stride + 127) / 128) + (key_res[h] >> 7)];
    }
    uint32_t listed = 0;
    uint64_t entry[2] = {0ull, 0ull};
    uint32_t at[2] = {0u, 0u};
    bool take[2] = {false, false};
  #pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int u = wave + kRoundWaves * h;
      if (u >= units) break;  // uniform over the wave
      float v;
      if (a.source) {
        v = valid[h] ? a.source[(size_t)row * a.source_stride + key_res[h]] : 0.f;
      } else {
        float sc[4];
  #pragma unroll
        for (int t = 0; t < 4; ++t) sc[t] = tile_contrib<Tag, 4, KF>(qa, wr, buf[h][t]);
        v = unit_reduce(sc, g) * scale[h];
      }
      const int key = key_res[h];
      if (valid[h]) buffer_store_f32(out, (uint32_t)key * 4u, v);
      const uint32_t o = float_to_ordered(v);
      take[h] = valid[h] && o > floor_key;
      const uint64_t m = __ballot(take[h]);
      if (take[h]) entry[h] = ((uint64_t)s_tile_group[4 * u + t_res] << 49) | ((uint64_t)key << 32) | o;
      at[h] = listed + lanes_below(m);
      listed += (uint32_t)__builtin_popcountll(m);
    }
    // One reservation per wave in the row's list of this round, and the key
    // rows the wave loaded.
    uint32_t base = 0;
    if (lane == 0 && listed)
      base = __hip_atomic_fetch_add(&a.ws.list_total[(size_t)row * kMaxRounds + rp.round], listed, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t rows_loaded = (uint32_t)__builtin_popcountll(__ballot(valid[0])) +
                                 (uint32_t)__builtin_popcountll(__ballot(valid[1]));
    if (lane == 0 && rows_loaded && !a.source)
      __hip_atomic_fetch_add(a.ws.loaded + row, rows_loaded, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
    uint64_t* list = a.ws.entries + (size_t)row * a.ws.list_capacity + base;
  #pragma unroll
    for (int h = 0; h < 2; ++h)
      if (take[h]) list[at[h]] = entry[h];
  } else {
    const int units = (int)(total + 3) >> 2;
    const int t_res = lane >> 4;  // the tile of this lane's result
    // The wave's units (u = wave, wave + kRoundWaves, ...) stream through two
    // register buffers: the next unit's loads are issued before the current one
    // is scored.  A seed's row is not loaded (its score is the seed pass's,
    // already in the scores row).
    const int count = units > wave ? (units - wave + kRoundWaves - 1) / kRoundWaves : 0;
    auto load_unit = [&](int u, uint4 (&b)[4][KF::kRaw], float& scale) {
  #pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int ti = 4 * u + t;
        int key = (int)kFarKey;
        if (ti < (int)total && !((s_tile_seeds[ti] >> r) & 1u)) key = (int)s_tile_key[ti] + r;
        KF::load_buf(keys, key < L ? key : (int)kFarKey, g, b[t]);
      }
      scale = 1.f;
      if constexpr (KF::kScaled) {
        const int ti = 4 * u + t_res;
        if (ti < (int)total && !a.source) {
          const int key = (int)s_tile_key[ti] + r;
          scale = a.scales[(size_t)row * ((a.key_stride + 127) / 128) + (min(key, L - 1) >> 7)];
        }
      }
    };
    uint4 buf[2][4][KF::kRaw];
    float scale[2] = {1.f, 1.f};
    if (count > 0) load_unit(wave, buf[0], scale[0]);
    uint32_t listed = 0, rows_loaded = 0, take_bits = 0;
    uint64_t entry[kRoundWaveUnits];
    uint32_t at[kRoundWaveUnits];
  #pragma unroll
    for (int i = 0; i < kRoundWaveUnits; ++i) {
      entry[i] = 0ull;
      at[i] = 0u;
      if (i < count) {  // uniform over the wave
        const int u = wave + kRoundWaves * i;
        if (i + 1 < count) load_unit(u + kRoundWaves, buf[(i + 1) & 1], scale[(i + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
        const int ti = 4 * u + t_res;
        bool valid = ti < (int)total && !((s_tile_seeds[ti] >> r) & 1u);
        const int key = valid ? (int)s_tile_key[ti] + r : 0;
        valid = valid && key < L;
        float v;
        if (a.source) {
          v = valid ? a.source[(size_t)row * a.source_stride + key] : 0.f;
        } else {
          float sc[4];
  #pragma unroll
          for (int t = 0; t < 4; ++t) sc[t] = tile_contrib<Tag, 4, KF>(qa, wr, buf[i & 1][t]);
          v = unit_reduce(sc, g) * scale[i & 1];
        }
        if (valid) buffer_store_f32(out, (uint32_t)key * 4u, v);
        const uint32_t o = float_to_ordered(v);
        const bool take = valid && o > floor_key;
        const uint64_t m = __ballot(take);
        if (take) entry[i] = ((uint64_t)s_tile_group[ti] << 49) | ((uint64_t)key << 32) | o;
        at[i] = listed + lanes_below(m);
        take_bits |= take ? 1u << i : 0u;
        listed += (uint32_t)__builtin_popcountll(m);
        rows_loaded += (uint32_t)__builtin_popcountll(__ballot(valid));
      }
    }
    // One reservation per wave in the row's list of this round, and the key
    // rows the wave loaded.
    uint32_t base = 0;
    if (lane == 0 && listed)
      base = __hip_atomic_fetch_add(&a.ws.list_total[(size_t)row * kMaxRounds + rp.round], listed, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
    if (lane == 0 && rows_loaded && !a.source)
      __hip_atomic_fetch_add(a.ws.loaded + row, rows_loaded, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
    uint64_t* list = a.ws.entries + (size_t)row * a.ws.list_capacity + base;
  #pragma unroll
    for (int i = 0; i < kRoundWaveUnits; ++i)
      if ((take_bits >> i) & 1u) list[at[i]] = entry[i];
  }
}

// ---------------------------------------------------------------------------
// 2. The replay of one row over the round's positions (one workgroup).
//
// Setup, by every thread: the running k largest (run, joined from the start)
// and every listed key of the round are sorted by bin of their ordered key,
// counting from the row's floor (every such key is at or above it) with bins
// as fine as the span of the keys allows, 4096 in all: bin b holds slots
// [end(b - 1), end(b)).  The listed keys are also sorted by threshold group
// (items: slot | block << 18).
//
// Then wave 0 walks the groups: decisions against the threshold in force
// (the seed threshold for the scan's first group; after it the k-th largest
// joined key), then the listed keys of kept blocks join.  The threshold is
// tracked by the bin holding it (the cut bin), the count of joined keys above
// that bin and E, the joined keys per bin: a bound outside the cut bin is
// decided by bins alone, one inside it needs the exact k-th largest, a select
// among the cut bin's joined keys.
// ---------------------------------------------------------------------------
constexpr int kResolveThreads = 512;
constexpr int kResolveWaves = kResolveThreads / kWave;
constexpr int kSortCap = 8192;  // keys the replay sorts in LDS (more: in the workspace)
constexpr int kBins = 4096;
constexpr int kCutDigits = 1024;  // 10-bit digits of the select inside the cut bin
constexpr int kKeyBatch = 8;      // key values per thread in flight in the replay's first read

struct ResolveShared {
  uint32_t val[kSortCap];   // ordered keys, by bin
  uint32_t item[kSortCap];  // listed keys by group: slot | block << 18
  uint8_t join[kSortCap];   // joined (evaluated) flag of each slot
  uint32_t end[kBins];      // past-the-end slot of each bin (after the scatter)
  alignas(16) uint32_t E[kBins];  // joined keys per bin (read four at a time)
  uint32_t gend[kMaxTemporalBlocks];  // past-the-end item of each group (after the scatter)
  uint32_t uk[kMaxTemporalBlocks];    // bound key at each of the round's positions
  uint16_t blk[kMaxTemporalBlocks];   // block at each
  uint8_t kept[kMaxTemporalBlocks];   // by block id
  uint16_t resets[kMaxTemporalBlocks];
  // Positions whose bound is at or below the upper edge of the bin holding
  // the k-th largest of every key of the round (the only ones a threshold of
  // the round can prune), in position order, with their bound keys.
  uint32_t risky_uk[kMaxTemporalBlocks];
  uint16_t risky_pos[kMaxTemporalBlocks];
  uint32_t digits[kCutDigits];
  uint32_t wsum[kResolveWaves];
  uint32_t above, nreset, tau, cut_bin, n_out, bin_hi, n_risky;
};

// The j-th largest (1-based) of the joined keys in slots [s0, s1) of bin `bin`
// (keys base .. base + 2^shift - 1), by one wave: a bitonic sort across the
// lanes for at most 64 slots, else radix digits of the key's offset from the
// bin's base (10 bits, then the rest).
template <class P8, class P32>
__device__ __forceinline__ uint32_t cut_select(P32 val, P8 join, uint32_t s0, uint32_t s1, uint32_t j, uint32_t base, uint32_t shift,
                               uint32_t* digits) {
  const uint32_t lane = lane_id();
  const uint32_t n = s1 - s0;
  if (n <= (uint32_t)kWave) {
    uint32_t v = 0u;  // 0 sorts last
    if (lane < n && join[s0 + lane]) v = val[s0 + lane];
#pragma unroll
    for (int size = 2; size <= kWave; size <<= 1) {
#pragma unroll
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        const uint32_t o = (uint32_t)__shfl_xor((int)v, stride, kWave);
        const bool lower = (lane & (uint32_t)stride) == 0;
        const bool descending = (lane & (uint32_t)size) == 0;
        v = (lower == descending) ? max(v, o) : min(v, o);
      }
    }
    return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)(j - 1));
  }
  const uint32_t lo_bits = shift > 10 ? shift - 10 : 0;  // bits below the first digit
  uint32_t want = j;
  uint32_t hi = 0;
#pragma unroll 1
  for (int pass = 0; pass < 2; ++pass) {
    if (pass == 1 && lo_bits == 0) break;
    for (int i = (int)lane; i < kCutDigits; i += kWave) digits[i] = 0;
    wave_sync();
    for (uint32_t i = s0 + lane; i < s1; i += kWave) {
      if (!join[i]) continue;
      const uint32_t d = val[i] - base;
      if (pass == 0)
        __hip_atomic_fetch_add(&digits[d >> lo_bits], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      else if ((d >> lo_bits) == hi)
        __hip_atomic_fetch_add(&digits[d & ((1u << lo_bits) - 1u)], 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    wave_sync();
    const Locate loc = wave_locate<kCutDigits / kWave>(digits, want, false);
    wave_sync();
    if (pass == 0) {
      hi = loc.digit;
      want = loc.rem;
      if (lo_bits == 0) return base + hi;
    } else {
      return base + (hi << lo_bits) + loc.digit;
    }
  }
  return base + (hi << lo_bits);
}

template <bool kSpill>
__device__ __forceinline__ void resolve_row(const TemporalArgs& a, const RoundPlan& rp, ResolveShared& sh,
                                            uint32_t n_listed, uint32_t max_key, uint32_t floor_key,
                                            uint32_t seed_tau, uint64_t t_start) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int row = blockIdx.x;
  const int nb = a.blocks;
  const int k = a.k;
  const int W = rp.group;
  const int g_begin = rp.pos_begin / W;
  const int n_groups = (rp.pos_end + W - 1) / W - g_begin;
  const int n_pos = rp.pos_end - rp.pos_begin;
  const uint32_t span = max_key - floor_key;
  const uint32_t shift = span < (uint32_t)kBins ? 0u : 32u - (uint32_t)__builtin_clz(span) - 12u;
  const size_t spill_at = (size_t)row * a.ws.spill_capacity;
  uint32_t* val = kSpill ? a.ws.spill_val + spill_at : sh.val;
  uint32_t* item = kSpill ? a.ws.spill_item + spill_at : sh.item;
  uint8_t* join = kSpill ? a.ws.spill_join + spill_at : sh.join;
  const uint32_t* run = a.ws.run + run_offset(a, rp.round, row);
  const uint64_t* list = a.ws.entries + (size_t)row * a.ws.list_capacity;
  auto each_run = [&](auto f) {
    batched<4>((uint32_t)tid, (uint32_t)k, kResolveThreads, [&](uint32_t i) { return run[i]; },
               [&](uint32_t, uint32_t v) { f(v); });
  };
  auto each_listed = [&](auto f) {
    batched<4>((uint32_t)tid, n_listed, kResolveThreads, [&](uint32_t e) { return list[e]; },
               [&](uint32_t, uint64_t x) { f(x); });
  };

  // Bin and group counts (E counts the joined keys: run's).
  for (int i = tid; i < kBins; i += kResolveThreads) {
    sh.end[i] = 0;
    sh.E[i] = 0;
  }
  for (int i = tid; i < n_groups; i += kResolveThreads) sh.gend[i] = 0;
  if (tid == 0) {
    sh.above = 0;
    sh.bin_hi = kBins - 1;
  }
  __syncthreads();
  uint32_t above = 0;
  each_run([&](uint32_t v) {
    const uint32_t b = (v - floor_key) >> shift;
    __hip_atomic_fetch_add(&sh.end[b], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __hip_atomic_fetch_add(&sh.E[b], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    above += b > 0 ? 1u : 0u;
  });
  for (int off = 32; off > 0; off >>= 1) above += (uint32_t)__shfl_xor((int)above, off, kWave);
  if (lane == 0 && above) __hip_atomic_fetch_add(&sh.above, above, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  each_listed([&](uint64_t x) {
    const uint32_t b = ((uint32_t)x - floor_key) >> shift;
    __hip_atomic_fetch_add(&sh.end[b], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __hip_atomic_fetch_add(&sh.gend[(int)(x >> 49) - g_begin], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  });
  __syncthreads();
  // Exclusive scans: end[b] <- first slot of bin b, gend[g] <- first item of
  // group g (the scatter's cursors; past it they hold each one's end).
  {
    constexpr int kPer = kBins / kResolveThreads;
    uint32_t c[kPer];
    uint32_t sum = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      c[j] = sh.end[tid * kPer + j];
      sum += c[j];
    }
    uint32_t total;
    uint32_t before = block_excl_scan<kResolveWaves>(sum, sh.wsum, total);
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      // The bin of the k-th largest of all keys (total - before keys sit in
      // bins at or above this one): no threshold of the round lies above it.
      if (c[j] && total - before >= (uint32_t)k && total - before - c[j] < (uint32_t)k) sh.bin_hi = tid * kPer + j;
      sh.end[tid * kPer + j] = before;
      before += c[j];
    }
    __syncthreads();
    // Group starts, and the positions a threshold of the round could prune
    // (bound key at or below the upper edge of the k-th largest's bin),
    // compacted in position order: both counts scanned in one word (listed
    // keys below 2^18 in the low bits, positions below 2^12 from bit 19).
    const uint64_t hi_edge = (uint64_t)floor_key + ((uint64_t)(sh.bin_hi + 1) << shift) - 1ull;
    constexpr int kGPer = kMaxTemporalBlocks / kResolveThreads;
    uint32_t gc[kGPer];
    bool risky[kGPer];
    uint32_t gsum = 0;
#pragma unroll
    for (int j = 0; j < kGPer; ++j) {
      const int gi = tid * kGPer + j;
      gc[j] = gi < n_groups ? sh.gend[gi] : 0u;
      risky[j] = gi < n_pos && (uint64_t)sh.uk[gi] <= hi_edge;
      gsum += gc[j] + (risky[j] ? 1u << 19 : 0u);
    }
    uint32_t gbefore = block_excl_scan<kResolveWaves>(gsum, sh.wsum, total);
    uint32_t rbefore = gbefore >> 19;
    gbefore &= (1u << 19) - 1u;
#pragma unroll
    for (int j = 0; j < kGPer; ++j) {
      const int gi = tid * kGPer + j;
      if (gi < n_groups) sh.gend[gi] = gbefore;
      gbefore += gc[j];
      if (risky[j]) {
        sh.risky_pos[rbefore] = (uint16_t)gi;
        sh.risky_uk[rbefore] = sh.uk[gi];
        ++rbefore;
      }
    }
    if (tid == 0) sh.n_risky = total >> 19;
  }
  __syncthreads();
  // Scatter: run's keys joined, listed keys not yet; listed keys' items by group.
  each_run([&](uint32_t v) {
    const uint32_t slot = __hip_atomic_fetch_add(&sh.end[(v - floor_key) >> shift], 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_WORKGROUP);
    val[slot] = v;
    join[slot] = 1;
  });
  each_listed([&](uint64_t x) {
    const uint32_t v = (uint32_t)x;
    const uint32_t slot = __hip_atomic_fetch_add(&sh.end[(v - floor_key) >> shift], 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_WORKGROUP);
    val[slot] = v;
    join[slot] = 0;
    const uint32_t blk = (uint32_t)((x >> 32) & 0x1ffffu) / (uint32_t)a.block_size;
    const uint32_t at = __hip_atomic_fetch_add(&sh.gend[(int)(x >> 49) - g_begin], 1u, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_WORKGROUP);
    item[at] = slot | (blk << 18);
  });
  __syncthreads();

  if (wave == 0) {
#ifdef DSA_PHASE_TRACE
    uint64_t trace_acc[kTraceMarks] = {};
    trace_acc[7] = wall_clock64() - t_start;
    trace_acc[6] = n_listed + ((uint64_t)(kSpill ? 1 : 0) << 48);
#endif
    uint32_t bin = 0;  // the cut bin: the floor (the k-th largest) is in bin 0
    uint32_t cut_above = sh.above;
    uint32_t tau = floor_key;
    bool tau_ok = true;
    uint32_t nreset = 0;
    RESOLVE_T0(t_all);
    auto bin_start = [&](uint32_t b) { return b ? sh.end[b - 1] : 0u; };
    auto exact_tau = [&]() {
      if (!tau_ok) {
        RESOLVE_T0(t_sel);
        tau = cut_select(val, join, bin_start(bin), sh.end[bin], (uint32_t)k - cut_above, floor_key + (bin << shift),
                         shift, sh.digits);
        tau_ok = true;
        RESOLVE_ADD(2, t_sel);
        RESOLVE_COUNT(3, 1ull);
      }
      return tau;
    };
    // Read ahead of each step: its first 64 decision inputs, and the items
    // of its first 256 listed keys (items are stored by group, so the next
    // step's start slot is this step's end), whose values are then read
    // while the step's decisions are made.  Reads past a step's end are
    // harmless (items of later groups, or the last item again) and unused.
    uint32_t pf_uk = 0u;
    int pf_blk = 0;
    auto prefetch = [&](int gi) {
      const int qc = max(min(gi * W + lane, n_pos - 1), 0);
      pf_uk = sh.uk[qc];
      pf_blk = (int)sh.blk[qc];
    };
    // (With no listed keys the read of item 0 is stale, so its slot and block
    // are replaced by 0: slot 0 holds a run key, block 0 exists.)
    const uint32_t item_last = n_listed ? n_listed - 1u : 0u;
    constexpr int kJoinHalves = 4;  // listed keys per lane per join pass
    uint32_t pf_it[kJoinHalves];
    auto prefetch_items = [&](uint32_t start) {
#pragma unroll
      for (int h = 0; h < kJoinHalves; ++h) {
        const uint32_t it = item[min(start + (uint32_t)(h * kWave + lane), item_last)];
        pf_it[h] = n_listed ? it : 0u;
      }
    };
    prefetch(0);
    prefetch_items(0u);
    uint32_t i0 = 0u;  // the group's first item
    // Positions whose decision is the same under every threshold between the
    // cut bin's lower edge (no later threshold is below it) and hi_edge (none
    // is above it): bound above hi_edge, kept; below the lower edge, pruned
    // (when neither edge admits a NaN threshold).  Only risky positions can
    // be open; rc is the first risky one that may still be.
    const uint64_t hi_edge = (uint64_t)floor_key + ((uint64_t)(sh.bin_hi + 1) << shift) - 1ull;
    const uint32_t n_risky = sh.n_risky;
    uint32_t rc = 0u;
    for (int gi = 0, g_end = 1; gi < n_groups; gi = g_end) {
      // The step covers group gi and every following group with no open
      // position: their decisions, and then their joins, need no threshold
      // beyond the one group gi is decided by.
      g_end = gi + 1;
      if (!(rp.first_round && gi == 0)) {
        const uint64_t lo_edge = (uint64_t)floor_key + ((uint64_t)bin << shift);
        const bool can_prune = lo_edge >= 0x007fffffull && hi_edge <= 0xff800000ull;
        const uint32_t q_first = (uint32_t)(gi * W);
        int g_open = n_groups;
        while (rc < n_risky) {
          const uint32_t i = rc + (uint32_t)lane;
          uint32_t pos = 0u;
          bool open = false;
          if (i < n_risky) {
            pos = sh.risky_pos[i];
            open = pos >= q_first && !(can_prune && (uint64_t)sh.risky_uk[i] < lo_edge);
          }
          const uint64_t m = __ballot(open);
          if (m) {
            g_open = __builtin_amdgcn_readlane((int)pos, (int)__builtin_ctzll(m)) / W;
            break;
          }
          rc += kWave;  // every entry is decided already or pruned at every later threshold
        }
        g_end = max(g_open, gi + 1);
      }
      RESOLVE_COUNT(6, 1ull << 24);
      const uint32_t i1 = sh.gend[g_end - 1];
      uint32_t pf_v[kJoinHalves];
#pragma unroll
      for (int h = 0; h < kJoinHalves; ++h) pf_v[h] = val[pf_it[h] & 0x3ffffu];
      const int q0 = gi * W;
      const int q1 = min(g_end * W, n_pos);
      const bool seed_group = rp.first_round && gi == 0;
      // The cut bin's keys, and whether NaN keys can fall in it (then every
      // decision takes the exact threshold).
      const uint64_t lo = (uint64_t)floor_key + ((uint64_t)bin << shift);
      const uint64_t hi = lo + (1ull << shift) - 1ull;
      const bool finite_bin = lo >= 0x007fffffull && hi <= 0xff800000ull;
      RESOLVE_T0(t_dec);
      for (int c0 = q0; c0 < q1; c0 += kWave) {
        const int q = c0 + lane;
        const bool active = q < q1;
        uint32_t uk = pf_uk;
        int blk = pf_blk;
        if (c0 != q0) {  // (read for every lane, clamped: no branch around the reads)
          const int qc = min(q, n_pos - 1);
          uk = sh.uk[qc];
          blk = (int)sh.blk[qc];
        }
        int verdict = 2;  // 0 pruned, 1 kept, 2 needs the exact threshold
        if (seed_group) {
          verdict = prunes(uk, seed_tau) ? 0 : 1;
        } else if (finite_bin) {
          verdict = uk < lo ? 0 : (uk > hi ? 1 : 2);
        }
        if (__ballot(active && verdict == 2)) {
          const uint32_t t = exact_tau();
          if (verdict == 2) verdict = prunes(uk, t) ? 0 : 1;
        }
        if (active) {
          a.evaluated[(size_t)row * nb + blk] = (uint8_t)verdict;
          sh.kept[blk] = (uint8_t)verdict;
        }
        const bool reset = active && verdict == 0 && !prunes(uk, floor_key);
        const uint64_t m = __ballot(reset);
        if (reset) sh.resets[nreset + lanes_below(m)] = (uint16_t)blk;
        nreset += (uint32_t)__builtin_popcountll(m);
      }
      wave_sync();
      prefetch(g_end);
      RESOLVE_ADD(1, t_dec);
      // The kept blocks' listed keys join, 256 at a time: the first 256 from
      // the values read ahead, the rest (long steps) read here, items and
      // values of all four quarters issued before any is used.
      RESOLVE_T0(t_join);
      auto join_keys = [&](uint32_t c0, const uint32_t (&it)[kJoinHalves], const uint32_t (&v)[kJoinHalves]) {
        // (Every item read is a valid one, so the flags are read for all
        // lanes at once, with no branch between the reads.)
        uint32_t b[kJoinHalves], kb[kJoinHalves];
        bool in[kJoinHalves];
#pragma unroll
        for (int h = 0; h < kJoinHalves; ++h) kb[h] = sh.kept[it[h] >> 18];
#pragma unroll
        for (int h = 0; h < kJoinHalves; ++h) {
          b[h] = (v[h] - floor_key) >> shift;
          in[h] = (c0 + (uint32_t)(h * kWave + lane) < i1) & (kb[h] != 0u);
        }
        bool reaches = false;
#pragma unroll
        for (int h = 0; h < kJoinHalves; ++h) {
          if (in[h]) {
            join[it[h] & 0x3ffffu] = 1;
            __hip_atomic_fetch_add(&sh.E[b[h]], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
          }
          cut_above += (uint32_t)__builtin_popcountll(__ballot(in[h] && b[h] > bin));
          reaches = reaches || (in[h] && b[h] >= bin);
        }
        if (__ballot(reaches)) tau_ok = false;
      };
      if (i0 < i1) join_keys(i0, pf_it, pf_v);
      for (uint32_t c0 = i0 + kJoinHalves * kWave; c0 < i1; c0 += kJoinHalves * kWave) {
        uint32_t it[kJoinHalves], v[kJoinHalves];
#pragma unroll
        for (int h = 0; h < kJoinHalves; ++h) it[h] = item[min(c0 + (uint32_t)(h * kWave + lane), item_last)];
#pragma unroll
        for (int h = 0; h < kJoinHalves; ++h) v[h] = val[it[h] & 0x3ffffu];
        join_keys(c0, it, v);
      }
      prefetch_items(i1);
      i0 = i1;
      wave_sync();
      RESOLVE_ADD(4, t_join);
      if (cut_above >= (uint32_t)k) {
        // The cut moves up to the highest bin b with at least k joined keys at
        // or above it.  Each step covers 256 bins, four per lane read at once
        // (bins at or below the old cut count as empty); c counts the keys of
        // the bins at or above the step's first, so the bin is found below
        // kBins and the bound only guards the loop.
        RESOLVE_T0(t_move);
        RESOLVE_COUNT(3, 1ull << 32);
        const uint32_t s_first = bin + 1;
        uint32_t s = s_first & ~3u;
        uint32_t c = cut_above;
        for (int guard = 0; guard < kBins / (4 * kWave); ++guard) {
          const uint32_t base = s + 4u * (uint32_t)lane;
          uint4 e4 = base < (uint32_t)kBins ? *reinterpret_cast<const uint4*>(&sh.E[base]) : make_uint4(0u, 0u, 0u, 0u);
          if (base < s_first) e4.x = 0u;
          if (base + 1u < s_first) e4.y = 0u;
          if (base + 2u < s_first) e4.z = 0u;
          const uint32_t sum4 = e4.x + e4.y + e4.z + e4.w;
          const uint32_t incl = wave_incl_scan(sum4);
          const uint64_t m = __ballot(c - incl < (uint32_t)k);
          if (m) {
            // In the lane that crosses: the first of its bins after which
            // fewer than k keys remain above.
            uint32_t rem = c - (incl - sum4) - e4.x;
            uint32_t off = 0u;
            if (rem >= (uint32_t)k) {
              rem -= e4.y;
              off = 1u;
              if (rem >= (uint32_t)k) {
                rem -= e4.z;
                off = 2u;
                if (rem >= (uint32_t)k) {
                  rem -= e4.w;
                  off = 3u;
                }
              }
            }
            const uint32_t l = (uint32_t)__builtin_ctzll(m);
            bin = s + 4u * l + (uint32_t)__builtin_amdgcn_readlane((int)off, (int)l);
            cut_above = (uint32_t)__builtin_amdgcn_readlane((int)rem, (int)l);
            break;
          }
          c -= (uint32_t)__builtin_amdgcn_readlane((int)incl, kWave - 1);
          s += 4u * kWave;
        }
        tau_ok = false;
        RESOLVE_ADD(5, t_move);
      }
    }
    RESOLVE_ADD(0, t_all);
#ifdef DSA_PHASE_TRACE
    if (lane == 0 && row < kTraceWgs)
      for (int i = 0; i < kTraceMarks; ++i) g_trace_resolve[(size_t)row * kTraceMarks + i] += trace_acc[i];
#endif
    if (lane == 0) {
      sh.nreset = nreset;
      sh.cut_bin = bin;
      sh.n_out = 0;
    }
    if (!rp.last_round || a.replay_topk) {
      const uint32_t t = exact_tau();
      if (lane == 0) sh.tau = t;
    }
  }
  __syncthreads();
#ifdef DSA_PHASE_TRACE
  const uint64_t t_tail0 = wall_clock64();
#endif
  // After the loop the LDS key arrays are free: sh.item and sh.val serve as
  // staging (in the spill case they were never used).
  const int bs = a.block_size;
  const int L = a.length;
  const uint32_t t = sh.tau;
  const size_t run_at = run_offset(a, rp.round, row);
  const uint32_t* run_in = a.ws.run + run_at;
  const uint32_t* idx_in = a.ws.run_idx + run_at;
  // A listed key joined iff its block was kept (every listed key's block was
  // decided by this round).
  auto listed_joined = [&](uint64_t x) { return sh.kept[((uint32_t)(x >> 32) & 0x1ffffu) / (uint32_t)bs] != 0; };
  if (!rp.last_round) {
    // The next round starts from the exact k largest, each with its key: the
    // joined keys above the threshold (the run's and the listed ones), then
    // copies of it, in the other of the two run buffers.
    const size_t out_at = run_offset(a, rp.round + 1, row);
    uint32_t* run_out = a.ws.run + out_at;
    uint32_t* idx_out = a.ws.run_idx + out_at;
    auto emit = [&](uint32_t v, uint32_t key) {
      const uint32_t j = __hip_atomic_fetch_add(&sh.n_out, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      run_out[j] = v;
      idx_out[j] = key;
    };
    for (int i = tid; i < k; i += kResolveThreads)
      if (run_in[i] > t) emit(run_in[i], idx_in[i]);
    for (uint32_t e = (uint32_t)tid; e < n_listed; e += kResolveThreads) {
      const uint64_t x = list[e];
      if ((uint32_t)x > t && listed_joined(x)) emit((uint32_t)x, (uint32_t)(x >> 32) & 0x1ffffu);
    }
    __syncthreads();
    for (uint32_t c = sh.n_out + (uint32_t)tid; c < (uint32_t)k; c += kResolveThreads) {
      run_out[c] = t;
      idx_out[c] = 0xffffffffu;
    }
    if (tid == 0) {
      a.ws.tau[row] = t;
      a.ws.floor[row] = t;
    }
  } else if (a.replay_topk) {
    // The step's top-k, when the last threshold lies above this round's floor
    // and is a number above -inf: every evaluated key at or above it is then
    // a joined key with a known index (evaluated keys left out of the joined
    // set are at or below the floor, and so are the run's copies), and when
    // exactly k of them are, they are the k largest of the scores row, -inf
    // elsewhere, with no tie to break.  Otherwise (ties across the cut,
    // repeated seeds) the top-k launched after the rounds does it.  The chosen
    // keys are marked in a bitmap over the row (sh.item) and written in index
    // order.
    const uint32_t words = (uint32_t)(L + 31) / 32u;  // at most 4096 (L <= 2^17)
    bool finished = false;  // uniform over the workgroup
    if (t > floor_key && t > 0x007fffffu && t <= 0xff800000u) {
      for (uint32_t w = (uint32_t)tid; w < words; w += kResolveThreads) sh.item[w] = 0u;
      __syncthreads();
      uint32_t chosen = 0u;
      auto mark = [&](uint32_t key) {
        ++chosen;
        if (key < (uint32_t)L) __hip_atomic_fetch_or(&sh.item[key >> 5], 1u << (key & 31u), __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_WORKGROUP);
        else chosen += 1u << 20;  // no index: not this path
      };
      for (int i = tid; i < k; i += kResolveThreads)
        if (run_in[i] >= t) mark(idx_in[i]);
      for (uint32_t e = (uint32_t)tid; e < n_listed; e += kResolveThreads) {
        const uint64_t x = list[e];
        if ((uint32_t)x >= t && listed_joined(x)) mark((uint32_t)(x >> 32) & 0x1ffffu);
      }
      uint32_t total;
      block_excl_scan<kResolveWaves>(chosen, sh.wsum, total);  // its barrier also ends the marking
      if (total == (uint32_t)k) {
        constexpr int kWordsPer = (1 << 17) / 32 / kResolveThreads;
        const uint32_t w0 = (uint32_t)tid * kWordsPer;
        uint32_t bits[kWordsPer];
        uint32_t n_bits = 0u;
#pragma unroll
        for (int j = 0; j < kWordsPer; ++j) {
          bits[j] = w0 + j < words ? sh.item[w0 + j] : 0u;
          n_bits += (uint32_t)__builtin_popcount(bits[j]);
        }
        __syncthreads();  // the previous scan's sums are read
        uint32_t marked;
        uint32_t at = block_excl_scan<kResolveWaves>(n_bits, sh.wsum, marked);
        if (marked == (uint32_t)k) {  // (repeated seeds would mark fewer)
          int64_t* out = a.replay_topk + (size_t)row * k;
#pragma unroll
          for (int j = 0; j < kWordsPer; ++j)
            for (uint32_t b = bits[j]; b; b &= b - 1u)
              out[at++] = (int64_t)((w0 + j) * 32u + (uint32_t)__builtin_ctz(b));
          finished = true;
        }
      }
    }
    if (finished || a.replay_qk) {
      // Keys scored: the seeds and every key of a kept block, each once.
      const int nb = a.blocks;
      const uint32_t* mask = a.ws.seed_mask + (size_t)row * words;
      uint32_t scored = 0u;
      for (uint32_t w = (uint32_t)tid; w < words; w += kResolveThreads) {
        uint32_t m = mask[w];
        for (uint32_t sub = 0; sub < 32u; sub += 16u) {  // blocks are multiples of 16 keys
          const int blk = (int)((w * 32u + sub) / (uint32_t)bs);
          if (blk < nb && a.evaluated[(size_t)row * nb + blk]) m |= 0xffffu << sub;
        }
        const uint32_t valid = min(32u, (uint32_t)L - w * 32u);
        if (valid < 32u) m &= (1u << valid) - 1u;
        scored += (uint32_t)__builtin_popcount(m);
      }
      __syncthreads();  // the previous scan's sums are read
      uint32_t qk;
      block_excl_scan<kResolveWaves>(scored, sh.wsum, qk);
      if (tid == 0) {
        a.qk_scored[row] = (int32_t)qk;
        if (finished) a.ws.done[row] = 1u;
      }
    }
  }
#ifdef DSA_PHASE_TRACE
  const uint64_t t_tail1 = wall_clock64();
#endif
  // Scored blocks the replay pruned: their keys back to -inf, seeds excepted.
  int bs_shift = 4;
  while ((1 << bs_shift) < bs) ++bs_shift;
  const uint32_t nreset = sh.nreset;
  const uint32_t* mask = a.ws.seed_mask + (size_t)row * ((L + 31) / 32);
  float* srow = a.scores + (size_t)row * L;
  // (Block sizes divide kRoundKeys: powers of two.)  Eight keys per thread
  // per pass, their seed-mask words read before any is written.
  const uint32_t n_reset_keys = nreset * (uint32_t)bs;
  for (uint32_t i0 = (uint32_t)tid; i0 < n_reset_keys; i0 += 8u * kResolveThreads) {
    int key[8];
    uint32_t word[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t i = min(i0 + (uint32_t)j * kResolveThreads, n_reset_keys - 1u);
      key[j] = (int)sh.resets[i >> bs_shift] * bs + (int)(i & (uint32_t)(bs - 1));
      word[j] = mask[min(key[j], L - 1) >> 5];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (i0 + (uint32_t)j * kResolveThreads < n_reset_keys && key[j] < L && !((word[j] >> (key[j] & 31)) & 1u))
        srow[key[j]] = -__builtin_inff();
  }
#ifdef DSA_PHASE_TRACE
  // Rows 1024 + row of the log (trace builds only): the tail after the group
  // loop, its write-back or top-k part, and the -inf resets.
  if (tid == 0 && row < 1024) {
    const uint64_t t_end = wall_clock64();
    g_trace_resolve[(size_t)(1024 + row) * kTraceMarks + 0] += t_end - t_tail0;
    g_trace_resolve[(size_t)(1024 + row) * kTraceMarks + 1] += t_tail1 - t_tail0;
    g_trace_resolve[(size_t)(1024 + row) * kTraceMarks + 2] += t_end - t_tail1;
  }
#endif
}

__global__ __launch_bounds__(kResolveThreads) void temporal_resolve_kernel(TemporalArgs a, RoundPlan rp) {
  __shared__ ResolveShared sh;
#ifdef DSA_PHASE_TRACE
  const uint64_t t_start = wall_clock64();
#else
  const uint64_t t_start = 0;
#endif
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int row = blockIdx.x;
  const int nb = a.blocks;
  const int k = a.k;
  const int n_pos = rp.pos_end - rp.pos_begin;
  const int wave = tid >> 6;
  const uint32_t* order = a.ws.order + (size_t)row * nb + rp.pos_begin;
  const double* upper = a.ws.upper_pos + (size_t)row * nb + rp.pos_begin;
  const uint32_t* run = a.ws.run + run_offset(a, rp.round, row);
  const uint64_t* list = a.ws.entries + (size_t)row * a.ws.list_capacity;
  // The setup's inputs are read in one round trip: the positions' blocks and
  // bounds (at most four per thread), the list's length, the floor, the
  // seeds' threshold, and the first kKeyBatch key values per thread, each
  // from the running k largest or the list (one dword: an entry's value is
  // its low word), list reads clamped to its capacity until its length is
  // known.
  const uint32_t n_listed = a.ws.list_total[(size_t)row * kMaxRounds + rp.round];
  const uint32_t floor_key = a.ws.floor[row];
  const uint32_t seed_tau = a.ws.tau[row];
  constexpr int kPosPer = kMaxTemporalBlocks / kResolveThreads;
  uint32_t pb[kPosPer];
  double pu[kPosPer];
#pragma unroll
  for (int j = 0; j < kPosPer; ++j) {
    const int i = max(min(tid + j * kResolveThreads, n_pos - 1), 0);
    pb[j] = order[i];
    pu[j] = upper[i];
  }
  const uint32_t cap_last = (uint32_t)a.ws.list_capacity - 1u;
  auto key_value = [&](uint32_t i, uint32_t last) {
    const uint32_t e = min(i - (uint32_t)k, last);  // (wraps below k: clamped, unused)
    const uint32_t* p = i < (uint32_t)k ? run + i : reinterpret_cast<const uint32_t*>(list + e);
    return *p;
  };
  uint32_t kv[kKeyBatch];
#pragma unroll
  for (int j = 0; j < kKeyBatch; ++j) kv[j] = key_value((uint32_t)(tid + j * kResolveThreads), cap_last);
#pragma unroll
  for (int j = 0; j < kPosPer; ++j) {
    const int i = tid + j * kResolveThreads;
    if (i < n_pos) {
      sh.blk[i] = (uint16_t)pb[j];
      sh.uk[i] = upper_key(pu[j]);
    }
  }
  // The largest key (the span of the bins): per wave, then over the waves.
  const uint32_t n_keys = (uint32_t)k + n_listed;
  uint32_t mx = 0;
#pragma unroll
  for (int j = 0; j < kKeyBatch; ++j)
    if ((uint32_t)(tid + j * kResolveThreads) < n_keys) mx = max(mx, kv[j]);
  const uint32_t list_last = n_listed ? n_listed - 1u : 0u;
  for (uint32_t i0 = (uint32_t)tid + kKeyBatch * kResolveThreads; i0 < n_keys; i0 += kKeyBatch * kResolveThreads) {
#pragma unroll
    for (int j = 0; j < kKeyBatch; ++j) kv[j] = key_value(i0 + (uint32_t)(j * kResolveThreads), list_last);
#pragma unroll
    for (int j = 0; j < kKeyBatch; ++j)
      if (i0 + (uint32_t)(j * kResolveThreads) < n_keys) mx = max(mx, kv[j]);
  }
  for (int off = 32; off > 0; off >>= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, off, kWave));
  if (lane == 0) sh.wsum[wave] = mx;
  __syncthreads();
  uint32_t max_key = 0;
#pragma unroll
  for (int w = 0; w < kResolveWaves; ++w) max_key = max(max_key, sh.wsum[w]);
  if (n_keys <= (uint32_t)kSortCap)
    resolve_row<false>(a, rp, sh, n_listed, max_key, floor_key, seed_tau, t_start);
  else
    resolve_row<true>(a, rp, sh, n_listed, max_key, floor_key, seed_tau, t_start);
}

// Round splits, as fractions of the scan's groups: DSA_AMD_TEMPORAL_ROUNDS, a
// comma-separated increasing list in (0, 1), or "1" for a single round (read
// at every step).  By default one split at a quarter of the scan, and two
// (a tenth, three tenths) for rows of 64K keys or more.  Each later round
// starts from a higher floor, so fewer of its blocks are scored and then
// pruned: fewer splits are faster but load more key bytes (C5 with a single
// split at a tenth: from as fast to 18 us faster per step, but 0.21 instead
// of 0.38 of the dense key bytes not loaded at gamma_sigma -0.25, and 0.017
// instead of 0.061 at 1.0; C3 with a split at a tenth: 2-3 us faster, 0
// instead of 0.0019 not loaded for the block-16 address scan at gamma_sigma
// 1.0).
std::vector<double> round_splits(int length) {
  std::vector<double> splits;
  const char* v = std::getenv("DSA_AMD_TEMPORAL_ROUNDS");
  const char* s = v ? v : (length >= 65536 ? "0.1,0.3" : "0.25");
  double last = 0.0;
  while (*s) {
    char* end = nullptr;
    const double f = std::strtod(s, &end);
    if (end == s) break;
    if (f > last && f < 1.0) {
      splits.push_back(f);
      last = f;
    }
    if (*end != ',') break;
    s = end + 1;
  }
  return splits;
}

template <class Tag, class KF>
int launch_rounds(TemporalArgs& a, int32_t wave, hipStream_t stream) {
  // Item and list packing: slots below 2^18, blocks below 2^14, keys below
  // 2^17, groups below 2^15.
  DSA_REQUIRE(wave > 0 && a.blocks <= kMaxTemporalBlocks && a.length <= (1 << 17) &&
                  a.ws.spill_capacity < (1 << 18) && kRoundKeys % a.block_size == 0,
              "step shape outside the dynamic rounds (blocks %d, length %d)", a.blocks, a.length);
  const int W = wave;
  const int nb = a.blocks;
  const int groups = (nb + W - 1) / W;
  std::vector<int> cuts = {0};
  for (double f : round_splits(a.length)) {
    const int c = (int)(f * groups + 0.5);
    if (c > cuts.back() && c < groups && (int)cuts.size() < kMaxRounds) cuts.push_back(c);
  }
  cuts.push_back(groups);
  const int span = kRoundKeys / a.block_size;  // scan positions of kRoundKeys keys
  for (size_t r = 0; r + 1 < cuts.size(); ++r) {
    RoundPlan rp;
    rp.pos_begin = cuts[r] * W;
    rp.pos_end = min(cuts[r + 1] * W, nb);
    // Wide rounds give each workgroup kRoundParts spans (fewer, longer
    // workgroups, each wave's units streamed); narrow ones one span, so that
    // the round still spreads over the whole GPU.
    const int64_t spans = (int64_t)a.rows * ((rp.pos_end - rp.pos_begin + span - 1) / span);
    const bool wide = spans >= kRoundWideSpans;
    const int per_wg = (wide ? kRoundParts : 1) * span;  // at most 64 positions: one per thread
    rp.per_wg = per_wg;
    rp.wgs_per_row = (rp.pos_end - rp.pos_begin + per_wg - 1) / per_wg;
    rp.group = W;
    rp.first_round = r == 0;
    rp.last_round = r + 2 == cuts.size();
    rp.round = (int32_t)r;
    if (wide)
      hipLaunchKernelGGL((temporal_round_kernel<Tag, KF, kRoundParts>), dim3((unsigned)(a.rows * rp.wgs_per_row)),
                         dim3(kRoundThreads), 0, stream, a, rp);
    else
      hipLaunchKernelGGL((temporal_round_kernel<Tag, KF, 1>), dim3((unsigned)(a.rows * rp.wgs_per_row)),
                         dim3(kRoundThreads), 0, stream, a, rp);
    if (int st = check_launch("temporal_round_kernel")) return st;
    hipLaunchKernelGGL(temporal_resolve_kernel, dim3((unsigned)a.rows), dim3(kResolveThreads), 0, stream, a, rp);
    if (int st = check_launch("temporal_resolve_kernel")) return st;
  }
  return DSA_STATUS_OK;
}

}  // namespace

int temporal_rounds(TemporalArgs& a, int32_t wave, int32_t key_dtype, hipStream_t stream) {
  switch (key_dtype) {
    case DSA_DTYPE_BF16: return launch_rounds<Bf16Tag, KeysB16>(a, wave, stream);
    case DSA_DTYPE_F16: return launch_rounds<F16Tag, KeysB16>(a, wave, stream);
    default: return launch_rounds<Bf16Tag, KeysFP8>(a, wave, stream);
  }
}

}  // namespace dsa

#ifdef DSA_PHASE_TRACE
// The replay's per-row phase totals (trace builds only).
extern "C" int dsa_trace_temporal_resolve(uint64_t* host, int64_t n, int32_t clear) {
  using namespace dsa;
  DSA_REQUIRE(host && n >= 0 && n <= int64_t(kTraceWgs) * kTraceMarks, "bad trace read");
  if (int st = check_hip(hipMemcpyFromSymbol(host, HIP_SYMBOL(g_trace_resolve), (size_t)n * 8), "trace read"))
    return st;
  if (clear) {
    static const uint64_t zeros[kTraceWgs * kTraceMarks] = {};
    return check_hip(hipMemcpyToSymbol(HIP_SYMBOL(g_trace_resolve), zeros, sizeof(zeros)), "trace clear");
  }
  return DSA_STATUS_OK;
}
#endif
