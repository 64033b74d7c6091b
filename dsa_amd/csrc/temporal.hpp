// Internal interface of the temporal step shared by temporal.hip and
// verifier.hip: argument and workspace layouts, the scan-order sort, the
// unit scorer, and the two halves of a step (the seeded block scan; then the
// histogram, the top-k select and the policy-state update).
#pragma once

#include "common.hpp"
#include "dsa_amd.h"
#include "indexer.hpp"
#include "select.hpp"
#include "waveops.hpp"

#include <cmath>

namespace dsa {

constexpr int kMaxTemporalBlocks = 2048;  // blocks per row (sorted in one workgroup)
constexpr int kMaxMerge = 8192;            // k + one wave's keys, merged in LDS
constexpr uint32_t kFarKey = 0x00ffffffu;  // a key index whose rows lie past every buffer
constexpr int kDigitBinsT = 2048;          // 11-bit radix digits of the threshold refresh

// Workgroups of the fused static step (temporal_fused.hip): one exchange slot
// and one scored-key count each, at fixed offsets at the start of the
// workspace so that they do not move with the step's shape.
constexpr int kMaxFusedWgs = 4096;

struct TemporalWorkspace {
  uint64_t* slots;      // [kMaxFusedWgs] (generation << 32) | least seed key of each fused workgroup; zero
                        // before the workspace's first use
  uint32_t* qk_parts;   // [kMaxFusedWgs] keys each fused workgroup scored; bit 31: its wait gave up
  uint32_t* tau;        // [rows] ordered key of the threshold in force
  uint32_t* floor;      // [rows] least of run (the k-th largest evaluated score), dynamic rounds
  uint32_t* loaded;     // [rows] key rows a dynamic step loaded (seeds + every key of its rounds' scored blocks)
  uint32_t* run;        // [2][rows][k] ordered keys of the k largest evaluated scores (the dynamic rounds
                        // alternate between the two buffers; every other path uses the first)
  uint32_t* run_idx;    // [2][rows][k] dynamic rounds: the key of each run entry (0xffffffff: a copy of the threshold)
  uint32_t* done;       // [rows] dynamic rounds: the last replay wrote the row's top-k and keys scored
  uint32_t* order;      // [rows][blocks] block ids in scan order
  double* upper;        // [rows][blocks] U_b, in double like the float64 reference
  double* upper_pos;    // [rows][blocks] the same, by scan position
  uint64_t* sort_hi;    // [rows][blocks] scan-order sort key of each block (~ordered float64 rank value)
  uint32_t* sort_lo;    // [rows][blocks] group << 31 | block
  uint32_t* seed_mask;  // [rows][ceil(L / 32)] keys evaluated as seeds
  // Dynamic rounds: the keys each round's scoring lists (a row's list is
  // entries [0, list_total[round])), and the replay's sorted keys when they
  // outgrow its LDS.
  uint32_t* list_total;  // [rows][kMaxRounds]
  uint64_t* entries;     // [rows][list_capacity] (group << 49) | (key << 32) | ordered score
  uint32_t* spill_val;   // [rows][spill_capacity]
  uint32_t* spill_item;  // [rows][spill_capacity]
  uint8_t* spill_join;   // [rows][spill_capacity]
  int64_t list_capacity;
  int64_t spill_capacity;
  SelectWorkspace select;  // final top-k over the evaluated keys
  int64_t bytes;
};

// Keys one scoring wave of a dynamic round covers at most (two 64-key units),
// keys per scoring workgroup (four waves), and rounds per scan.
constexpr int kRoundWaveKeys = 128;
constexpr int kRoundKeys = 4 * kRoundWaveKeys;
constexpr int kMaxRounds = 8;

inline TemporalWorkspace temporal_layout(void* base, int64_t rows, int64_t length, int64_t k, int32_t block_size) {
  const int64_t blocks = (length + block_size - 1) / block_size;
  auto round = [](int64_t bytes) { return (bytes + 255) / 256 * 256; };
  // A round's scoring workgroups cover at most blocks * block_size + kRoundKeys
  // keys of region space; the replay sorts k of them more.
  const int64_t list_capacity = blocks * block_size + kRoundKeys;
  const int64_t spill_capacity = list_capacity + k;
  const int64_t slots_off = 0;
  const int64_t parts_off = slots_off + kMaxFusedWgs * 8;
  const int64_t tau_off = parts_off + kMaxFusedWgs * 4;
  const int64_t floor_off = tau_off + round(rows * 4);
  const int64_t loaded_off = floor_off + round(rows * 4);
  const int64_t run_off = loaded_off + round(rows * 4);
  const int64_t run_idx_off = run_off + round(2 * rows * k * 4);
  const int64_t done_off = run_idx_off + round(2 * rows * k * 4);
  const int64_t order_off = done_off + round(rows * 4);
  const int64_t upper_off = order_off + round(rows * blocks * 4);
  const int64_t upos_off = upper_off + round(rows * blocks * 8);
  const int64_t shi_off = upos_off + round(rows * blocks * 8);
  const int64_t slo_off = shi_off + round(rows * blocks * 8);
  const int64_t mask_off = slo_off + round(rows * blocks * 4);
  const int64_t count_off = mask_off + round(rows * ((length + 31) / 32) * 4);
  const int64_t entries_off = count_off + round(rows * kMaxRounds * 4);
  const int64_t sval_off = entries_off + round(rows * list_capacity * 8);
  const int64_t sitem_off = sval_off + round(rows * spill_capacity * 4);
  const int64_t sjoin_off = sitem_off + round(rows * spill_capacity * 4);
  const int64_t select_off = sjoin_off + round(rows * spill_capacity);
  TemporalWorkspace ws;
  const uintptr_t p = reinterpret_cast<uintptr_t>(base);
  ws.select = select_workspace_layout(base ? reinterpret_cast<void*>(p + select_off) : nullptr, rows, length);
  ws.bytes = select_off + round(ws.select.bytes);
  ws.list_capacity = list_capacity;
  ws.spill_capacity = spill_capacity;
  ws.slots = base ? reinterpret_cast<uint64_t*>(p + slots_off) : nullptr;
  ws.qk_parts = base ? reinterpret_cast<uint32_t*>(p + parts_off) : nullptr;
  ws.tau = base ? reinterpret_cast<uint32_t*>(p + tau_off) : nullptr;
  ws.floor = base ? reinterpret_cast<uint32_t*>(p + floor_off) : nullptr;
  ws.loaded = base ? reinterpret_cast<uint32_t*>(p + loaded_off) : nullptr;
  ws.run = base ? reinterpret_cast<uint32_t*>(p + run_off) : nullptr;
  ws.run_idx = base ? reinterpret_cast<uint32_t*>(p + run_idx_off) : nullptr;
  ws.done = base ? reinterpret_cast<uint32_t*>(p + done_off) : nullptr;
  ws.order = base ? reinterpret_cast<uint32_t*>(p + order_off) : nullptr;
  ws.upper = base ? reinterpret_cast<double*>(p + upper_off) : nullptr;
  ws.upper_pos = base ? reinterpret_cast<double*>(p + upos_off) : nullptr;
  ws.sort_hi = base ? reinterpret_cast<uint64_t*>(p + shi_off) : nullptr;
  ws.sort_lo = base ? reinterpret_cast<uint32_t*>(p + slo_off) : nullptr;
  ws.seed_mask = base ? reinterpret_cast<uint32_t*>(p + mask_off) : nullptr;
  ws.list_total = base ? reinterpret_cast<uint32_t*>(p + count_off) : nullptr;
  ws.entries = base ? reinterpret_cast<uint64_t*>(p + entries_off) : nullptr;
  ws.spill_val = base ? reinterpret_cast<uint32_t*>(p + sval_off) : nullptr;
  ws.spill_item = base ? reinterpret_cast<uint32_t*>(p + sitem_off) : nullptr;
  ws.spill_join = base ? reinterpret_cast<uint8_t*>(p + sjoin_off) : nullptr;
  return ws;
}

// Own-trajectory policy state (approx.py:42-50), [rows][stride] per field.
struct ApproxDev {
  float* last_max;
  float* ema;
  float* vol;
  int16_t* age;
  int16_t* cold;
  int64_t stride;
  const double* gamma_rows;  // per-row gamma, or null for p.gamma
  dsa_approx_policy p;
};

struct TemporalArgs {
  const uint16_t* q;      // [rows][64][128]
  const float* w;         // [rows][64]
  const uint8_t* keys;    // [rows][key_stride] key rows (the first length are scored)
  int64_t key_stride;     // key rows between sequences
  const float* scales;    // fp8: [rows][ceil(key_stride / 128)]
  const float* prev_max;  // [rows][prev_blocks]
  const int64_t* seeds;   // [rows][k]
  const float* gamma;     // [rows]
  const double* gamma_d;  // [rows] or null: a float64 margin (replay over recorded scores)
  const double* margins;  // [rows][prev_blocks] or null: per-block margins (certified bound) in place of gamma
  const float* source;    // [rows][source_stride] or null: recorded scores read instead of scoring keys
  int64_t source_stride;
  int32_t* order_out;     // [rows][blocks] or null: the scan order, for the caller
  const float* order_key; // [rows][blocks]: the sort key of scan order 3 (larger first, then address)
  float* scores;          // [rows][length]
  uint8_t* evaluated;     // [rows][blocks]
  int32_t* qk_scored;     // [rows]
  int64_t* replay_topk;   // [rows][k] or null: the dynamic rounds' last replay writes the top-k and keys scored
                          // where it can (then ws.done[row] is set and the finishing select skips the row)
  int32_t replay_qk;      // with replay_topk: the last replay writes the keys scored of every row
  int32_t* waits_given_up;  // [rows] or null: fused static workgroups whose wait for the row's seed minima ran out
  int32_t rows, length, k, block_size, blocks, prev_length, prev_blocks;
  int32_t scan_order;     // 0 address, 1 previous-hot, 2 upper, 3 order_key
  int32_t wave_start, wave_len;
  int32_t policy_mode;    // 0: bound prev_max + gamma (replay filter); 1: own-trajectory policy
  ApproxDev ap;
  const int64_t* teacher_topk;  // [rows][k]: dense top-k of the step (teacher history only)
  TemporalWorkspace ws;
};

// Order-preserving double -> uint64 map (NaN as -inf, -0.0 as +0.0, so the
// sort sees the values a float64 sort key would).
__device__ __forceinline__ uint64_t double_to_ordered(double d) {
  if (__builtin_isnan(d)) d = -HUGE_VAL;
  if (d == 0.0) d = 0.0;
  const uint64_t u = (uint64_t)__double_as_longlong(d);
  return (u >> 63) ? ~u : (u | (1ull << 63));
}

// Risk of a block under the policy (approx.py:178-189).  The float32 product
// volatility_lambda * volatility and the left-to-right float64 sums follow
// numpy's evaluation of the reference expression.
__device__ __forceinline__ double policy_risk(const dsa_approx_policy& p, double gamma, float last_max, float ema,
                                              float vol, int age) {
#pragma clang fp contract(off)
  const double aged = p.age_slope * (double)age;
  if (p.risk_model == DSA_RISK_EMA) {
    const float spread = (float)p.volatility_lambda * vol;
    return (((double)ema + (double)spread) + gamma) + aged;
  }
  return ((double)last_max + gamma) + aged;
}

// Sort entries: ascending (lo >> 31, hi, lo & 0x7fffffff).  Branch-free: the
// sort is VALU-bound on one CU, so each compare is a handful of v_cmp with
// the masks combined on the scalar unit.
__device__ __forceinline__ bool sorts_before(uint64_t hi_a, uint32_t lo_a, uint64_t hi_b, uint32_t lo_b) {
  const uint32_t ga = lo_a >> 31;
  const uint32_t gb = lo_b >> 31;
  const uint32_t aa = lo_a & 0x7fffffffu;
  const uint32_t ab = lo_b & 0x7fffffffu;
  return (ga < gb) | ((ga == gb) & ((hi_a < hi_b) | ((hi_a == hi_b) & (aa < ab))));
}

constexpr int kSortN = kMaxTemporalBlocks;  // most entries one 1024-thread workgroup sorts

// Bitonic sort of n entries (a power of two, 2 <= n <= kSortN) held two per
// thread (entries 2t and 2t+1 of thread t; threads with 2t >= n only join
// the barriers).  Compare-exchange partners at distance 1 are in the same
// thread, at distance 2..64 in the same wave (lane shuffles, no barrier), and
// further apart they meet through LDS (xh, xl: kSortN entries).  Partners of
// an active entry are active: e ^ stride < n for every e < n.
__device__ inline void block_sort(uint64_t (&h)[2], uint32_t (&l)[2], uint64_t* xh, uint32_t* xl, int n) {
  const int t = threadIdx.x;
  const bool active = 2 * t < n;
  for (int size = 2; size <= n; size <<= 1) {
    const bool up = ((2 * t) & size) == 0;
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      if (stride == 1) {
        const bool second_first = sorts_before(h[1], l[1], h[0], l[0]);
        const bool same = (h[0] == h[1]) & (l[0] == l[1]);
        const bool swap = up ? second_first : !(second_first | same);
        const uint64_t h0 = swap ? h[1] : h[0];
        const uint64_t h1 = swap ? h[0] : h[1];
        const uint32_t l0 = swap ? l[1] : l[0];
        const uint32_t l1 = swap ? l[0] : l[1];
        h[0] = h0;
        h[1] = h1;
        l[0] = l0;
        l[1] = l1;
        continue;
      }
      const int mask = stride >> 1;  // partner thread t ^ mask
      const bool lower = (t & mask) == 0;
      uint64_t oh[2];
      uint32_t ol[2];
      if (stride <= 64) {
        if (!active) continue;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          oh[j] = __shfl_xor(h[j], mask, kWave);
          ol[j] = __shfl_xor(l[j], mask, kWave);
        }
      } else {
        if (active) {
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            xh[2 * t + j] = h[j];
            xl[2 * t + j] = l[j];
          }
        }
        __syncthreads();
        if (active) {
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            oh[j] = xh[(2 * t + j) ^ stride];
            ol[j] = xl[(2 * t + j) ^ stride];
          }
        }
        __syncthreads();
        if (!active) continue;
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        // other-first decides for the lower entry of an ascending pair and the
        // upper entry of a descending one; the rest take the other entry iff
        // it is strictly later (equal entries are padding).
        const bool other_first = sorts_before(oh[j], ol[j], h[j], l[j]);
        const bool same = (oh[j] == h[j]) & (ol[j] == l[j]);
        const bool take = (up == lower) ? other_first : !(other_first | same);
        h[j] = take ? oh[j] : h[j];
        l[j] = take ? ol[j] : l[j];
      }
    }
  }
}

// The same network over single 64-bit keys, ascending (padding: ~0).  One
// 64-bit compare and two selects per compare-exchange, against the three
// compares of the (hi, lo) entries above: the scan-order sort packs its keys
// into 64 bits where it can.
__device__ inline void block_sort64(uint64_t (&v)[2], uint64_t* x, int n) {
  const int t = threadIdx.x;
  const bool active = 2 * t < n;
  for (int size = 2; size <= n; size <<= 1) {
    const bool up = ((2 * t) & size) == 0;
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      if (stride == 1) {
        const bool swap = up ? v[1] < v[0] : v[0] < v[1];
        const uint64_t a0 = swap ? v[1] : v[0];
        const uint64_t a1 = swap ? v[0] : v[1];
        v[0] = a0;
        v[1] = a1;
        continue;
      }
      const int mask = stride >> 1;  // partner thread t ^ mask
      const bool lower = (t & mask) == 0;
      uint64_t o[2];
      if (stride <= 64) {
        if (!active) continue;
#pragma unroll
        for (int j = 0; j < 2; ++j) o[j] = __shfl_xor(v[j], mask, kWave);
      } else {
        if (active) {
          x[2 * t] = v[0];
          x[2 * t + 1] = v[1];
        }
        __syncthreads();
        if (active) {
#pragma unroll
          for (int j = 0; j < 2; ++j) o[j] = x[(2 * t + j) ^ stride];
        }
        __syncthreads();
        if (!active) continue;
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) v[j] = (up == lower) ? min(v[j], o[j]) : max(v[j], o[j]);
    }
  }
}

// Scores 64 keys of one row with the dense kernel's unit code: lane (r, g)
// loads, for each tile t, its slice of key tile_key[t] (kFarKey: nothing is
// loaded and the result is not a key's score).  Lane l returns the score of
// the key that lane (l & 15, .) of tile l >> 4 loaded.
template <class Tag, class KF>
__device__ __forceinline__ float score_unit(const TemporalArgs& a, int row, const int (&tile_key)[4],
                                            int r, int g) {
  uint4 qa[4][4];
  float wr[4][4];
  load_dense_head_tiles<4, KF::kNaturalK>(a.q + (size_t)row * kHeads * kHeadDim, a.w + (size_t)row * kHeads,
                                          r, g, qa, wr);
  const BufferRsrc keys = make_buffer(a.keys + (size_t)row * a.key_stride * KF::kRowBytes,
                                      (uint32_t)a.length * KF::kRowBytes);
  uint4 buf[4][KF::kRaw];
#pragma unroll
  for (int t = 0; t < 4; ++t) KF::load_buf(keys, tile_key[t], g, buf[t]);
  float s[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) s[t] = tile_contrib<Tag, 4, KF>(qa, wr, buf[t]);
  return unit_reduce(s, g);
}

// First half of a step: clean slate, bounds and scan order, the seeds, and the
// block scan (with threshold refreshes when wave > 0).  Leaves the scores of
// the evaluated keys (-inf elsewhere) and the refreshed-block flags.
int temporal_scan(TemporalArgs& a, int32_t wave, int32_t key_dtype, hipStream_t stream);

// Second half: the select histogram and the keys-scored count, the stable
// top-k of the scores row into out_topk, and (policy mode) the state update
// of every block refreshed by the scan or flagged in `rescued` (may be null).
int temporal_finish(TemporalArgs& a, int64_t* out_topk, const uint8_t* rescued, hipStream_t stream);

// The policy-mode state update alone (nothing in replay-filter mode), after
// the top-k is in out_topk.
int policy_state(TemporalArgs& a, const int64_t* out_topk, const uint8_t* rescued, hipStream_t stream);

// The static replay-filter step (wave 0, no policy, live keys) as one
// scoring launch plus the candidate-list select.  Returns
// DSA_STATUS_OK with `ran` false, launching nothing, when the step's shape
// does not fit that path (the caller then runs temporal_scan and
// temporal_finish).
int temporal_static_fused(TemporalArgs& a, int32_t key_dtype, int64_t* out_topk, hipStream_t stream, bool& ran);

// The dynamic scan (wave > 0) in rounds (temporal_rounds.hip), after the prep
// and seed kernels: each round scores every block of its scan positions whose
// bound clears the threshold in force at the round's start, then one
// workgroup per row replays the scan's decisions over those positions
// exactly.
int temporal_rounds(TemporalArgs& a, int32_t wave, int32_t key_dtype, hipStream_t stream);

// Scan paths: DSA_AMD_TEMPORAL_PATH=launch keeps every step on the
// multi-launch paths (static: prep, seeds, blocks, histogram select; dynamic:
// per-wave launches or the persistent per-row scan), for comparisons.
bool legacy_paths_forced();

// Shared argument checks of the step entry points.
int check_step(const void* queries, const void* keys, int64_t key_stride, const float* key_scales,
               int64_t prev_length, int64_t batch, int64_t length, int64_t k, int32_t block_size, int32_t wave,
               int32_t key_dtype, const void* workspace);

}  // namespace dsa
