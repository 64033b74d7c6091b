// The static replay-filter step in one scoring launch.
//
// With a fixed threshold (wave 0: the reference's static filter,
// replay.py:172-222 with the threshold never refreshed) a block's fate does
// not depend on the scan order: block b is kept iff !(U_b < tau), tau being
// the least score of the previous step's top-k (the seeds).  The step is then
// a dense decode step whose workgroups skip the keys of pruned blocks:
//
//  1. each workgroup owns one chunk of a row's keys (the candidate-list plan
//     of the decode step) and scores the seeds that fall inside it, loading
//     only those key rows;
//  2. it publishes the least of them in its own exchange slot, stamped with
//     the call's generation, and waits until every workgroup of the row has
//     published; tau is the least over the row's slots;
//  3. it decides its blocks against tau and streams its units with the key
//     rows of pruned blocks replaced by an out-of-range offset (no memory
//     access), writing kept keys' scores, seeds' scores and -inf elsewhere;
//  4. its candidate list goes to the decode step's list select, which also
//     totals the keys scored.
//
// The only data that crosses workgroups inside the launch is the slots, each
// a 64-bit atomic written once per call; nothing else needs ordering.  The
// grid is launched only when all of it fits on the device at once (at most
// the occupancy limit times the CU count), so every workgroup a row waits for
// becomes resident once the work ahead of it on the stream drains.  The
// residency check counts the device's whole capacity, not the CUs other work
// holds, so the wait is also bounded: a workgroup that gives up keeps every
// block of its chunk (a superset of the filter's decisions) and the kernel
// still ends.  It marks bit 31 of its scored-key count, and the list select
// reports the row's marks in waits_given_up.  (A cooperative launch would
// promise residency outright, but costs ~20 us of host-side setup per call
// here.)
//
// Scores use the dense kernel's tile code (indexer.hpp), so an evaluated key
// gets the dense score bit for bit.

#include "lists.hpp"
#include "status.hpp"
#include "temporal.hpp"

namespace dsa {
namespace {

constexpr int kFusedWaves = kDecodeWaves;
constexpr int kFusedThreads = 64 * kFusedWaves;
constexpr uint32_t kOutOfRange = 0x80000000u;  // a buffer offset past every unit resource
constexpr uint32_t kSpinLimit = 1u << 22;      // polls (each ~1 us) before a workgroup stops waiting
constexpr uint32_t kGaveUp = 0x80000000u;      // scored-key count bit: the workgroup's wait ran out

#ifdef DSA_PHASE_TRACE
// Per workgroup (by blockIdx.x): 0 start, 1 seeds listed, 2 seeds scored,
// 3 threshold exchanged, 4 blocks decided, 5 units scored, 6 list written.
__device__ uint64_t g_trace_static[kTraceWgs * kTraceMarks];
#endif

struct FusedPlan {
  int32_t chunk_keys;
  int32_t chunks;  // per row
  uint32_t quota;
  uint32_t total_wgs;
  uint32_t gen;
  uint32_t spin_limit;  // polls of the exchange before giving up
};

template <class Tag, class KF>
__global__ __launch_bounds__(kFusedThreads, 2) void temporal_static_kernel(TemporalArgs a, FusedPlan p) {
  __shared__ uint32_t hist[kSelectBins];
  __shared__ uint32_t seed_bits[kListChunkMax / 32];   // seeds of the chunk
  __shared__ uint16_t seed_list[kListChunkMax];         // the same, as chunk-local positions
  __shared__ uint32_t s_nseeds;
  __shared__ uint32_t tile_bits[kListChunkMax / 512];  // 16-key tiles of the chunk's kept blocks
  __shared__ uint32_t s_least, s_tau, s_count, s_list_bin, s_gave_up;
  // Scaled keys: the chunk's 128-key block scales, read once here, so that
  // no scale load sits behind a unit's MFMAs (waiting for one there made the
  // compiler drain every unit in flight).
  __shared__ float s_scales[KF::kScaled ? kListChunkMax / 128 + 1 : 1];
  __shared__ __align__(16) uint32_t s_wsum[kFusedWaves];
  extern __shared__ float chunk_scores[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15;
  const int g = lane >> 4;
  const uint32_t logical = logical_block();
  if (logical >= p.total_wgs) return;
  DSA_TRACE_MARK(g_trace_static, blockIdx.x, 0);
  const int row = (int)(logical / (uint32_t)p.chunks);
  const int c = (int)(logical % (uint32_t)p.chunks);
  const int L = a.length;
  const int base = c * p.chunk_keys;
  const int n_chunk = min(p.chunk_keys, L - base);
  const int units = (n_chunk + 63) >> 6;
  const int bs = a.block_size;

  for (int i = tid; i < kSelectBins; i += kFusedThreads) hist[i] = 0;
  for (int i = tid; i < kListChunkMax / 32; i += kFusedThreads) seed_bits[i] = 0;
  if (tid < kListChunkMax / 512) tile_bits[tid] = 0;
  if constexpr (KF::kScaled) {
    const int s_first = base >> 7;
    const int n_scales = n_chunk > 0 ? ((base + n_chunk - 1) >> 7) - s_first + 1 : 0;
    if (tid < n_scales)
      s_scales[tid] = a.scales[(size_t)row * ((a.key_stride + 127) / 128) + s_first + tid];
  }
  if (tid == 0) {
    s_least = 0xffffffffu;
    s_count = 0;
    s_nseeds = 0;
  }
  uint4 qa[4][4];
  float wr[4][4];
  load_dense_head_tiles<4, KF::kNaturalK>(a.q + (size_t)row * kHeads * kHeadDim, a.w + (size_t)row * kHeads, r, g,
                                          qa, wr);
  // The bounds of the chunk's blocks (at most 512: two per thread) and the
  // first seeds are loaded now, with the query tiles, unconditionally (clamped
  // indices), so that their latencies overlap: the bounds are combined only
  // after the exchange, which needs no memory round trip for them.
  const int first_new = a.prev_length / bs;
  const bool grown = a.prev_length < L;
  const int b_first = base / bs;
  const int b_end = (base + n_chunk + bs - 1) / bs;
  const int last_prev = a.prev_blocks - 1;  // prev_blocks >= 1
  float pm_raw[2];
  double margin_raw[2] = {0.0, 0.0};
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const size_t at = (size_t)row * a.prev_blocks + min(b_first + tid + kFusedThreads * j, last_prev);
    pm_raw[j] = a.prev_max[at];
    if (a.margins) margin_raw[j] = a.margins[at];  // uniform
  }
  const int64_t* seeds = a.seeds + (size_t)row * a.k;
  int64_t first_keys[8];  // seeds tid + kFusedThreads * j
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int i = tid + kFusedThreads * j;
    first_keys[j] = seeds[min(i, a.k - 1)];
  }

  const double gamma = a.margins ? 0.0 : (a.gamma_d ? a.gamma_d[row] : (double)a.gamma[row]);

  __syncthreads();
  // The chunk's seeds into its bitmask and position list (seeds i0 + tid +
  // kFusedThreads * j; entries past k are -1).
  auto list_seeds = [&](int i0, const int64_t (&key)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const bool in = i0 + tid + kFusedThreads * j < a.k && key[j] >= base && key[j] < base + n_chunk;
      if (in) {
        const uint32_t bit = 1u << (key[j] & 31);
        const uint32_t was = __hip_atomic_fetch_or(&seed_bits[(key[j] - base) >> 5], bit, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_WORKGROUP);
        if (!(was & bit))  // listed once, even if the caller repeats a seed
          seed_list[__hip_atomic_fetch_add(&s_nseeds, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)] =
              (uint16_t)(key[j] - base);
      }
    }
  };
  list_seeds(0, first_keys);
  for (int i0 = 8 * kFusedThreads; i0 < a.k; i0 += 8 * kFusedThreads) {  // eight loads in flight per thread
    int64_t key[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) key[j] = seeds[min(i0 + tid + kFusedThreads * j, a.k - 1)];
    list_seeds(i0, key);
  }
  __syncthreads();
  DSA_TRACE_MARK(g_trace_static, blockIdx.x, 1);

  const uint8_t* row_keys = a.keys + (size_t)row * a.key_stride * KF::kRowBytes;
  const int valid_bytes = L * KF::kRowBytes;  // below 2^31 (L <= 131072)
  uint32_t loff[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) loff[t] = KF::lane_offset(t, r, g);
  // Unit ul of the chunk through its own resource, tile t loaded iff bit t of
  // `tiles` (else an offset past the resource: zeros, no memory access).
  // A seed's row is not loaded again: its score is the seed phase's.
  auto load_unit = [&](int ul, uint32_t tiles, uint4 (&buf)[4][KF::kRaw]) {
    const int ub = (base + 64 * ul) * KF::kRowBytes;
    const BufferRsrc unit = make_buffer(row_keys + ub, (uint32_t)max(valid_bytes - ub, 0));
    const uint32_t sw[2] = {seed_bits[2 * ul], seed_bits[2 * ul + 1]};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const bool seed = (sw[t >> 1] >> (16 * (t & 1) + r)) & 1u;
      KF::load_at(unit, ((tiles >> t) & 1u) && !seed ? loff[t] : kOutOfRange, buf[t]);
    }
  };
  // Lane l's score of key l of the unit.
  auto score_of = [&](int ul, const uint4 (&buf)[4][KF::kRaw]) {
    float s[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) s[t] = tile_contrib<Tag, 4, KF>(qa, wr, buf[t]);
    float v = unit_reduce(s, g);
    if constexpr (KF::kScaled) v *= s_scales[((base + 64 * ul) >> 7) - (base >> 7)];
    return v;
  };

  // The wave's first unit is loaded now, before the threshold is known, with
  // every tile but the seeds' rows: its latency then overlaps the seed phase
  // and the exchange, and the tiles the decisions prune are discarded (a
  // static step so loads at most one unit per wave of pruned keys).
  constexpr int NB = KF::kBuffers;
  uint4 buf[NB][4][KF::kRaw];
  if (units > wave) load_unit(wave, 0xfu, buf[0]);

  // 1. The chunk's seeds, gathered 64 per wave-tile so that every wave's
  // loads are in flight together: only their key rows are loaded.
  uint32_t least = 0xffffffffu;
  {
    const uint32_t n_seeds = s_nseeds;
    const BufferRsrc row_rsrc = make_buffer(row_keys, (uint32_t)valid_bytes);
    constexpr int kPerWave = 1;  // gathered tiles a wave loads before scoring them (one: the first unit is held)
    for (uint32_t e0 = 64u * kPerWave * wave; e0 < n_seeds; e0 += 64u * kPerWave * kFusedWaves) {
      uint4 sbuf[kPerWave][4][KF::kRaw];
#pragma unroll
      for (int q = 0; q < kPerWave; ++q)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const uint32_t e = e0 + 64u * q + 16u * t + (uint32_t)r;
          const int key = e < n_seeds ? base + (int)seed_list[e] : (int)kFarKey;
          KF::load_buf(row_rsrc, key, g, sbuf[q][t]);
        }
#pragma unroll
      for (int q = 0; q < kPerWave; ++q) {
        const uint32_t e = e0 + 64u * q + (uint32_t)lane;  // lane l holds entry e0 + 64q + l
        float sc[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) sc[t] = tile_contrib<Tag, 4, KF>(qa, wr, sbuf[q][t]);
        float v = unit_reduce(sc, g);
        if (e < n_seeds) {
          const int local = seed_list[e];
          if constexpr (KF::kScaled) v *= s_scales[((base + local) >> 7) - (base >> 7)];
          chunk_scores[local] = v;
          least = min(least, float_to_ordered(v));
        }
      }
    }
  }
  for (int off = 32; off > 0; off >>= 1) least = min(least, (uint32_t)__shfl_xor((int)least, off, kWave));
  if (lane == 0 && least != 0xffffffffu)
    __hip_atomic_fetch_min(&s_least, least, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  __syncthreads();

  DSA_TRACE_MARK(g_trace_static, blockIdx.x, 2);
  // 2. Exchange: publish this chunk's least seed key, then wait for the row's.
  uint64_t* slots = a.ws.slots;
  if (tid == 0)
    __hip_atomic_store(&slots[logical], ((uint64_t)p.gen << 32) | s_least, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  if (wave == 0) {
    const uint32_t first = (uint32_t)row * (uint32_t)p.chunks;
    uint32_t tau = float_to_ordered(-__builtin_inff());  // if the wait gives up: keep every block
    uint32_t gave_up = kGaveUp;
    for (uint32_t it = 0; it < p.spin_limit; ++it) {
      bool ready = true;
      uint32_t mn = 0xffffffffu;
      for (int j = lane; j < p.chunks; j += kWave) {
        const uint64_t v = __hip_atomic_load(&slots[first + j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ready = ready && (uint32_t)(v >> 32) == p.gen;
        mn = min(mn, (uint32_t)v);
      }
      if (__ballot(!ready) == 0) {
        for (int off = 32; off > 0; off >>= 1) mn = min(mn, (uint32_t)__shfl_xor((int)mn, off, kWave));
        tau = mn;
        gave_up = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    if (lane == 0) {
      s_tau = tau;
      s_gave_up = gave_up;
    }
  }
  __syncthreads();

  DSA_TRACE_MARK(g_trace_static, blockIdx.x, 3);
  // 3. Decisions for the chunk's blocks (whole blocks: chunks are multiples
  // of 256 keys), their flags, and the keys scored.
  const double bound = (double)ordered_to_float(s_tau);
  uint32_t count = 0;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int b = b_first + tid + kFusedThreads * j;
    if (b >= b_end) continue;
    // U_b: +inf for a block with keys the previous step did not have.
    const float pm = b < a.prev_blocks ? pm_raw[j] : -__builtin_inff();
    const double upper = grown && b >= first_new ? HUGE_VAL : (double)pm + (a.margins ? margin_raw[j] : gamma);
    const bool keep = !(upper < bound);
    a.evaluated[(size_t)row * a.blocks + b] = keep ? 1 : 0;
    const int k0 = b * bs;
    const int k1 = min(L, k0 + bs);
    for (int key = k0; key < k1; key += 16) {  // 16-key tiles
      const int t = (key - base) >> 4;
      if (keep) {
        __hip_atomic_fetch_or(&tile_bits[t >> 5], 1u << (t & 31), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        count += (uint32_t)min(16, k1 - key);
      } else {
        uint32_t bits = (seed_bits[t >> 1] >> (16 * (t & 1))) & 0xffffu;
        if (k1 - key < 16) bits &= (1u << (k1 - key)) - 1u;
        count += (uint32_t)__builtin_popcount(bits);
      }
    }
  }
  if (count) __hip_atomic_fetch_add(&s_count, count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  __syncthreads();
  if (tid == 0) a.ws.qk_parts[logical] = s_count | s_gave_up;  // s_count <= chunk_keys < 2^31

  DSA_TRACE_MARK(g_trace_static, blockIdx.x, 4);
  // 4. The chunk's scores: kept tiles scored, the rest -inf but for seeds.
  // Units stream through a ring of KF::kBuffers register buffers as in the
  // dense kernel (the unit kBuffers - 1 ahead is always in flight; past the
  // wave's last unit the prefetch repeats that unit).
  const BufferRsrc out = make_buffer(a.scores + (size_t)row * L, (uint32_t)L * 4u);
  const int count_units = units > wave ? (units - wave + kFusedWaves - 1) / kFusedWaves : 0;
  auto tiles_of = [&](int ul) {
    return __builtin_amdgcn_readfirstlane((tile_bits[ul >> 3] >> (4 * (ul & 7))) & 0xfu);
  };
  auto finish_unit = [&](int ul, const uint4 (&buf)[4][KF::kRaw]) {
    const uint32_t tiles = tiles_of(ul);
    float v = 0.f;
    if (tiles) v = score_of(ul, buf);
    const uint32_t word = seed_bits[2 * ul + (lane >> 5)];
    const bool seed = (word >> (lane & 31)) & 1u;
    const bool kept = (tiles >> (lane >> 4)) & 1u;
    const int local = 64 * ul + lane;
    const float s = seed ? chunk_scores[local] : (kept ? v : -__builtin_inff());
    buffer_store_f32(out, (uint32_t)(base + local) * 4u, s);  // stores past L are dropped
    chunk_scores[local] = s;
    if (base + local < L)
      __hip_atomic_fetch_add(&hist[float_to_ordered(s) >> 20], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  };
  if (count_units > 0) {
    const int last = wave + kFusedWaves * (count_units - 1);
#pragma unroll
    for (int s = 1; s < NB - 1; ++s) {  // (unit 0, the wave's first, is in flight already)
      const int ul = min(wave + kFusedWaves * s, last);
      load_unit(ul, tiles_of(ul), buf[s]);
    }
    for (int i = 0; i < count_units; i += NB) {
#pragma unroll
      for (int s = 0; s < NB; ++s) {
        if (i + s >= count_units) break;
        const int ahead = min(wave + kFusedWaves * (i + s + NB - 1), last);
        load_unit(ahead, tiles_of(ahead), buf[(s + NB - 1) % NB]);
        __builtin_amdgcn_sched_barrier(0);
        finish_unit(wave + kFusedWaves * (i + s), buf[s]);
      }
    }
  }
  __syncthreads();

  DSA_TRACE_MARK(g_trace_static, blockIdx.x, 5);
  // 5. The chunk's candidate list for the list select.
  write_chunk_list<kFusedWaves>(hist, chunk_scores, p.chunk_keys, n_chunk, base, p.quota,
                                a.ws.select.cand + (size_t)row * L + base,
                                a.ws.select.list_meta + 2 * ((size_t)row * kMaxListChunks + c), &s_list_bin, s_wsum);
  DSA_TRACE_MARK(g_trace_static, blockIdx.x, 6);
}

// Polls of the exchange before a workgroup gives up: kSpinLimit, or
// DSA_AMD_STATIC_SPIN_LIMIT from the environment (a test sets 0 to make
// every wait give up from the host, so the kernel still ends normally).
uint32_t spin_limit() { return env_limit("DSA_AMD_STATIC_SPIN_LIMIT", kSpinLimit, kSpinLimit); }

template <class Tag, class KF>
int launch_static(TemporalArgs& a, const ListPlan& plan, hipStream_t stream, bool& ran) {
  const int64_t total = (int64_t)a.rows * plan.chunks;
  const int64_t grid = (total + kXcds - 1) / kXcds * kXcds;
  const size_t lds = (size_t)plan.chunk_keys * sizeof(float);
  int64_t capacity = 0;
  if (int st = resident_capacity(reinterpret_cast<const void*>(&temporal_static_kernel<Tag, KF>), kFusedThreads, lds,
                                 capacity))
    return st;
  if (total > kMaxFusedWgs || grid > capacity) return DSA_STATUS_OK;  // not resident at once: the launch path
  FusedPlan p;
  p.chunk_keys = plan.chunk_keys;
  p.chunks = plan.chunks;
  p.quota = (uint32_t)plan.quota;
  p.total_wgs = (uint32_t)total;
  p.gen = next_generation();
  p.spin_limit = spin_limit();
  hipLaunchKernelGGL((temporal_static_kernel<Tag, KF>), dim3((unsigned)grid), dim3(kFusedThreads), (uint32_t)lds,
                     stream, a, p);
  if (int st = check_launch("temporal_static_kernel")) return st;
  ran = true;
  return DSA_STATUS_OK;
}

}  // namespace

int temporal_static_fused(TemporalArgs& a, int32_t key_dtype, int64_t* out_topk, hipStream_t stream, bool& ran) {
  ran = false;
  if (a.policy_mode != 0 || a.source) return DSA_STATUS_OK;
  const ListPlan plan = list_plan(a.rows, a.length, a.k);
  if (!plan.on) return DSA_STATUS_OK;
  int st;
  switch (key_dtype) {
    case DSA_DTYPE_BF16: st = launch_static<Bf16Tag, KeysB16>(a, plan, stream, ran); break;
    case DSA_DTYPE_F16: st = launch_static<F16Tag, KeysB16>(a, plan, stream, ran); break;
    default: st = launch_static<Bf16Tag, KeysFP8>(a, plan, stream, ran); break;
  }
  if (st || !ran) return st;
  return launch_select_lists(a.scores, a.rows, a.length, a.k, plan, a.ws.select, out_topk, nullptr, stream, nullptr,
                             nullptr, a.ws.qk_parts, a.qk_scored, a.waits_given_up);
}

}  // namespace dsa

#ifdef DSA_PHASE_TRACE
// The fused static temporal kernel's phase log (trace builds only).
extern "C" int dsa_trace_temporal_static(uint64_t* host, int64_t n, int32_t clear) {
  using namespace dsa;
  DSA_REQUIRE(host && n >= 0 && n <= int64_t(kTraceWgs) * kTraceMarks, "bad trace read");
  if (int st = check_hip(hipMemcpyFromSymbol(host, HIP_SYMBOL(g_trace_static), (size_t)n * 8), "trace read"))
    return st;
  if (clear) {
    static const uint64_t zeros[kTraceWgs * kTraceMarks] = {};
    return check_hip(hipMemcpyToSymbol(HIP_SYMBOL(g_trace_static), zeros, sizeof(zeros)), "trace clear");
  }
  return DSA_STATUS_OK;
}
#endif
