// Indexer scoring kernels: dense batched scores (the decode hot path), the
// fp32 accuracy path, and the block-granular H8 / masked / progressive kernels.
//
// score[s] = sum_h w_h * ReLU(q_h . k_s) over 64 heads x 128 dims.  The
// 64x128 . 128xN head contraction runs on v_mfma_f32_16x16x32_{bf16,f16}; the
// ReLU, the signed head weight and the 64-head reduction are applied to the
// accumulators in registers, so only the fp32 score leaves the kernel.
#include "common.hpp"
#include "indexer.hpp"
#include "lists.hpp"
#include "select.hpp"
#include "status.hpp"
#include "waveops.hpp"

namespace dsa {
namespace {

// ---------------------------------------------------------------------------
// Dense scores for many query "sequences".  Sequence s has its own query block
// (head_count heads gathered by head_ids, or heads 0..head_count-1) and weights,
// and reads key set s / queries_per_keyset.  This one kernel covers batched
// decode (one query per key set), multi-query scoring with an optional causal
// mask (many queries per key set) and head-sparse verifier scoring.
//
// Flat grid: workgroup x = s * wgs_per_seq + chunk, 4 waves per workgroup; a
// unit is 64 consecutive keys (4 MFMA tiles).  Each wave keeps its sequence's
// query block in registers (16 VGPRs per 16-head tile of A fragments) and
// streams units with a two-deep register prefetch.  After the four tiles of a
// unit the per-lane partials are transposed and reduced across the four lane
// groups so that lane l ends with the score of key 64u + l and the store is one
// coalesced 256-byte row.
// ---------------------------------------------------------------------------
#ifdef DSA_PHASE_TRACE
// Decode scoring (candidate-list variant), per workgroup (by blockIdx.x):
// 0 start, 1 first unit scored, 2 last unit scored, 3 list written.
__device__ uint64_t g_trace_dense[kTraceWgs * kTraceMarks];
#endif

struct DenseArgs {
  const uint16_t* q;
  int64_t q_stride;  // elements between sequences' query blocks
  const float* w;
  int64_t w_stride;
  const int32_t* head_ids;  // nullable
  int64_t ids_stride;       // 0: one id list shared by all sequences
  int32_t head_count;
  const uint8_t* keys;
  int64_t key_stride;  // key rows between key sets
  int32_t queries_per_keyset;
  const float* scales;
  int64_t scale_stride;
  float* out;
  int64_t out_stride;
  int32_t length;
  int32_t causal_offset;  // < 0: no mask; else key j is valid for query t iff j <= t + offset
  int32_t units_per_wg;
  int32_t wgs_per_seq;
  int64_t total_wgs;  // the launch pads the grid to a multiple of kXcds
  uint32_t* hist;  // [sequences][kSelectBins] score histogram (kHist only)
  // Candidate lists (kLists only): list (s, chunk) at lists[s * length + chunk * chunk_keys].
  uint64_t* lists;
  uint32_t* list_meta;  // [sequences][kMaxListChunks][2]: length, lowest bin listed
  int32_t list_quota;
  // Top-k of every score row inside the prefill kernel (kTopK only).
  int32_t topk;
  int64_t* topk_idx;  // [sequences][topk_stride]
  float* topk_val;    // nullable, same layout
  int64_t topk_stride;
};

// The key rows a wave streams: the key set's base, its valid bytes (below
// 2^31), and the lane's offsets of the four tiles of a unit (loop-invariant
// registers).
template <class KF>
struct KeyStream {
  const uint8_t* base;
  uint32_t valid_bytes;
  uint32_t loff[4];
  __device__ __forceinline__ KeyStream(const uint8_t* b, uint32_t bytes, int r, int g) : base(b), valid_bytes(bytes) {
#pragma unroll
    for (int t = 0; t < 4; ++t) loff[t] = KF::lane_offset(t, r, g);
  }
};

// Each unit is loaded through its own buffer resource, based at the unit's
// first key and bounded by the valid keys (keys past them read as zeros).
// The resource is wave-uniform (scalar registers) and the lane offsets never
// change, so no address register of the loop is ever a load destination: the
// compiler then has no reason to drain the loads in flight at the loop head.
// Scaled keys also fetch the unit's scale (a 64-key unit lies in one 128-key
// scale block) with the keys, so the compute never waits on it.
template <class KF>
__device__ __forceinline__ void dense_load_unit(const KeyStream<KF>& ks, int u, uint4 (&buf)[4][KF::kRaw],
                                                const float* scales, int L, float& scale) {
  const uint32_t ub = (uint32_t)u * 64u * KF::kRowBytes;
  // Signed difference and max, which stay scalar (an unsigned saturating
  // subtract becomes a vector instruction, and with it the resource).
  const int rem = max((int)ks.valid_bytes - (int)ub, 0);
  const BufferRsrc unit = make_buffer(ks.base + ub, (uint32_t)rem);
#pragma unroll
  for (int t = 0; t < 4; ++t) KF::load_at(unit, ks.loff[t], buf[t]);
  if constexpr (KF::kScaled) scale = scales[min(u * 64, L - 1) >> 7];
}

template <class Tag, class KF, int M, bool kHist, bool kLists>
__device__ __forceinline__ void dense_compute_unit(const uint4 (&qa)[M][4], const float (&wr)[M][4],
                                                   const uint4 (&buf)[4][KF::kRaw], int u,
                                                   int valid, int L, int lane, int g,
                                                   float scale, BufferRsrc out,
                                                   uint32_t* hist, float* chunk_scores, int chunk_base) {
  float s[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) s[t] = tile_contrib<Tag, M, KF>(qa, wr, buf[t]);
  float keep = unit_reduce(s, g);
  const int key = u * 64 + lane;
  if constexpr (KF::kScaled) keep *= scale;
  // Stores past L are dropped by the buffer bounds check.
  buffer_store_f32(out, (uint32_t)key * 4, key < valid ? keep : -__builtin_inff());
  if constexpr (kLists) chunk_scores[key - chunk_base] = keep;
  if constexpr (kHist)
    __hip_atomic_fetch_add(&hist[float_to_ordered(keep) >> 20], key < valid ? 1u : 0u,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// The streaming part of dense_scores_kernel: query block into registers, then
// the two-buffer unit loop.  `after_issue` runs once the query tiles and the
// first units' loads are in flight (the workgroup's barrier, for the kernels
// that clear an LDS histogram first), so that its wait overlaps them.
template <class Tag, class KF, int M, bool kGather, bool kHist, bool kLists, class AfterIssue>
__device__ __forceinline__ void dense_stream(const DenseArgs& a, int count, int u_first, int u_stride,
                                             int64_t seq, int valid, int L, int lane, int r, int g,
                                             const uint8_t* key_base, uint32_t key_bytes, BufferRsrc out,
                                             const float* scales,
                                             uint32_t* hist, float* chunk_scores, int chunk_base,
                                             AfterIssue after_issue) {
  uint4 qa[M][4];
  float wr[M][4];
  if constexpr (kGather) {
    const int32_t* ids = a.head_ids ? a.head_ids + seq * a.ids_stride : nullptr;
    load_head_tiles<M, KF::kNaturalK>(a.q + seq * a.q_stride, a.w + seq * a.w_stride, ids, a.head_count, r, g, qa,
                       wr);
  } else {
    load_dense_head_tiles<M, KF::kNaturalK>(a.q + seq * a.q_stride, a.w + seq * a.w_stride, r, g, qa, wr);
  }

  // A ring of KF::kBuffers register buffers.  The loads of the unit
  // kBuffers - 1 ahead are always issued before the current unit is computed;
  // past the wave's last unit the prefetch re-reads that last unit (an L2
  // hit), so no load is conditional and the compiler's vmcnt waits cover
  // exactly the buffer being consumed.
  constexpr int NB = KF::kBuffers;
  const KeyStream<KF> ks(key_base, key_bytes, r, g);
  const int u_last = u_first + u_stride * (count - 1);
  uint4 buf[NB][4][KF::kRaw];
  float scale[NB] = {};
#pragma unroll
  for (int s = 0; s < NB - 1; ++s)
    dense_load_unit<KF>(ks, min(u_first + u_stride * s, u_last), buf[s], scales, L, scale[s]);
  after_issue();
  for (int i = 0; i < count; i += NB) {
    const int u = u_first + u_stride * i;
#pragma unroll
    for (int s = 0; s < NB; ++s) {
      if (i + s >= count) break;
      dense_load_unit<KF>(ks, min(u + u_stride * (s + NB - 1), u_last), buf[(s + NB - 1) % NB], scales, L,
                          scale[(s + NB - 1) % NB]);
      // The next unit's loads stay ahead of this unit's MFMAs: left to
      // itself the scheduler sinks them below the first unit's compute, so
      // every wave would start with a unit whose latency nothing hides.
      __builtin_amdgcn_sched_barrier(0);
      dense_compute_unit<Tag, KF, M, kHist, kLists>(qa, wr, buf[s], u + u_stride * s, valid, L, lane, g,
                                                    scale[s], out, hist, chunk_scores, chunk_base);
      if constexpr (kLists)
        if (i == 0 && s == 0) DSA_TRACE_MARK(g_trace_dense, blockIdx.x, 1);
    }
  }
  if constexpr (kLists) DSA_TRACE_MARK(g_trace_dense, blockIdx.x, 2);
}

template <class Tag, class KF, int M, bool kGather, bool kHist, bool kLists, int kWaves>
__global__ __launch_bounds__(64 * kWaves, kWaves == 4 ? 2 : 1) void dense_scores_kernel(DenseArgs a) {
  constexpr int kThreads = 64 * kWaves;
  // kHist: also count every valid score into a histogram of the top 12 bits
  // of its order-preserving key; without kLists it is added to the sequence's
  // histogram (input of the distributed top-k).  kLists: the workgroup keeps
  // its chunk's scores in LDS (dynamic shared memory, chunk_keys floats) and
  // writes its candidate list instead (input of the list top-k).
  static_assert(kHist || !kLists, "candidate lists come with the histogram");
  __shared__ uint32_t hist[kHist ? kSelectBins : 1];
  extern __shared__ float chunk_scores[];
  args_in_sgprs(a.q, a.q_stride, a.w, a.w_stride, a.keys, a.key_stride, a.queries_per_keyset, a.out,
                a.out_stride, a.length, a.causal_offset, a.units_per_wg, a.wgs_per_seq, a.total_wgs,
                gridDim.x);
  if constexpr (kHist && !kLists) args_in_sgprs(a.hist);
  if constexpr (kLists) args_in_sgprs(a.lists, a.list_meta, a.list_quota);
  if constexpr (KF::kScaled) args_in_sgprs(a.scales, a.scale_stride);
  if constexpr (kGather) args_in_sgprs(a.head_ids, a.ids_stride, a.head_count);
  const int lane = threadIdx.x & 63;
  // Wave-uniform control flow: every loop bound below lives in SGPRs.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15;
  const int g = lane >> 4;
  // Workgroups are dispatched round-robin over the 8 XCDs; renumber them so
  // that consecutive logical workgroups (one sequence's chunks) share an XCD
  // and its L2 fetches that sequence's query block once.  (The launch keeps
  // the grid below 2^31 workgroups.)
  const uint32_t logical = (blockIdx.x % kXcds) * (gridDim.x / kXcds) + blockIdx.x / kXcds;
  if (logical >= (uint64_t)a.total_wgs) return;
  if constexpr (kLists) DSA_TRACE_MARK(g_trace_dense, blockIdx.x, 0);
  const int64_t seq = logical / (uint32_t)a.wgs_per_seq;
  const int chunk = (int)(logical % (uint32_t)a.wgs_per_seq);
  const int L = a.length;
  const int64_t keyset = seq / a.queries_per_keyset;
  int valid = L;
  if (a.causal_offset >= 0)
    valid = min(L, (int)(seq % a.queries_per_keyset) + a.causal_offset + 1);

  const uint8_t* key_base = a.keys + keyset * a.key_stride * KF::kRowBytes;
  const uint32_t key_bytes = (uint32_t)valid * KF::kRowBytes;
  float* out_ptr = a.out + seq * a.out_stride;
  const BufferRsrc out = make_buffer(out_ptr, (uint32_t)L * 4u);
  const float* scales = KF::kScaled ? a.scales + keyset * a.scale_stride : nullptr;

  // This wave owns units u_first, u_first + 4, ... of the workgroup's chunk
  // (a contiguous run of units_per_wg units); those at or past u_compute_end
  // lie wholly beyond the causal limit and only get -inf.  (Interleaving the
  // units over all of a sequence's waves measured ~10 % slower; handing them
  // out from a per-sequence atomic counter serialises on that counter.)
  const int u_stride = kWaves;
  const int u_end = min((L + 63) >> 6, (chunk + 1) * a.units_per_wg);
  const int u_first = chunk * a.units_per_wg + wave;
  const int u_compute_end = min(u_end, (valid + 63) >> 6);
  const int count = u_compute_end > u_first ? (u_compute_end - u_first + u_stride - 1) / u_stride : 0;
  for (int uu = u_first + u_stride * count; uu < u_end; uu += u_stride)
    buffer_store_f32(out, (uint32_t)(uu * 64 + lane) * 4, -__builtin_inff());
  if constexpr (kHist) {
#pragma unroll
    for (int j = 0; j < kSelectBins / kThreads; ++j) hist[threadIdx.x + kThreads * j] = 0;
    // The cleared histogram is published by one barrier per wave, taken after
    // the wave's first loads are issued (a wave with no units takes it here).
    auto publish = [] {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
    };
    const int chunk_keys = a.units_per_wg * 64;
    const int chunk_base = chunk * chunk_keys;
    if (count > 0)
      dense_stream<Tag, KF, M, kGather, kHist, kLists>(a, count, u_first, u_stride, seq, valid, L, lane, r, g,
                                                       key_base, key_bytes, out, scales, hist, chunk_scores,
                                                       chunk_base, publish);
    else
      publish();
    __syncthreads();
    if constexpr (kLists) {
      // The chunk's list: every valid key whose bin is at least the bin of
      // the chunk's list_quota-th largest score (all valid keys when the
      // chunk has no more), in index order.
      __shared__ uint32_t s_list_bin;
      __shared__ __align__(16) uint32_t s_list_wsum[kWaves];
      write_chunk_list<kWaves>(hist, chunk_scores, chunk_keys, min(chunk_keys, valid - chunk_base), chunk_base,
                               (uint32_t)a.list_quota, a.lists + seq * (int64_t)L + chunk_base,
                               a.list_meta + 2 * (seq * kMaxListChunks + chunk), &s_list_bin, s_list_wsum);
      DSA_TRACE_MARK(g_trace_dense, blockIdx.x, 3);
      return;
    }
    // All sixteen LDS reads first, then the atomics for the bins in use: one
    // LDS round trip instead of one per bin.
    uint32_t* ghist = a.hist + seq * kSelectBins;
    uint32_t n[kSelectBins / kThreads];
#pragma unroll
    for (int j = 0; j < kSelectBins / kThreads; ++j) n[j] = hist[threadIdx.x + kThreads * j];
#pragma unroll
    for (int j = 0; j < kSelectBins / kThreads; ++j)
      if (n[j])
        __hip_atomic_fetch_add(&ghist[threadIdx.x + kThreads * j], n[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  if (count == 0) return;
  dense_stream<Tag, KF, M, kGather, kHist, kLists>(a, count, u_first, u_stride, seq, valid, L, lane, r, g, key_base,
                                                   key_bytes, out, scales, hist, chunk_scores, 0, [] {});
}


// ---------------------------------------------------------------------------
// Multi-query (prefill) scoring: many query blocks against one shared key set.
// A workgroup owns kPrefillQueries consecutive queries of one key set, one
// per wave, and streams the key units they see through LDS: each 64-key unit
// is loaded from memory once and scored for all four queries, instead of
// once per query.  Rows are padded to kPrefillRow bytes so the 16 rows a lane
// group reads fall on different banks.  With a causal limit the heaviest
// query blocks are dispatched first.  One query per wave needs about half the
// registers of two; a workgroup holds one wave per SIMD and two or three
// workgroups share a CU, so one workgroup's barrier waits and its top-k
// epilogue run under another's MFMAs (eight queries per workgroup, one
// workgroup per CU, measured 5 us slower per C4 layer; two, 60 us slower).
// ---------------------------------------------------------------------------
constexpr int kPrefillQueries = 4;
constexpr int kPrefillRow = 272;

// ---------------------------------------------------------------------------
// Exact top-k of one query's score row at the end of the prefill kernel, with
// stable_topk's set (metrics.py:9-22: every score above the k-th largest, ties
// at it to the lower index, -0.0 equal to +0.0) written in ascending index
// order.  One wave per row of at most kTopKRowMax keys, after the wave's own
// score stores have completed: it reads the row back (lane l holds keys
// 256 j + 4 l + c), counts the valid scores into kTopKBins LDS bins spaced
// linearly between the row's minimum and maximum, and finds the bin of the
// k-th largest.  Inside that bin the cut is resolved by ranking its keys
// against each other when there are at most 64 of them, else by a radix over
// their order-preserving keys (digits of 10, 10, 10 and 2 bits).  The cut is
// a (value, index) pair of the (value desc, index asc) order; a last pass
// writes every valid key at or above it.  Rows with at most k valid keys
// return all of them, padded with index -1 / value -inf.
// ---------------------------------------------------------------------------
constexpr int kTopKRowMax = 4096;
constexpr int kTopKBins = 1024;
// the bins, then 64 candidates (values, indices), then 4 spare words
constexpr int kTopKScratch = kTopKBins + 2 * kWave + 4;

// Completes this wave's LDS operations before the next ones are issued (a
// wave's own LDS traffic, so no barrier).
__device__ __forceinline__ void wave_lds_fence() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

__device__ __forceinline__ void zero_wave_bins(uint32_t* bins, int lane) {
  uint4* b4 = reinterpret_cast<uint4*>(bins);
#pragma unroll
  for (int q = 0; q < kTopKBins / 4 / kWave; ++q) b4[lane + kWave * q] = make_uint4(0u, 0u, 0u, 0u);
}

// Key of register slot e of a lane in the read-back row, and the linear bin
// of a value.
__device__ __forceinline__ int topk_key(int e, int lane) { return 256 * (e >> 2) + 4 * lane + (e & 3); }
// x * scale + nlo, nlo = -lo * scale, is monotone in x.  v_cvt_i32_f32
// saturates (-inf to INT_MIN) and converts NaN to 0, so -inf (a key past the
// visible ones, or any key when scale is 0) lands in bin 0; it is issued
// directly because the C++ conversion leaves those inputs undefined.
__device__ __forceinline__ int topk_bin(float x, float /*lo*/, float scale, float nlo) {
  int b;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(b) : "v"(fmaf(x, scale, nlo)));
  return min(max(b, 0), kTopKBins - 1);
}

// Every pass below walks the row in blocks of 256 keys (one float4 per lane):
// blocks wholly past the visible keys are skipped (a wave-uniform branch),
// and within the others each key is tested against the visible count.
#define DSA_TOPK_BLOCKS(BODY)                                  \
  _Pragma("unroll") for (int j = 0; j < 16; ++j) {             \
    if (256 * j < vis) {                                       \
      [[maybe_unused]] constexpr bool kPartial = true;         \
      BODY                                                     \
    }                                                          \
  }

__device__ __forceinline__ void prefill_topk_row(BufferRsrc row, int vis, int length, int k, int64_t* out_idx,
                                                 float* out_val, uint32_t* scratch, int lane) {
  float v[64];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    uint4 q = make_uint4(0u, 0u, 0u, 0u);
    if (256 * j < vis) q = buffer_load_16(row, (uint32_t)(256 * j + 4 * lane) * 4u);
    v[4 * j + 0] = __uint_as_float(q.x);
    v[4 * j + 1] = __uint_as_float(q.y);
    v[4 * j + 2] = __uint_as_float(q.z);
    v[4 * j + 3] = __uint_as_float(q.w);
  }
  // The kernel stored -inf at the row's keys past the visible ones; keys past
  // the row's length (in its last block) read 0 from the buffer and become
  // -inf here, so that every key past the visible ones is -inf below.
#pragma unroll
  for (int j = 0; j < 16; ++j)
    if (256 * j < vis && 256 * j + 256 > length)
#pragma unroll
      for (int t = 0; t < 4; ++t) v[4 * j + t] = 256 * j + 4 * lane + t < length ? v[4 * j + t] : -__builtin_inff();
  // key 256 j + 4 lane + t of the last block is visible iff t < tail
  const int tail = vis - 4 * lane;
  const bool all = vis <= k;
  // The cut: key i with value x is kept iff x > tv or (x == tv and i <= ti).
  // With at most k visible keys it keeps every finite score, and no -inf
  // (the keys past the visible ones).
  float tv = -__builtin_inff();
  int ti = -1;
  if (!all) {
    // The kernel stored -inf past the visible keys, and a visible score is
    // finite: the range needs no visibility test.
    float lo = __builtin_inff(), hi = -__builtin_inff();
    DSA_TOPK_BLOCKS(
      const float* x = &v[4 * j];
      hi = fmaxf(fmaxf(hi, x[0]), fmaxf(x[1], fmaxf(x[2], x[3])));
_Pragma("unroll")
      for (int t = 0; t < 4; ++t) lo = fminf(lo, x[t] == -__builtin_inff() ? __builtin_inff() : x[t]);)
    lo = wave_min(lo);
    hi = wave_max(hi);
    // Monotone binning: bin(x) > bin(y) implies x > y.  A single value, or a
    // span that overflows, puts every key in bin 0 (the radix below resolves it).
    float scale = (float)kTopKBins / (hi - lo);
    float nlo = -lo * scale;
    if (!(scale <= 3.0e38f) || !(fabsf(nlo) <= 3.0e38f)) scale = nlo = 0.f;
    zero_wave_bins(scratch, lane);
    wave_lds_fence();
    // Keys past the visible ones (-inf) count into bin 0: the counts above
    // the cut bin, and so the rank wanted inside it, are exact; only bin 0's
    // own count may exceed its visible keys, which the passes below test.
    DSA_TOPK_BLOCKS(
_Pragma("unroll")
      for (int t = 0; t < 4; ++t)
        __hip_atomic_fetch_add(&scratch[topk_bin(v[4 * j + t], lo, scale, nlo)], 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);)
    wave_lds_fence();
    const Locate loc = wave_locate<kTopKBins / kWave>(scratch, (uint32_t)k, false);
    const int cut_bin = (int)loc.digit;
    if (loc.count <= (uint32_t)kWave) {
      // The cut bin's keys, listed in index order, each ranked against all.
      float* cval = reinterpret_cast<float*>(scratch + kTopKBins);
      int* cidx = reinterpret_cast<int*>(scratch + kTopKBins + kWave);
      uint32_t n = 0;
      DSA_TOPK_BLOCKS(
        bool c[4];
        uint32_t cnt = 0;
_Pragma("unroll")
        for (int t = 0; t < 4; ++t) {
          c[t] = topk_bin(v[4 * j + t], lo, scale, nlo) == cut_bin && v[4 * j + t] != -__builtin_inff();
          cnt += c[t] ? 1u : 0u;
        }
        if (__ballot(cnt != 0) != 0) {
          const uint32_t incl = wave_incl_scan(cnt);
          uint32_t pos = n + incl - cnt;
_Pragma("unroll")
          for (int t = 0; t < 4; ++t)
            if (c[t] && pos < (uint32_t)kWave) {
              cval[pos] = v[4 * j + t];
              cidx[pos] = topk_key(4 * j + t, lane);
              ++pos;
            }
          n += __builtin_amdgcn_readlane(incl, kWave - 1);
        })
      wave_lds_fence();
      float cv = 0.f;
      int ci = 0;
      uint32_t rank = 0;
      if ((uint32_t)lane < n) {
        cv = cval[lane];
        ci = cidx[lane];
        for (uint32_t m = 0; m < n; ++m) {
          const float ov = cval[m];
          const int oi = cidx[m];
          rank += (ov > cv || (ov == cv && oi < ci)) ? 1u : 0u;
        }
      }
      const uint64_t hit = __ballot((uint32_t)lane < n && rank == loc.rem - 1);
      const int owner = (int)__builtin_ctzll(hit);
      tv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cv), owner));
      ti = __builtin_amdgcn_readlane(ci, owner);
    } else {
      // Radix over the order keys of the cut bin's keys, most significant
      // digit first; then the want-th of the keys equal to the cut, by index.
      uint32_t prefix = 0, pmask = 0, want = loc.rem;
#pragma unroll
      for (int pass = 0; pass < 4; ++pass) {
        const int shift = pass < 3 ? 22 - 10 * pass : 0;
        const uint32_t dmask = pass < 3 ? 1023u : 3u;
        wave_lds_fence();
        zero_wave_bins(scratch, lane);
        wave_lds_fence();
        DSA_TOPK_BLOCKS(
_Pragma("unroll")
          for (int t = 0; t < 4; ++t) {
            const uint32_t o = float_to_ordered(v[4 * j + t]);
            if ((!kPartial || 256 * j + t < tail) && topk_bin(v[4 * j + t], lo, scale, nlo) == cut_bin &&
                (o & pmask) == prefix)
              __hip_atomic_fetch_add(&scratch[(o >> shift) & dmask], 1u, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_WORKGROUP);
          })
        wave_lds_fence();
        const Locate d = wave_locate<kTopKBins / kWave>(scratch, want, false);
        prefix |= d.digit << shift;
        pmask |= dmask << shift;
        want = d.rem;
      }
      uint32_t seen = 0;
      DSA_TOPK_BLOCKS(
        bool eq[4];
        uint32_t cnt = 0;
_Pragma("unroll")
        for (int t = 0; t < 4; ++t) {
          eq[t] = (!kPartial || 256 * j + t < tail) && float_to_ordered(v[4 * j + t]) == prefix;
          cnt += eq[t] ? 1u : 0u;
        }
        const uint32_t incl = wave_incl_scan(cnt);
        const uint32_t total = __builtin_amdgcn_readlane(incl, kWave - 1);
        if (ti < 0 && seen + total >= want) {
          const uint32_t before = seen + incl - cnt;
          const uint64_t m = __ballot(before < want && want <= seen + incl);
          const int owner = (int)__builtin_ctzll(m);
          uint32_t r = want - before;  // meaningful on the owner lane
          int found = 0;
_Pragma("unroll")
          for (int t = 0; t < 4; ++t)
            if (eq[t] && r != 0) {
              if (--r == 0) found = topk_key(4 * j + t, lane);
            }
          ti = __builtin_amdgcn_readlane(found, owner);
        }
        seen += total;)
      tv = ordered_to_float(prefix);
    }
  }
  uint32_t base = 0;
  DSA_TOPK_BLOCKS(
    bool s[4];
    uint32_t cnt = 0;
_Pragma("unroll")
    for (int t = 0; t < 4; ++t) {
      const int key = topk_key(4 * j + t, lane);
      const float x = v[4 * j + t];
      s[t] = x > tv || (x == tv && key <= ti);
      cnt += s[t] ? 1u : 0u;
    }
    const uint32_t incl = wave_incl_scan(cnt);
    uint32_t pos = base + incl - cnt;
_Pragma("unroll")
    for (int t = 0; t < 4; ++t)
      if (s[t] && pos < (uint32_t)k) {
        out_idx[pos] = topk_key(4 * j + t, lane);
        if (out_val) out_val[pos] = v[4 * j + t];
        ++pos;
      }
    base += __builtin_amdgcn_readlane(incl, kWave - 1);)
  for (int p = (int)base + lane; p < k; p += kWave) {
    out_idx[p] = -1;
    if (out_val) out_val[p] = -__builtin_inff();
  }
}
#undef DSA_TOPK_BLOCKS

// The unit loop is software-pipelined across tiles and units: step t issues
// the MFMAs of tile t and the ReLU / weight work of tile t - 1 (tile 3 of the
// previous unit at step 0), interleaved by scheduling groups, while the next
// tile's LDS reads are in flight.  The
// previous unit's reduction and store follow step 0.
__device__ __forceinline__ void mfma_valu_interleave() {
  // One MFMA to up to three VALU instructions (a tile's 32 ReLU / FMA
  // instructions, plus the unit reduction's after step 0); one to two and two
  // to four measured 1-2 % slower.
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
    __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // three VALU
  }
}

template <class Tag, bool kTopK>
__global__ __launch_bounds__(64 * kPrefillQueries, 2) void prefill_scores_kernel(DenseArgs a, int32_t qblocks,
                                                                            int32_t keysets) {
  constexpr int kThreads = 64 * kPrefillQueries;
  constexpr int kRowSplit = kThreads / 64;
  constexpr int kRowBytesPer = 256 / kRowSplit;
  constexpr int kVecs = kRowBytesPer / 16;
  __shared__ __align__(16) uint8_t lds[2][64 * kPrefillRow];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15;
  const int g = lane >> 4;
  const int qb = qblocks - 1 - (int)(blockIdx.x / keysets);  // heaviest first
  const int64_t keyset = blockIdx.x % keysets;
  const int L = a.length;
  const int qpk = a.queries_per_keyset;
  auto visible = [&](int t) { return a.causal_offset >= 0 ? min(L, t + a.causal_offset + 1) : L; };
  const int t_last = min(qpk - 1, qb * kPrefillQueries + kPrefillQueries - 1);
  const int units = (visible(t_last) + 63) >> 6;

  uint4 qa[4][4];
  float wr[4][4];
  const int t = qb * kPrefillQueries + wave;
  const bool active = t < qpk;
  const int64_t seq = keyset * qpk + (active ? t : 0);
  load_dense_head_tiles<4, KeysB16::kNaturalK>(a.q + seq * a.q_stride, a.w + seq * a.w_stride, r, g, qa, wr);
  const int vis = active ? visible(t) : 0;
  float* orow = a.out + seq * a.out_stride;
  const BufferRsrc orsrc = make_buffer(orow, active ? (uint32_t)L * 4u : 0u);

  const BufferRsrc kr = make_buffer(a.keys + keyset * a.key_stride * KeysB16::kRowBytes,
                                    (uint32_t)L * KeysB16::kRowBytes);
  const int lrow = threadIdx.x / kRowSplit;
  const int lpart = threadIdx.x % kRowSplit;
  uint4 stage[kVecs];  // the next unit, in flight while this one is scored
  auto fetch = [&](int u) {
    const uint32_t off = (uint32_t)(u * 64 + lrow) * KeysB16::kRowBytes + lpart * kRowBytesPer;
#pragma unroll
    for (int k = 0; k < kVecs; ++k) stage[k] = buffer_load_16(kr, off + 16 * k);
  };
  auto put = [&](int buf) {
    uint8_t* dst = lds[buf] + lrow * kPrefillRow + lpart * kRowBytesPer;
#pragma unroll
    for (int k = 0; k < kVecs; ++k) *reinterpret_cast<uint4*>(dst + 16 * k) = stage[k];
  };
  auto read_tile = [&](const uint8_t* base, int tile, uint4 (&raw)[KeysB16::kRaw]) {
    const uint8_t* row = base + (16 * tile + r) * kPrefillRow + g * 16;
#pragma unroll
    for (int c = 0; c < KeysB16::kRaw; ++c) raw[c] = *reinterpret_cast<const uint4*>(row + 64 * c);
  };
  // Stores are unconditional: the buffer bounds drop keys past L, every key
  // of an inactive query and the "previous unit" of the first iteration.
  auto store_unit = [&](const float (&sp)[4], int u) {
    const float score = unit_reduce(sp, g);
    const int key = u * 64 + lane;
    buffer_store_f32(orsrc, (uint32_t)key * 4u, key < vis ? score : -__builtin_inff());
  };

  // Every load is unconditional (a fetch past the last unit re-reads it), so
  // that the compiler counts the memory operations in flight exactly.
  const int last_unit = max(units - 1, 0);
  fetch(0);
  put(0);
  // The query tiles, weights and first unit have landed.  Without this wait
  // the compiler sees the query loads in flight at the loop head and places
  // their waits inside the loop, where they also wait for each iteration's
  // prefetch.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  floatx4 acc0[4], acc1[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) acc1[m] = floatx4{0.f, 0.f, 0.f, 0.f};
  float sp[4] = {0.f, 0.f, 0.f, 0.f};
  uint4 rawA[KeysB16::kRaw], rawB[KeysB16::kRaw];
  for (int u = 0; u < units; ++u) {
    fetch(min(u + 1, last_unit));
    // Keep the loads ahead of the scoring: left to itself the scheduler
    // sinks them to the put at the end of the iteration.
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t* base = lds[u & 1];
    read_tile(base, 0, rawA);
    read_tile(base, 1, rawB);
    // Step 0: tile 0's MFMAs; the previous unit's tile 3 reduced.
    tile_mfma<Tag, 4, KeysB16>(qa, rawA, acc0);
    sp[3] = tile_reduce<4>(wr, acc1);
    mfma_valu_interleave();
    store_unit(sp, u - 1);
    read_tile(base, 2, rawA);
    tile_mfma<Tag, 4, KeysB16>(qa, rawB, acc1);
    sp[0] = tile_reduce<4>(wr, acc0);
    mfma_valu_interleave();
    read_tile(base, 3, rawB);
    tile_mfma<Tag, 4, KeysB16>(qa, rawA, acc0);
    sp[1] = tile_reduce<4>(wr, acc1);
    mfma_valu_interleave();
    tile_mfma<Tag, 4, KeysB16>(qa, rawB, acc1);
    sp[2] = tile_reduce<4>(wr, acc0);
    mfma_valu_interleave();
    // Into the buffer scored last iteration; unconditional (past the last
    // unit it stages a re-read nobody scores), so that the iteration is one
    // basic block and no reduction is sunk below a branch, away from the
    // MFMAs it is interleaved with.
    put((u + 1) & 1);
    __syncthreads();
  }
  if (units > 0) {
    sp[3] = tile_reduce<4>(wr, acc1);
    store_unit(sp, units - 1);
  }
  // Keys past this workgroup's units are invisible to all of its queries.
  if (active)
    for (int key = units * 64 + lane; key < L; key += 64) orow[key] = -__builtin_inff();
  if constexpr (kTopK) {
    __shared__ __align__(16) uint32_t topk_scratch[kPrefillQueries][kTopKScratch];
    if (active) {
      // The row is read back by the wave that stored it, once its stores
      // have completed.
      __builtin_amdgcn_s_waitcnt(0);
      const int64_t at = seq * a.topk_stride;
      prefill_topk_row(orsrc, vis, L, a.topk, a.topk_idx + at, a.topk_val ? a.topk_val + at : nullptr,
                       topk_scratch[wave], lane);
    }
  }
}

// ---------------------------------------------------------------------------
// fp32 keys and queries (accuracy path): v_mfma_f32_16x16x4_f32, queries
// staged once per workgroup in LDS (rows padded to 129 floats), one 16-key
// tile per wave.  k-step j of lane group g uses dim 32 * g + j.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dense_scores_f32_kernel(const float* q_all,
                                                               const float* w_all,
                                                               const float* keys_all,
                                                               float* out_all, int L) {
  __shared__ float qs[kHeads][kHeadDim + 1];
  const int64_t b = blockIdx.y;
  const float* q = q_all + b * (kHeads * kHeadDim);
  for (int i = threadIdx.x; i < kHeads * kHeadDim; i += blockDim.x)
    qs[i / kHeadDim][i % kHeadDim] = q[i];
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int key0 = (blockIdx.x * 4 + wave) * 16;
  if (key0 >= L) return;
  const float* w = w_all + b * kHeads;
  const float* keys = keys_all + b * (int64_t)L * kHeadDim;
  const int key = min(key0 + r, L - 1);
  float kv[32];
  const float4* kp = reinterpret_cast<const float4*>(keys + (size_t)key * kHeadDim + 32 * g);
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const float4 v = kp[c];
    kv[4 * c + 0] = v.x;
    kv[4 * c + 1] = v.y;
    kv[4 * c + 2] = v.z;
    kv[4 * c + 3] = v.w;
  }
  float total = 0.f;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 32; ++j)
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qs[16 * m + r][32 * g + j], kv[j], acc, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) total = fmaf(w[16 * m + 4 * g + i], fmaxf(acc[i], 0.f), total);
  }
  total = reduce_lane_groups(total);
  if (g == 0 && key0 + r < L) out_all[b * (int64_t)L + key0 + r] = total;
}

// ---------------------------------------------------------------------------
// Block-granular kernels (one wave per decision block of 16 * T keys).
// ---------------------------------------------------------------------------
enum BlockMode { kModeH8 = 0, kModeMasked = 1, kModeProgressive = 2 };

struct BlockArgs {
  const uint16_t* q;
  const float* w;
  const uint8_t* keys;
  const float* scales;
  const int32_t* selected;
  const int32_t* remaining;
  const uint8_t* mask;  // cold (H8), keep (masked), direct (progressive)
  const float* threshold;
  float* out_scores;
  int32_t* out_indices;
  int8_t* accepted;
  float* block_max;
  int32_t* counter;
  int32_t length;
  int32_t compact;
};

// Sequence `seq` of a batched launch (grid.y = sequences of one length, all
// arrays packed per sequence): every pointer moves to that sequence's rows.
template <class KF>
__device__ __forceinline__ BlockArgs sequence_args(BlockArgs a, int64_t seq, int block_size) {
  if (seq == 0) return a;
  const int64_t L = a.length;
  const int64_t nb = (L + block_size - 1) / block_size;
  a.q += seq * kHeads * kHeadDim;
  a.w += seq * kHeads;
  a.keys += seq * L * KF::kRowBytes;
  if (a.scales) a.scales += seq * ((L + 127) / 128);
  if (a.selected) a.selected += seq * kVerifierHeads;
  if (a.remaining) a.remaining += seq * (kHeads - kVerifierHeads);
  a.mask += seq * nb;
  if (a.threshold) a.threshold += seq;
  a.out_scores += seq * L;
  if (a.out_indices) a.out_indices += seq * L;
  if (a.accepted) a.accepted += seq * nb;
  if (a.block_max) a.block_max += seq * nb;
  if (a.counter) a.counter += seq;
  return a;
}

template <class KF>
__device__ __forceinline__ float key_scale(const float* scales, int key) {
  if constexpr (KF::kScaled) return scales[key >> 7];
  return 1.f;
}

template <class Tag, class KF, int MODE, int T>
__global__ __launch_bounds__(256) void block_kernel(BlockArgs args) {
  const BlockArgs a = sequence_args<KF>(args, blockIdx.y, 16 * T);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int L = a.length;
  constexpr int kBlock = 16 * T;
  const int nb = (L + kBlock - 1) / kBlock;
  const int block = blockIdx.x * 4 + wave;
  if (block >= nb) return;
  const int start = block * kBlock;
  const float neg_inf = -__builtin_inff();
  const bool flag = a.mask[block] != 0;

  if constexpr (MODE == kModeMasked) {
    if (!flag) {
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int key = start + 16 * t + r;
        if (g == 0 && key < L) a.out_scores[key] = neg_inf;
      }
      return;
    }
    uint4 qa[4][4];
    float wr[4][4];
    load_head_tiles<4, KF::kNaturalK>(a.q, a.w, nullptr, kHeads, r, g, qa, wr);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      uint4 raw[KF::kRaw];
      const int key = start + 16 * t + r;
      KF::load(a.keys, min(key, L - 1), g, raw);
      float v = reduce_lane_groups(tile_contrib<Tag, 4, KF>(qa, wr, raw));
      if (g == 0 && key < L) a.out_scores[key] = v * key_scale<KF>(a.scales, key);
    }
  } else if constexpr (MODE == kModeH8) {
    if (!flag) {
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int key = start + 16 * t + r;
        if (g == 0 && key < L) a.out_scores[key] = neg_inf;
      }
      if (lane == 0) a.block_max[block] = neg_inf;
      return;
    }
    uint4 qa[1][4];
    float wr[1][4];
    load_head_tiles<1, KF::kNaturalK>(a.q, a.w, a.selected, kVerifierHeads, r, g, qa, wr);
    float maximum = neg_inf;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      uint4 raw[KF::kRaw];
      const int key = start + 16 * t + r;
      KF::load(a.keys, min(key, L - 1), g, raw);
      float v = reduce_lane_groups(tile_contrib<Tag, 1, KF>(qa, wr, raw));
      v = key < L ? v * key_scale<KF>(a.scales, key) : neg_inf;
      maximum = fmaxf(maximum, v);
      if (g == 0 && key < L) a.out_scores[key] = v;
    }
    maximum = wave_max(maximum);
    if (lane == 0) a.block_max[block] = maximum;
  } else {  // kModeProgressive
    uint4 qs[1][4];
    float ws[1][4];
    load_head_tiles<1, KF::kNaturalK>(a.q, a.w, a.selected, kVerifierHeads, r, g, qs, ws);
    uint4 raw[T][KF::kRaw];
    float p[T];
    float maximum = neg_inf;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int key = start + 16 * t + r;
      KF::load(a.keys, min(key, L - 1), g, raw[t]);
      p[t] = reduce_lane_groups(tile_contrib<Tag, 1, KF>(qs, ws, raw[t]));
      if (key < L) maximum = fmaxf(maximum, p[t] * key_scale<KF>(a.scales, key));
    }
    maximum = wave_max(maximum);
    const bool promote = !flag && maximum >= *a.threshold;
    const bool accept = flag || promote;
    if (accept) {
      uint4 qr[4][4];
      float wrr[4][4];
      load_head_tiles<4, KF::kNaturalK>(a.q, a.w, a.remaining, kHeads - kVerifierHeads, r, g, qr, wrr);
#pragma unroll
      for (int t = 0; t < T; ++t) p[t] += reduce_lane_groups(tile_contrib<Tag, 4, KF>(qr, wrr, raw[t]));
    }
    if (lane == 0) {
      a.accepted[block] = accept ? 1 : 0;
      a.block_max[block] = flag ? neg_inf : maximum;
    }
    if (!a.compact) {
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int key = start + 16 * t + r;
        if (g == 0 && key < L)
          a.out_scores[key] = accept ? p[t] * key_scale<KF>(a.scales, key) : neg_inf;
      }
    } else if (accept) {
      const int valid = min(kBlock, L - start);
      int slot = 0;
      if (lane == 0) slot = atomicAdd(a.counter, valid);
      slot = __shfl(slot, 0, kWave);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int offset = 16 * t + r;
        if (g == 0 && offset < valid) {
          a.out_scores[slot + offset] = p[t] * key_scale<KF>(a.scales, start + offset);
          a.out_indices[slot + offset] = start + offset;
        }
      }
    }
  }
}

__global__ void promote_blocks_kernel(const uint8_t* direct, const float* block_max,
                                      const float* threshold, uint8_t* accepted, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) accepted[i] = (direct[i] != 0 || block_max[i] >= *threshold) ? 1 : 0;
}

// ---------------------------------------------------------------------------
// Host-side launch helpers.
// ---------------------------------------------------------------------------
template <class Tag, class KF, int M, bool kGather, bool kHist = false, bool kLists = false>
int launch_dense_m(DenseArgs a, int64_t sequences, hipStream_t stream, hipEvent_t start = nullptr,
                   hipEvent_t stop = nullptr) {
  // Waves per workgroup of the decode step (histogram / candidate lists).
  // Eight (two per SIMD, twice the loads in flight per CU) measured slower
  // than four at C2.
  constexpr int kWaves = kHist ? kDecodeWaves : 4;
  const int64_t units = (a.length + 63) / 64;
  a.units_per_wg = dense_units_per_wg(sequences, a.length, 256, kWaves);
  a.wgs_per_seq = (int32_t)((units + a.units_per_wg - 1) / a.units_per_wg);
  a.total_wgs = sequences * a.wgs_per_seq;
  const int64_t grid = (a.total_wgs + kXcds - 1) / kXcds * kXcds;
  if (grid > 0x7fffffffLL) return fail(DSA_STATUS_INVALID_ARGUMENT, "problem too large");
  const size_t lds = kLists ? (size_t)a.units_per_wg * 64 * sizeof(float) : 0;
  launch_timed(dense_scores_kernel<Tag, KF, M, kGather, kHist, kLists, kWaves>, dim3((unsigned)grid), dim3(64 * kWaves),
               (uint32_t)lds, stream, start, stop, a);
  return check_launch("dense_scores_kernel");
}

template <class Tag, class KF>
int launch_dense(const DenseArgs& a, int64_t sequences, hipStream_t stream) {
  if constexpr (KF::kRowBytes == KeysB16::kRowBytes) {
    if (!a.head_ids && a.head_count == kHeads && a.queries_per_keyset >= kPrefillQueries) {
      const int64_t keysets = sequences / a.queries_per_keyset;
      const int64_t qblocks = (a.queries_per_keyset + kPrefillQueries - 1) / kPrefillQueries;
      if (keysets * a.queries_per_keyset == sequences && qblocks * keysets <= 0x7fffffffLL) {
        hipLaunchKernelGGL((prefill_scores_kernel<Tag, false>), dim3((unsigned)(qblocks * keysets)),
                           dim3(64 * kPrefillQueries), 0, stream, a, (int32_t)qblocks, (int32_t)keysets);
        return check_launch("prefill_scores_kernel");
      }
    }
  }
  if (!a.head_ids && a.head_count == kHeads) return launch_dense_m<Tag, KF, 4, false>(a, sequences, stream);
  switch ((a.head_count + 15) / 16) {
    case 1: return launch_dense_m<Tag, KF, 1, true>(a, sequences, stream);
    case 2: return launch_dense_m<Tag, KF, 2, true>(a, sequences, stream);
    case 3: return launch_dense_m<Tag, KF, 3, true>(a, sequences, stream);
    default: return launch_dense_m<Tag, KF, 4, true>(a, sequences, stream);
  }
}

template <class Tag, class KF, int MODE>
int launch_block(const BlockArgs& a, int block_size, hipStream_t stream, int64_t batch) {
  const int nb = (a.length + block_size - 1) / block_size;
  dim3 grid((unsigned)((nb + 3) / 4), (unsigned)batch);
  switch (block_size) {
    case 16: hipLaunchKernelGGL((block_kernel<Tag, KF, MODE, 1>), grid, dim3(256), 0, stream, a); break;
    case 32: hipLaunchKernelGGL((block_kernel<Tag, KF, MODE, 2>), grid, dim3(256), 0, stream, a); break;
    case 64: hipLaunchKernelGGL((block_kernel<Tag, KF, MODE, 4>), grid, dim3(256), 0, stream, a); break;
    default: hipLaunchKernelGGL((block_kernel<Tag, KF, MODE, 8>), grid, dim3(256), 0, stream, a); break;
  }
  return check_launch("block_kernel");
}

template <int MODE>
int dispatch_block(BlockArgs& a, int block_size, int dtype, hipStream_t stream, int64_t batch = 1) {
  switch (dtype) {
    case kBF16: return launch_block<Bf16Tag, KeysB16, MODE>(a, block_size, stream, batch);
    case kF16: return launch_block<F16Tag, KeysB16, MODE>(a, block_size, stream, batch);
    case kFP8E4M3: return launch_block<Bf16Tag, KeysFP8, MODE>(a, block_size, stream, batch);
    default:
      return fail(DSA_STATUS_INVALID_ARGUMENT, "block kernels take fp16/bf16/fp8 keys, got dtype %d",
                  dtype);
  }
}

int check_block_common(const void* q, const float* w, const void* keys, int64_t length,
                       int32_t block_size) {
  DSA_REQUIRE(q && w && keys, "queries, weights and keys must be non-null");
  DSA_REQUIRE(length > 0 && length < (int64_t(1) << 30), "length %lld out of range",
              (long long)length);
  DSA_REQUIRE(block_size == 16 || block_size == 32 || block_size == 64 || block_size == 128,
              "block_size must be 16, 32, 64 or 128 (got %d)", block_size);
  return DSA_STATUS_OK;
}

}  // namespace
}  // namespace dsa

using namespace dsa;

extern "C" int dsa_score_queries(const void* queries, int64_t q_stride, const float* weights,
                                 int64_t w_stride, const int32_t* head_ids, int64_t ids_stride,
                                 int32_t head_count, const void* keys, int64_t key_stride,
                                 int64_t queries_per_keyset, const float* key_scales,
                                 int64_t scale_stride, float* out, int64_t out_stride,
                                 int64_t sequences, int64_t length, int64_t causal_offset,
                                 int32_t key_dtype, void* stream) {
  DSA_REQUIRE(queries && weights && keys && out, "null pointer argument");
  DSA_REQUIRE(sequences > 0, "sequences must be positive");
  DSA_REQUIRE(length > 0 && length < (int64_t(1) << 30), "length %lld out of range",
              (long long)length);
  DSA_REQUIRE(head_count > 0 && head_count <= kHeads, "head_count %d outside [1, 64]", head_count);
  DSA_REQUIRE(queries_per_keyset > 0 && queries_per_keyset < (int64_t(1) << 31),
              "queries_per_keyset out of range");
  DSA_REQUIRE(causal_offset < (int64_t(1) << 30), "causal_offset out of range");
  DSA_REQUIRE(out_stride >= length, "out_stride < length");
  DSA_REQUIRE(reinterpret_cast<uintptr_t>(queries) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(keys) % 16 == 0,
              "queries and keys must be 16-byte aligned");
  DSA_REQUIRE(q_stride % 8 == 0, "q_stride must keep 16-byte alignment");
  DSA_REQUIRE(length * (key_dtype == kFP8E4M3 ? 128 : 256) < (int64_t(1) << 32),
              "one key set must stay below 4 GiB");
  DenseArgs a = {};
  a.q = static_cast<const uint16_t*>(queries);
  a.q_stride = q_stride;
  a.w = weights;
  a.w_stride = w_stride;
  a.head_ids = head_ids;
  a.ids_stride = ids_stride;
  a.head_count = head_count;
  a.keys = static_cast<const uint8_t*>(keys);
  a.key_stride = key_stride;
  a.queries_per_keyset = (int32_t)queries_per_keyset;
  a.scales = key_scales;
  a.scale_stride = scale_stride;
  a.out = out;
  a.out_stride = out_stride;
  a.length = (int32_t)length;
  a.causal_offset = causal_offset < 0 ? -1 : (int32_t)causal_offset;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (key_dtype) {
    case kBF16: return launch_dense<Bf16Tag, KeysB16>(a, sequences, s);
    case kF16: return launch_dense<F16Tag, KeysB16>(a, sequences, s);
    case kFP8E4M3:
      DSA_REQUIRE(key_scales, "fp8 keys need key_scales");
      return launch_dense<Bf16Tag, KeysFP8>(a, sequences, s);
    default:
      return fail(DSA_STATUS_INVALID_ARGUMENT, "dsa_score_queries takes fp16/bf16/fp8 keys (got %d)",
                  key_dtype);
  }
}

extern "C" int dsa_score_queries_topk(const void* queries, int64_t q_stride, const float* weights,
                                      int64_t w_stride, const void* keys, int64_t key_stride,
                                      int64_t queries_per_keyset, float* out, int64_t out_stride,
                                      int64_t sequences, int64_t length, int64_t causal_offset,
                                      int32_t key_dtype, int32_t k, int64_t* out_indices, float* out_values,
                                      int64_t topk_stride, void* stream) {
  DSA_REQUIRE(queries && weights && keys && out && out_indices, "null pointer argument");
  DSA_REQUIRE(key_dtype == kBF16 || key_dtype == kF16, "dsa_score_queries_topk takes fp16/bf16 keys (got %d)",
              key_dtype);
  DSA_REQUIRE(length > 0 && length <= kTopKRowMax, "length %lld outside [1, %d]", (long long)length,
              kTopKRowMax);
  DSA_REQUIRE(queries_per_keyset >= kPrefillQueries && queries_per_keyset < (int64_t(1) << 31),
              "queries_per_keyset %lld outside [%d, 2^31)", (long long)queries_per_keyset, kPrefillQueries);
  DSA_REQUIRE(sequences > 0 && sequences % queries_per_keyset == 0,
              "sequences must be a positive multiple of queries_per_keyset");
  DSA_REQUIRE(k > 0, "k must be positive (got %d)", k);
  DSA_REQUIRE(topk_stride >= k, "topk_stride < k");
  DSA_REQUIRE(causal_offset < (int64_t(1) << 30), "causal_offset out of range");
  DSA_REQUIRE(out_stride >= length, "out_stride < length");
  DSA_REQUIRE(reinterpret_cast<uintptr_t>(queries) % 16 == 0 && reinterpret_cast<uintptr_t>(keys) % 16 == 0,
              "queries and keys must be 16-byte aligned");
  DSA_REQUIRE(q_stride % 8 == 0, "q_stride must keep 16-byte alignment");
  const int64_t keysets = sequences / queries_per_keyset;
  const int64_t qblocks = (queries_per_keyset + kPrefillQueries - 1) / kPrefillQueries;
  DSA_REQUIRE(qblocks * keysets <= 0x7fffffffLL, "problem too large");
  DenseArgs a = {};
  a.q = static_cast<const uint16_t*>(queries);
  a.q_stride = q_stride;
  a.w = weights;
  a.w_stride = w_stride;
  a.head_count = kHeads;
  a.keys = static_cast<const uint8_t*>(keys);
  a.key_stride = key_stride;
  a.queries_per_keyset = (int32_t)queries_per_keyset;
  a.out = out;
  a.out_stride = out_stride;
  a.length = (int32_t)length;
  a.causal_offset = causal_offset < 0 ? -1 : (int32_t)causal_offset;
  a.topk = k;
  a.topk_idx = out_indices;
  a.topk_val = out_values;
  a.topk_stride = topk_stride;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)(qblocks * keysets));
  if (key_dtype == kBF16)
    hipLaunchKernelGGL((prefill_scores_kernel<Bf16Tag, true>), grid, dim3(64 * kPrefillQueries), 0, s, a,
                       (int32_t)qblocks, (int32_t)keysets);
  else
    hipLaunchKernelGGL((prefill_scores_kernel<F16Tag, true>), grid, dim3(64 * kPrefillQueries), 0, s, a,
                       (int32_t)qblocks, (int32_t)keysets);
  return check_launch("prefill_scores_kernel");
}

extern "C" int dsa_full_scores(const void* queries, const float* weights, const void* keys,
                               const float* key_scales, float* out, int64_t batch, int64_t length,
                               int32_t key_dtype, void* stream) {
  DSA_REQUIRE(queries && weights && keys && out, "null pointer argument");
  DSA_REQUIRE(batch > 0 && batch <= 65535, "batch %lld out of range", (long long)batch);
  DSA_REQUIRE(length > 0 && length < (int64_t(1) << 30), "length %lld out of range",
              (long long)length);
  if (key_dtype == kF32) {
    dim3 grid((unsigned)((length + 63) / 64), (unsigned)batch);
    hipLaunchKernelGGL(dense_scores_f32_kernel, grid, dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const float*>(queries),
                       weights, static_cast<const float*>(keys), out, (int)length);
    return check_launch("dense_scores_f32_kernel");
  }
  return dsa_score_queries(queries, kHeads * kHeadDim, weights, kHeads, nullptr, 0, kHeads, keys,
                           length, 1, key_scales, (length + 127) / 128, out, length, batch, length,
                           -1, key_dtype, stream);
}

extern "C" int64_t dsa_score_topk_workspace_bytes(int64_t batch, int64_t length) {
  if (batch <= 0 || length <= 0) return 0;
  return select_workspace_layout(nullptr, batch, length).bytes;
}

static int score_hist(const void* queries, const float* weights, const void* keys, const float* key_scales,
                      float* scores, int64_t batch, int64_t length, int64_t k, int32_t key_dtype, void* workspace,
                      int64_t workspace_bytes, void* stream, hipEvent_t start, hipEvent_t stop) {
  DSA_REQUIRE(queries && weights && keys && scores, "null pointer argument");
  DSA_REQUIRE(batch > 0 && batch <= 65535, "batch %lld out of range", (long long)batch);
  DSA_REQUIRE(length > 0 && length <= int64_t(kSelectChunk) * kMaxSelectChunks,
              "length %lld outside [1, %d]", (long long)length, kSelectChunk * kMaxSelectChunks);
  DSA_REQUIRE(k > 0 && k <= (int64_t(1) << 27), "k=%lld out of range", (long long)k);
  DSA_REQUIRE(key_dtype == kBF16 || key_dtype == kF16 || key_dtype == kFP8E4M3,
              "dsa_score_hist takes fp16/bf16/fp8 keys (got %d)", key_dtype);
  DSA_REQUIRE(key_dtype != kFP8E4M3 || key_scales, "fp8 keys need key_scales");
  DSA_REQUIRE(reinterpret_cast<uintptr_t>(queries) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(keys) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(workspace) % 256 == 0,
              "queries, keys (16 B) and workspace (256 B) must be aligned");
  const int64_t need = dsa_score_topk_workspace_bytes(batch, length);
  if (!workspace || workspace_bytes < need)
    return fail(DSA_STATUS_WORKSPACE_TOO_SMALL, "the decode step needs %lld workspace bytes",
                (long long)need);
  const SelectWorkspace ws = select_workspace_layout(workspace, batch, length);
  DenseArgs a = {};
  a.q = static_cast<const uint16_t*>(queries);
  a.q_stride = kHeads * kHeadDim;
  a.w = weights;
  a.w_stride = kHeads;
  a.head_count = kHeads;
  a.keys = static_cast<const uint8_t*>(keys);
  a.key_stride = length;
  a.queries_per_keyset = 1;
  a.scales = key_scales;
  a.scale_stride = (length + 127) / 128;
  a.out = scores;
  a.out_stride = length;
  a.length = (int32_t)length;
  a.causal_offset = -1;
  a.hist = ws.hist;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const ListPlan plan = list_plan(batch, length, k);
  if (plan.on) {
    // Each scoring workgroup writes its chunk's candidate list; the row
    // histogram stays untouched (and zero).
    a.lists = ws.cand;
    a.list_meta = ws.list_meta;
    a.list_quota = plan.quota;
    switch (key_dtype) {
      case kBF16: return launch_dense_m<Bf16Tag, KeysB16, 4, false, true, true>(a, batch, s, start, stop);
      case kF16: return launch_dense_m<F16Tag, KeysB16, 4, false, true, true>(a, batch, s, start, stop);
      default: return launch_dense_m<Bf16Tag, KeysFP8, 4, false, true, true>(a, batch, s, start, stop);
    }
  }
  switch (key_dtype) {
    case kBF16: return launch_dense_m<Bf16Tag, KeysB16, 4, false, true>(a, batch, s, start, stop);
    case kF16: return launch_dense_m<F16Tag, KeysB16, 4, false, true>(a, batch, s, start, stop);
    default: return launch_dense_m<Bf16Tag, KeysFP8, 4, false, true>(a, batch, s, start, stop);
  }
}

extern "C" int dsa_score_hist(const void* queries, const float* weights, const void* keys,
                              const float* key_scales, float* scores, int64_t batch,
                              int64_t length, int64_t k, int32_t key_dtype, void* workspace,
                              int64_t workspace_bytes, void* stream) {
  return score_hist(queries, weights, keys, key_scales, scores, batch, length, k, key_dtype, workspace,
                    workspace_bytes, stream, nullptr, nullptr);
}

extern "C" int dsa_score_hist_timed(const void* queries, const float* weights, const void* keys,
                                    const float* key_scales, float* scores, int64_t batch,
                                    int64_t length, int64_t k, int32_t key_dtype, void* workspace,
                                    int64_t workspace_bytes, void* stream, void* start_event,
                                    void* stop_event) {
  return score_hist(queries, weights, keys, key_scales, scores, batch, length, k, key_dtype, workspace,
                    workspace_bytes, stream, static_cast<hipEvent_t>(start_event),
                    static_cast<hipEvent_t>(stop_event));
}

extern "C" int dsa_score_topk(const void* queries, const float* weights, const void* keys,
                              const float* key_scales, float* scores, int64_t batch,
                              int64_t length, int64_t k, int32_t key_dtype, int64_t* out_indices,
                              float* out_values, void* workspace, int64_t workspace_bytes,
                              void* stream) {
  if (int st = dsa_score_hist(queries, weights, keys, key_scales, scores, batch, length, k, key_dtype,
                              workspace, workspace_bytes, stream))
    return st;
  return dsa_select_topk(scores, batch, length, k, out_indices, out_values, workspace,
                         workspace_bytes, stream);
}

extern "C" int dsa_h8_block_max(const void* queries, const float* weights, const void* keys,
                                const float* key_scales, const int32_t* selected_heads,
                                const uint8_t* cold_blocks, float* partial, float* block_max, int64_t length,
                                int32_t block_size, int32_t key_dtype, void* stream) {
  if (int st = check_block_common(queries, weights, keys, length, block_size)) return st;
  DSA_REQUIRE(selected_heads && cold_blocks && partial && block_max, "null pointer argument");
  DSA_REQUIRE(key_dtype != kFP8E4M3 || key_scales, "fp8 keys need key_scales");
  BlockArgs a = {};
  a.q = static_cast<const uint16_t*>(queries);
  a.w = weights;
  a.keys = static_cast<const uint8_t*>(keys);
  a.scales = key_scales;
  a.selected = selected_heads;
  a.mask = cold_blocks;
  a.out_scores = partial;
  a.block_max = block_max;
  a.length = (int32_t)length;
  return dispatch_block<kModeH8>(a, block_size, key_dtype, static_cast<hipStream_t>(stream));
}

extern "C" int dsa_masked_full_scores(const void* queries, const float* weights, const void* keys,
                                      const float* key_scales, const uint8_t* keep_blocks, float* out,
                                      int64_t length, int32_t block_size, int32_t key_dtype, void* stream) {
  if (int st = check_block_common(queries, weights, keys, length, block_size)) return st;
  DSA_REQUIRE(keep_blocks && out, "null pointer argument");
  DSA_REQUIRE(key_dtype != kFP8E4M3 || key_scales, "fp8 keys need key_scales");
  BlockArgs a = {};
  a.q = static_cast<const uint16_t*>(queries);
  a.w = weights;
  a.keys = static_cast<const uint8_t*>(keys);
  a.scales = key_scales;
  a.mask = keep_blocks;
  a.out_scores = out;
  a.length = (int32_t)length;
  return dispatch_block<kModeMasked>(a, block_size, key_dtype, static_cast<hipStream_t>(stream));
}

static int progressive_scores(const void* queries, const float* weights, const void* keys, const float* key_scales,
                              const int32_t* selected_heads, const int32_t* remaining_heads,
                              const uint8_t* direct_blocks, const float* threshold, float* out_scores,
                              int32_t* out_indices, int8_t* accepted, float* block_max, int32_t* counter,
                              int64_t batch, int64_t length, int32_t block_size, int32_t compact, int32_t key_dtype,
                              void* stream) {
  if (int st = check_block_common(queries, weights, keys, length, block_size)) return st;
  DSA_REQUIRE(batch > 0 && batch <= 65535, "batch %lld out of range", (long long)batch);
  DSA_REQUIRE(selected_heads && remaining_heads && direct_blocks && threshold && out_scores &&
                  accepted && block_max,
              "null pointer argument");
  DSA_REQUIRE(!compact || (out_indices && counter), "compact output needs indices and counter");
  DSA_REQUIRE(key_dtype != kFP8E4M3 || key_scales, "fp8 keys need key_scales");
  BlockArgs a = {};
  a.q = static_cast<const uint16_t*>(queries);
  a.w = weights;
  a.keys = static_cast<const uint8_t*>(keys);
  a.scales = key_scales;
  a.selected = selected_heads;
  a.remaining = remaining_heads;
  a.mask = direct_blocks;
  a.threshold = threshold;
  a.out_scores = out_scores;
  a.out_indices = out_indices;
  a.accepted = accepted;
  a.block_max = block_max;
  a.counter = counter;
  a.length = (int32_t)length;
  a.compact = compact ? 1 : 0;
  return dispatch_block<kModeProgressive>(a, block_size, key_dtype, static_cast<hipStream_t>(stream), batch);
}

extern "C" int dsa_progressive_scores(const void* queries, const float* weights, const void* keys,
                                      const float* key_scales, const int32_t* selected_heads,
                                      const int32_t* remaining_heads,
                                      const uint8_t* direct_blocks, const float* threshold,
                                      float* out_scores, int32_t* out_indices, int8_t* accepted,
                                      float* block_max, int32_t* counter, int64_t length,
                                      int32_t block_size, int32_t compact, int32_t key_dtype,
                                      void* stream) {
  return progressive_scores(queries, weights, keys, key_scales, selected_heads, remaining_heads, direct_blocks,
                            threshold, out_scores, out_indices, accepted, block_max, counter, 1, length, block_size,
                            compact, key_dtype, stream);
}

extern "C" int dsa_progressive_scores_batched(const void* queries, const float* weights, const void* keys,
                                              const float* key_scales, const int32_t* selected_heads,
                                              const int32_t* remaining_heads, const uint8_t* direct_blocks,
                                              const float* thresholds, float* out_scores, int32_t* out_indices,
                                              int8_t* accepted, float* block_max, int32_t* counters, int64_t batch,
                                              int64_t length, int32_t block_size, int32_t compact,
                                              int32_t key_dtype, void* stream) {
  return progressive_scores(queries, weights, keys, key_scales, selected_heads, remaining_heads, direct_blocks,
                            thresholds, out_scores, out_indices, accepted, block_max, counters, batch, length,
                            block_size, compact, key_dtype, stream);
}

extern "C" int dsa_promote_blocks(const uint8_t* direct_blocks, const float* block_max,
                                  const float* threshold, uint8_t* accepted, int64_t blocks,
                                  void* stream) {
  DSA_REQUIRE(direct_blocks && block_max && threshold && accepted, "null pointer argument");
  DSA_REQUIRE(blocks > 0, "blocks must be positive");
  const unsigned grid = (unsigned)((blocks + 255) / 256);
  hipLaunchKernelGGL(promote_blocks_kernel, dim3(grid), dim3(256), 0,
                     static_cast<hipStream_t>(stream), direct_blocks, block_max, threshold,
                     accepted, blocks);
  return check_launch("promote_blocks_kernel");
}

#ifdef DSA_PHASE_TRACE
// The decode scoring kernel's phase log (trace builds only): copies n
// entries to host memory, then zeroes the log if `clear`.
extern "C" int dsa_trace_dense_scores(uint64_t* host, int64_t n, int32_t clear) {
  DSA_REQUIRE(host && n >= 0 && n <= int64_t(kTraceWgs) * kTraceMarks, "bad trace read");
  if (int st = check_hip(hipMemcpyFromSymbol(host, HIP_SYMBOL(g_trace_dense), (size_t)n * 8), "trace read"))
    return st;
  if (clear) {
    static const uint64_t zeros[kTraceWgs * kTraceMarks] = {};
    return check_hip(hipMemcpyToSymbol(HIP_SYMBOL(g_trace_dense), zeros, sizeof(zeros)), "trace clear");
  }
  return DSA_STATUS_OK;
}
#endif
