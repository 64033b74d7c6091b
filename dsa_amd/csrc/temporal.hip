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
// Keys are scored with the tile code of the dense kernel (indexer.hpp), so
// an evaluated key's score equals the dense score bit for bit, and pruned
// blocks load no key bytes.
#include "common.hpp"
#include "dsa_amd.h"
#include "indexer.hpp"
#include "status.hpp"
#include "waveops.hpp"

#include <cmath>

namespace dsa {
namespace {

constexpr int kMaxTemporalBlocks = 2048;  // blocks per row (sorted in one workgroup)
constexpr int kMaxMerge = 8192;            // k + one wave's keys, merged in LDS
constexpr uint32_t kFarKey = 0x00ffffffu;  // a key index whose rows lie past every buffer
constexpr int kDigitBinsT = 2048;          // 11-bit radix digits of the threshold refresh

struct TemporalWorkspace {
  uint32_t* tau;        // [rows] ordered key of the threshold in force
  uint32_t* run;        // [rows][k] ordered keys of the k largest evaluated scores
  uint32_t* order;      // [rows][blocks] block ids in scan order
  double* upper;        // [rows][blocks] U_b, in double like the float64 reference
  uint32_t* seed_mask;  // [rows][ceil(L / 32)] keys evaluated as seeds
  int64_t bytes;
};

TemporalWorkspace temporal_layout(void* base, int64_t rows, int64_t length, int64_t k, int32_t block_size) {
  const int64_t blocks = (length + block_size - 1) / block_size;
  auto round = [](int64_t bytes) { return (bytes + 255) / 256 * 256; };
  const int64_t tau_off = 0;
  const int64_t run_off = tau_off + round(rows * 4);
  const int64_t order_off = run_off + round(rows * k * 4);
  const int64_t upper_off = order_off + round(rows * blocks * 4);
  const int64_t mask_off = upper_off + round(rows * blocks * 8);
  TemporalWorkspace ws;
  ws.bytes = mask_off + round(rows * ((length + 31) / 32) * 4);
  const uintptr_t p = reinterpret_cast<uintptr_t>(base);
  ws.tau = base ? reinterpret_cast<uint32_t*>(p + tau_off) : nullptr;
  ws.run = base ? reinterpret_cast<uint32_t*>(p + run_off) : nullptr;
  ws.order = base ? reinterpret_cast<uint32_t*>(p + order_off) : nullptr;
  ws.upper = base ? reinterpret_cast<double*>(p + upper_off) : nullptr;
  ws.seed_mask = base ? reinterpret_cast<uint32_t*>(p + mask_off) : nullptr;
  return ws;
}

struct TemporalArgs {
  const uint16_t* q;      // [rows][64][128]
  const float* w;         // [rows][64]
  const uint8_t* keys;    // [rows][length] key rows
  const float* scales;    // fp8: [rows][ceil(length / 128)]
  const float* prev_max;  // [rows][prev_blocks]
  const int64_t* seeds;   // [rows][k]
  const float* gamma;     // [rows]
  float* scores;          // [rows][length]
  uint8_t* evaluated;     // [rows][blocks]
  int32_t* qk_scored;     // [rows]
  int32_t rows, length, k, block_size, blocks, prev_length, prev_blocks;
  int32_t scan_order;     // 0 address, 1 previous-hot, 2 upper
  int32_t wave_start, wave_len;
  TemporalWorkspace ws;
};

// Bounds, scan order and a clean slate for one row (one workgroup per row).
__global__ __launch_bounds__(1024) void temporal_prep_kernel(TemporalArgs a) {
  __shared__ uint64_t sort_keys[kMaxTemporalBlocks];
  __shared__ uint8_t hot[kMaxTemporalBlocks];
  const int tid = threadIdx.x;
  const int row = blockIdx.x;
  const int L = a.length;
  const int nb = a.blocks;
  float* srow = a.scores + (size_t)row * L;
  for (int i = tid; i < L; i += 1024) srow[i] = -__builtin_inff();
  const int words = (L + 31) / 32;
  for (int i = tid; i < words; i += 1024) a.ws.seed_mask[(size_t)row * words + i] = 0;
  for (int i = tid; i < nb; i += 1024) a.evaluated[(size_t)row * nb + i] = 0;
  if (tid == 0) a.ws.tau[row] = 0xffffffffu;
  const int first_new = a.prev_length / a.block_size;
  const bool grown = a.prev_length < L;
  const double gamma = (double)a.gamma[row];
  for (int b = tid; b < nb; b += 1024) {
    const bool fresh = grown && b >= first_new;
    const float pm = b < a.prev_blocks ? a.prev_max[(size_t)row * a.prev_blocks + b] : -__builtin_inff();
    a.ws.upper[(size_t)row * nb + b] = fresh ? HUGE_VAL : (double)pm + gamma;
  }
  if (a.scan_order == 0) {
    for (int b = tid; b < nb; b += 1024) a.ws.order[(size_t)row * nb + b] = b;
    return;
  }
  for (int b = tid; b < nb; b += 1024) hot[b] = 0;
  __syncthreads();
  if (a.scan_order == 1) {
    for (int i = tid; i < a.k; i += 1024) {
      const int64_t key = a.seeds[(size_t)row * a.k + i];
      if (key >= 0 && key < L) hot[min((int)(key / a.block_size), nb - 1)] = 1;
    }
  }
  __syncthreads();
  // Descending sort of (hot, U, -address).  For a fixed gamma, U orders the
  // blocks as the previous block maxima do, so the 32-bit ordered key of the
  // maximum (+inf for blocks with new keys) stands for U.
  int n = 1;
  while (n < nb) n <<= 1;
  for (int b = tid; b < n; b += 1024) {
    uint64_t key = 0;
    if (b < nb) {
      const bool fresh = grown && b >= first_new;
      const float pm = b < a.prev_blocks ? a.prev_max[(size_t)row * a.prev_blocks + b] : -__builtin_inff();
      key = (uint64_t(hot[b]) << 63) | (uint64_t(float_to_ordered(fresh ? __builtin_inff() : pm)) << 31) |
            (uint64_t)(~(uint32_t)b & 0x7fffffffu);
    }
    sort_keys[b] = key;
  }
  __syncthreads();
  for (int size = 2; size <= n; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = tid; i < n; i += 1024) {
        const int j = i ^ stride;
        if (j > i) {
          const uint64_t x = sort_keys[i];
          const uint64_t y = sort_keys[j];
          const bool descending = (i & size) == 0;
          if (descending ? x < y : x > y) {
            sort_keys[i] = y;
            sort_keys[j] = x;
          }
        }
      }
      __syncthreads();
    }
  }
  for (int p = tid; p < nb; p += 1024)
    a.ws.order[(size_t)row * nb + p] = ~(uint32_t)sort_keys[p] & 0x7fffffffu;
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
  const BufferRsrc keys = make_buffer(a.keys + (size_t)row * a.length * KF::kRowBytes,
                                      (uint32_t)a.length * KF::kRowBytes);
  uint4 buf[4][KF::kRaw];
#pragma unroll
  for (int t = 0; t < 4; ++t) KF::load_buf(keys, tile_key[t], g, buf[t]);
  float s[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) s[t] = tile_contrib<Tag, 4, KF>(qa, wr, buf[t]);
  return unit_reduce(s, g);
}

// The seeds: 64 per wave, gathered by index.
template <class Tag, class KF>
__global__ __launch_bounds__(256) void temporal_seed_kernel(TemporalArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15;
  const int g = lane >> 4;
  const int per_row = (a.k + 255) / 256;
  const int row = blockIdx.x / per_row;
  const int base = (blockIdx.x % per_row) * 256 + wave * 64;
  if (base >= a.k) return;
  const int64_t* seeds = a.seeds + (size_t)row * a.k;
  int tile_key[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int i = base + 16 * t + r;
    const int64_t key = i < a.k ? seeds[i] : -1;
    tile_key[t] = (key >= 0 && key < a.length) ? (int)key : (int)kFarKey;
  }
  float v = score_unit<Tag, KF>(a, row, tile_key, r, g);
  const int i = base + lane;
  if (i >= a.k) return;
  const int64_t key = seeds[i];
  if (key < 0 || key >= a.length) {
    a.ws.run[(size_t)row * a.k + i] = 0;  // below every score
    return;
  }
  if constexpr (KF::kScaled) v *= a.scales[(size_t)row * ((a.length + 127) / 128) + (key >> 7)];
  a.scores[(size_t)row * a.length + key] = v;
  const int words = (a.length + 31) / 32;
  __hip_atomic_fetch_or(a.ws.seed_mask + (size_t)row * words + (key >> 5), 1u << (key & 31), __ATOMIC_RELAXED,
                        __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t ord = float_to_ordered(v);
  a.ws.run[(size_t)row * a.k + i] = ord;
  __hip_atomic_fetch_min(a.ws.tau + row, ord, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
    float v = score_unit<Tag, KF>(a, row, tile_key, r, g);
    const int key = u * 64 + lane;
    if (key >= first && key < end) {
      if constexpr (KF::kScaled) v *= a.scales[(size_t)row * ((a.length + 127) / 128) + (key >> 7)];
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

// Keys scored: the seeds plus every key of a kept block (each counted once).
__global__ __launch_bounds__(256) void temporal_count_kernel(TemporalArgs a) {
  __shared__ __align__(16) uint32_t wsum[4];
  const int tid = threadIdx.x;
  const int row = blockIdx.x;
  const int words = (a.length + 31) / 32;
  const int bs = a.block_size;
  uint32_t count = 0;
  for (int wd = tid; wd < words; wd += 256) {
    uint32_t bits = a.ws.seed_mask[(size_t)row * words + wd];
    for (int sub = 0; sub < 32; sub += 16) {  // blocks are multiples of 16 keys
      const int blk = (wd * 32 + sub) / bs;
      if (blk < a.blocks && a.evaluated[(size_t)row * a.blocks + blk]) bits |= 0xffffu << sub;
    }
    const int valid = min(32, a.length - wd * 32);
    if (valid < 32) bits &= (1u << valid) - 1u;
    count += __popc(bits);
  }
  uint32_t total;
  block_excl_scan<4>(count, wsum, total);
  if (tid == 0) a.qk_scored[row] = (int32_t)total;
}

template <class Tag, class KF>
int launch_temporal(TemporalArgs a, int32_t wave, int64_t* out_topk, hipStream_t stream) {
  hipLaunchKernelGGL(temporal_prep_kernel, dim3(a.rows), dim3(1024), 0, stream, a);
  if (int st = check_launch("temporal_prep_kernel")) return st;
  hipLaunchKernelGGL((temporal_seed_kernel<Tag, KF>), dim3(a.rows * ((a.k + 255) / 256)), dim3(256), 0, stream, a);
  if (int st = check_launch("temporal_seed_kernel")) return st;
  const int step = wave > 0 ? wave : a.blocks;
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
  hipLaunchKernelGGL(temporal_count_kernel, dim3(a.rows), dim3(256), 0, stream, a);
  if (int st = check_launch("temporal_count_kernel")) return st;
  return dsa_topk(a.scores, nullptr, a.rows, a.length, a.length, nullptr, a.k, 0, out_topk, nullptr, stream);
}

}  // namespace
}  // namespace dsa

using namespace dsa;

extern "C" int64_t dsa_temporal_workspace_bytes(int64_t batch, int64_t length, int64_t k, int32_t block_size) {
  if (batch <= 0 || length <= 0 || k <= 0 || block_size <= 0) return 0;
  return temporal_layout(nullptr, batch, length, k, block_size).bytes;
}

extern "C" int dsa_temporal_step(const void* queries, const float* weights, const void* keys,
                                 const float* key_scales, const float* prev_block_max, int64_t prev_length,
                                 const int64_t* prev_topk, const float* gamma, float* scores,
                                 uint8_t* evaluated_blocks, int64_t* out_topk, int32_t* qk_scored,
                                 int64_t batch, int64_t length, int64_t k, int32_t block_size,
                                 int32_t scan_order, int32_t wave, int32_t key_dtype, void* workspace,
                                 int64_t workspace_bytes, void* stream) {
  DSA_REQUIRE(queries && weights && keys && prev_block_max && prev_topk && gamma && scores && evaluated_blocks &&
                  out_topk && qk_scored,
              "null pointer argument");
  DSA_REQUIRE(batch > 0 && batch <= 65535, "batch %lld out of range", (long long)batch);
  DSA_REQUIRE(block_size == 16 || block_size == 32 || block_size == 64 || block_size == 128,
              "block_size %d not in {16, 32, 64, 128}", block_size);
  DSA_REQUIRE(length > 0 && length <= 32768, "length %lld outside [1, 32768]", (long long)length);
  DSA_REQUIRE(prev_length > 0 && prev_length <= length, "prev_length %lld outside [1, length]",
              (long long)prev_length);
  DSA_REQUIRE(k > 0 && k <= 4096 && k <= prev_length, "k=%lld must be in [1, min(4096, prev_length)]",
              (long long)k);
  DSA_REQUIRE(scan_order >= 0 && scan_order <= 2, "scan_order %d not in {0, 1, 2}", scan_order);
  DSA_REQUIRE(wave >= 0, "wave must be >= 0");
  DSA_REQUIRE(k + int64_t(wave) * block_size <= kMaxMerge, "k + wave * block_size exceeds %d", kMaxMerge);
  DSA_REQUIRE(key_dtype == DSA_DTYPE_BF16 || key_dtype == DSA_DTYPE_F16 || key_dtype == DSA_DTYPE_FP8_E4M3,
              "dsa_temporal_step takes fp16/bf16/fp8 keys (got %d)", key_dtype);
  DSA_REQUIRE(key_dtype != DSA_DTYPE_FP8_E4M3 || key_scales, "fp8 keys need key_scales");
  DSA_REQUIRE(reinterpret_cast<uintptr_t>(queries) % 16 == 0 && reinterpret_cast<uintptr_t>(keys) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(workspace) % 256 == 0,
              "queries, keys (16 B) and workspace (256 B) must be aligned");
  const int64_t blocks = (length + block_size - 1) / block_size;
  DSA_REQUIRE(blocks <= kMaxTemporalBlocks, "%lld blocks exceed %d", (long long)blocks, kMaxTemporalBlocks);
  const TemporalWorkspace ws = temporal_layout(workspace, batch, length, k, block_size);
  if (!workspace || workspace_bytes < ws.bytes)
    return fail(DSA_STATUS_WORKSPACE_TOO_SMALL, "the temporal step needs %lld workspace bytes", (long long)ws.bytes);
  TemporalArgs a = {};
  a.q = static_cast<const uint16_t*>(queries);
  a.w = weights;
  a.keys = static_cast<const uint8_t*>(keys);
  a.scales = key_scales;
  a.prev_max = prev_block_max;
  a.seeds = prev_topk;
  a.gamma = gamma;
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
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (key_dtype) {
    case DSA_DTYPE_BF16: return launch_temporal<Bf16Tag, KeysB16>(a, wave, out_topk, s);
    case DSA_DTYPE_F16: return launch_temporal<F16Tag, KeysB16>(a, wave, out_topk, s);
    default: return launch_temporal<Bf16Tag, KeysFP8>(a, wave, out_topk, s);
  }
}
