// Two-path verifier step and the dimension-sketch kernels.
//
// A verifier step (reference verifier.py:173-392) is an own-trajectory
// temporal step (temporal.hip) followed by a current-query check of every
// key the temporal scan left unscored ("cold" keys):
//   1. the temporal block scan: seeds, risk-bounded blocks (scores of the
//      evaluated keys, -inf elsewhere);
//   2. the verifier scan: a cheap score of every cold key, either the
//      head path (selected heads, full 128 dims, read from the key rows) or
//      the dim path (all 64 heads over a few rotated, optionally quantized
//      dims, read from a per-key sketch of `width` bytes or bf16 values);
//      per block, the largest cold verifier score and the cold-key count;
//   3. the rescue ranking, one workgroup per row: cold blocks sorted by
//      larger verifier score, then lower block id; the first
//      min(cold, ceil(rescue_fraction * cold)) blocks are rescued, or every
//      cold block at or above a fixed promotion threshold;
//   4. the rescued blocks' cold keys are scored in full (the dense kernel's
//      unit code, so the scores equal the dense scores bit for bit);
//   5. the stable top-k of every scored key (the candidate union), and the
//      policy-state update of refreshed and rescued blocks, with the cold
//      streak restarted from the final top-k.
// Only rescued blocks' keys beyond the temporal scan's are read in full, and
// the dim path reads `width` bytes per cold key instead of 256.
//
// The sketch of a row x of D (<= 128, a power of two) elements: the
// normalized Walsh-Hadamard transform (reference verifier_scoring.py:9-26;
// butterfly stages left + right, left - right at strides 1, 2, .., D/2, each
// sum rounded to the row dtype, then one multiply by D^-0.5 rounded to the
// dtype), the chosen dims, and optional symmetric fake quantization
// (verifier_scoring.py:29-41): code = clamp(rint(v / scale), +-limit),
// value = code * scale rounded to the dtype.  One wave per row: lane l holds
// elements l and l + 64; strides below 64 are lane shuffles.
#include "temporal.hpp"

#include "status.hpp"

namespace dsa {
namespace {

constexpr int kCountFields = 4;  // cold tokens, cold blocks, rescued blocks, rescued cold tokens

__device__ __forceinline__ float round_bf16_rn(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return x;
  u += 0x7fffu + ((u >> 16) & 1u);
  return __uint_as_float(u & 0xffff0000u);
}

// Rounds a float to the row dtype (DSA_DTYPE_*), as a float.
template <int kDtype>
__device__ __forceinline__ float round_to(float x) {
  if constexpr (kDtype == DSA_DTYPE_BF16) return round_bf16_rn(x);
  if constexpr (kDtype == DSA_DTYPE_F16) return (float)(_Float16)x;
  return x;
}

template <int kDtype>
__device__ __forceinline__ float load_as_float(const void* p, int64_t i) {
  if constexpr (kDtype == DSA_DTYPE_BF16) return __uint_as_float(uint32_t(static_cast<const uint16_t*>(p)[i]) << 16);
  if constexpr (kDtype == DSA_DTYPE_F16) return (float)static_cast<const _Float16*>(p)[i];
  return static_cast<const float*>(p)[i];
}

template <int kDtype>
__device__ __forceinline__ void store_from_float(void* p, int64_t i, float v) {  // v already in the dtype's grid
  if constexpr (kDtype == DSA_DTYPE_BF16)
    static_cast<uint16_t*>(p)[i] = (uint16_t)(__float_as_uint(v) >> 16);
  else if constexpr (kDtype == DSA_DTYPE_F16)
    static_cast<_Float16*>(p)[i] = (_Float16)v;
  else
    static_cast<float*>(p)[i] = v;
}

struct SketchArgs {
  const void* x;        // [rows][dim]
  const int32_t* dims;  // [width] kept dims (null: dims 0 .. width-1)
  void* out;            // [rows][width]: int8 codes or dtype values
  int64_t rows;
  int32_t dim, width, rotate, limit;  // limit 0: no quantization
  int32_t out_codes;
  float scale;                        // quantization scale (float32, as torch divides by it)
  float norm;                         // D^-0.5 as a float32 scalar
};

// One wave per row (four rows per workgroup).
template <int kDtype>
__global__ __launch_bounds__(256) void sketch_kernel(SketchArgs a) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const int D = a.dim;
  const int64_t base = row * D;
  float x0 = lane < D ? load_as_float<kDtype>(a.x, base + lane) : 0.f;
  float x1 = lane + 64 < D ? load_as_float<kDtype>(a.x, base + lane + 64) : 0.f;
  if (a.rotate) {
    for (int s = 1; s < D && s < 64; s <<= 1) {
      const float p0 = __shfl_xor(x0, s, kWave);
      const float p1 = __shfl_xor(x1, s, kWave);
      const bool upper = lane & s;  // element index has bit s set: left - right with left = partner
      x0 = round_to<kDtype>(upper ? p0 - x0 : x0 + p0);
      x1 = round_to<kDtype>(upper ? p1 - x1 : x1 + p1);
    }
    if (D == 128) {
      const float l = x0, r = x1;
      x0 = round_to<kDtype>(l + r);
      x1 = round_to<kDtype>(l - r);
    }
    x0 = round_to<kDtype>(x0 * a.norm);
    x1 = round_to<kDtype>(x1 * a.norm);
  }
  // Output slot d = 64 * pass + lane takes element dims[d]; every lane joins
  // every shuffle (a shuffle reads only lanes that execute it).
  for (int pass = 0; pass * 64 < a.width; ++pass) {
    const int d = pass * 64 + lane;
    const bool live = d < a.width;
    const int e = live ? (a.dims ? a.dims[d] : d) : 0;
    const float lo = __shfl(x0, e & 63, kWave);
    const float hi = __shfl(x1, e & 63, kWave);
    if (!live) continue;
    float v = e < 64 ? lo : hi;
    const int64_t at = row * a.width + d;
    if (a.limit > 0) {
      const float code = fminf(fmaxf(rintf(__fdiv_rn(v, a.scale)), (float)-a.limit), (float)a.limit);
      if (a.out_codes) {
        static_cast<int8_t*>(a.out)[at] = (int8_t)code;
        continue;
      }
      v = round_to<kDtype>(code * a.scale);
    }
    store_from_float<kDtype>(a.out, at, v);
  }
}

// Largest |x| of n values (float bits of non-negative values order as uints).
template <int kDtype>
__global__ __launch_bounds__(256) void abs_max_kernel(const void* x, int64_t n, uint32_t* out) {
  float m = 0.f;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    m = fmaxf(m, fabsf(load_as_float<kDtype>(x, i)));
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) atomicMax(out, __float_as_uint(m));
}

__global__ void zero_u32_kernel(uint32_t* p) { *p = 0u; }

// Elementwise symmetric fake quantization of n values.
template <int kDtype>
__global__ __launch_bounds__(256) void fake_quantize_kernel(const void* x, int64_t n, float scale, int32_t limit,
                                                            void* values, int8_t* codes) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float code = fminf(fmaxf(rintf(__fdiv_rn(load_as_float<kDtype>(x, i), scale)), (float)-limit), (float)limit);
  if (codes) codes[i] = (int8_t)code;
  if (values) store_from_float<kDtype>(values, i, round_to<kDtype>(code * scale));
}

// ---------------------------------------------------------------------------
// Sketch scoring: all 64 heads against `width` sketch dims.  Lane (r, g) of a
// 16-key tile supplies, for k-step j, dims 32j + 8g .. +8 of key r (zero past
// width); the query sketch's A fragments use the same dims.
// ---------------------------------------------------------------------------
struct SketchKeys {
  const uint8_t* base;  // [keys][width] int8 codes, or [keys][width] bf16 values
  int32_t width;
  int32_t codes;
  float scale;
};

__device__ __forceinline__ uint4 sketch_fragment(const SketchKeys& s, int key, int g, int j) {
  const int d = 32 * j + 8 * g;
  if (d >= s.width) return make_uint4(0u, 0u, 0u, 0u);
  if (!s.codes) return *reinterpret_cast<const uint4*>(s.base + ((size_t)key * s.width + d) * 2);
  const uint2 c = *reinterpret_cast<const uint2*>(s.base + (size_t)key * s.width + d);
  uint32_t out[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const uint32_t word = p < 2 ? c.x : c.y;
    const int sh = (p & 1) * 16;
    const float lo = round_bf16_rn((float)(int8_t)((word >> sh) & 0xffu) * s.scale);
    const float hi = round_bf16_rn((float)(int8_t)((word >> (sh + 8)) & 0xffu) * s.scale);
    out[p] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);
  }
  return make_uint4(out[0], out[1], out[2], out[3]);
}

// A fragments of the 64-head query sketch [64][width] (bf16), and weights.
template <int J>
__device__ __forceinline__ void load_sketch_queries(const uint16_t* q, const float* w, int width, int heads, int r,
                                                    int g, uint4 (&qa)[4][J], float (&wr)[4][4]) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int head = 16 * m + r;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int d = 32 * j + 8 * g;
      qa[m][j] = (head < heads && d < width) ? *reinterpret_cast<const uint4*>(q + (size_t)head * width + d)
                                             : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 16 * m + 4 * g + i;
      wr[m][i] = h < heads ? w[h] : 0.f;
    }
  }
}

template <int J>
__device__ __forceinline__ float sketch_tile_score(const uint4 (&qa)[4][J], const float (&wr)[4][4],
                                                   const SketchKeys& s, int key, int g) {
  floatx4 acc[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) acc[m] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const uint4 kb = sketch_fragment(s, key, g, j);
#pragma unroll
    for (int m = 0; m < 4; ++m) acc[m] = mfma_16x16x32(Bf16Tag{}, qa[m][j], kb, acc[m]);
  }
  return reduce_lane_groups(tile_reduce<4>(wr, acc));
}

// Dense sketch scores out[q][key] for Q queries (score_dim_sparse): grid
// (Q, ceil(K / 64)), one 16-key tile per wave.
template <int J>
__global__ __launch_bounds__(256) void sketch_scores_kernel(const uint16_t* qs, const float* w, int heads,
                                                            SketchKeys s, float* out, int64_t keys) {
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int64_t q = blockIdx.y;
  const int64_t key0 = (int64_t)blockIdx.x * 64 + (threadIdx.x >> 6) * 16;
  if (key0 >= keys) return;
  uint4 qa[4][J];
  float wr[4][4];
  load_sketch_queries<J>(qs + q * heads * s.width, w + q * heads, s.width, heads, r, g, qa, wr);
  const int64_t key = min(key0 + r, keys - 1);
  const float v = sketch_tile_score<J>(qa, wr, s, (int)key, g);
  if (g == 0 && key0 + r < keys) out[q * keys + key0 + r] = v;
}

// ---------------------------------------------------------------------------
// The verifier step.
// ---------------------------------------------------------------------------
struct VerifierArgs {
  const int32_t* head_ids;  // head path: [width] or [rows][id_stride]
  int64_t id_stride;
  int32_t width;
  const uint16_t* q_sketch;   // dim path: [rows][64][width] bf16
  const uint8_t* key_sketch;  // dim path: [rows][sketch_stride][width] codes or bf16 values
  int64_t sketch_stride;
  int32_t sketch_codes;
  float sketch_scale;
  float* verifier_scores;  // [rows][length] or null
  float* block_scores;     // [rows][blocks]
  uint8_t* cold_count;     // [rows][blocks] cold keys per block (0 .. 128)
  uint8_t* rescued;        // [rows][blocks]
  int32_t* ranking;        // [rows][blocks] or null
  int32_t* counts;         // [rows][kCountFields]
  int32_t promotion;       // 0: global budget, 1: fixed threshold
  double fraction;
  float threshold;
  const float* vsource;    // [rows][vsource_stride] or null: recorded verifier scores (trace replay)
  int64_t vsource_stride;
};

// Cold keys of a block: count, and whether key `key` is cold.
__device__ __forceinline__ bool is_cold(const float* srow, int key, int end) {
  return key < end && srow[key] == -__builtin_inff();
}

__device__ __forceinline__ int block_cold_count(const float* srow, int first, int end, int lane) {
  int n = 0;
  for (int key = first + lane; key - lane < end; key += 64) n += __popcll(__ballot(is_cold(srow, key, end)));
  return n;
}

// Writes a block without cold keys: no verifier score, count 0.
__device__ __forceinline__ void finish_warm_block(const TemporalArgs& a, const VerifierArgs& v, int row, int blk,
                                                  int first, int end, int lane) {
  if (v.verifier_scores)
    for (int key = first + lane; key < end; key += 64) v.verifier_scores[(size_t)row * a.length + key] = -__builtin_inff();
  if (lane == 0) {
    v.block_scores[(size_t)row * a.blocks + blk] = -__builtin_inff();
    v.cold_count[(size_t)row * a.blocks + blk] = 0;
  }
}

// Head path: one wave per block; selected heads (M tiles of 16) over the full
// key rows of blocks that hold cold keys.
template <class Tag, class KF, int M>
__global__ __launch_bounds__(256) void verifier_head_scan_kernel(TemporalArgs a, VerifierArgs v) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15;
  const int g = lane >> 4;
  const int per_row = (a.blocks + 3) / 4;
  const int row = blockIdx.x / per_row;
  const int blk = (blockIdx.x % per_row) * 4 + wave;
  if (blk >= a.blocks) return;
  const int first = blk * a.block_size;
  const int end = min(a.length, first + a.block_size);
  const float* srow = a.scores + (size_t)row * a.length;
  const int cold = block_cold_count(srow, first, end, lane);
  if (cold == 0) {
    finish_warm_block(a, v, row, blk, first, end, lane);
    return;
  }
  uint4 qa[M][4];
  float wr[M][4];
  const int32_t* ids = v.head_ids + (size_t)row * v.id_stride;
  load_head_tiles<M, KF::kNaturalK>(a.q + (size_t)row * kHeads * kHeadDim, a.w + (size_t)row * kHeads, ids, v.width,
                                    r, g, qa, wr);
  const BufferRsrc keys = make_buffer(a.keys + (size_t)row * a.key_stride * KF::kRowBytes,
                                      (uint32_t)a.length * KF::kRowBytes);
  float best = -__builtin_inff();
  for (int tile = first; tile < end; tile += 16) {
    const int key = tile + r;
    uint4 raw[KF::kRaw];
    KF::load_buf(keys, key, g, raw);  // past the row: zeros (range-checked)
    float s = reduce_lane_groups(tile_contrib<Tag, M, KF>(qa, wr, raw));
    if constexpr (KF::kScaled)
      s *= a.scales[(size_t)row * ((a.key_stride + 127) / 128) + (min(key, a.length - 1) >> 7)];
    const float out = is_cold(srow, key, end) ? s : -__builtin_inff();
    best = fmaxf(best, out);
    if (g == 0 && key < end && v.verifier_scores) v.verifier_scores[(size_t)row * a.length + key] = out;
  }
  best = wave_max(best);
  if (lane == 0) {
    v.block_scores[(size_t)row * a.blocks + blk] = best;
    v.cold_count[(size_t)row * a.blocks + blk] = (uint8_t)cold;
  }
}

// Dim path: one wave per block; all heads over the key sketch.
template <int J>
__global__ __launch_bounds__(256) void verifier_dim_scan_kernel(TemporalArgs a, VerifierArgs v) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15;
  const int g = lane >> 4;
  const int per_row = (a.blocks + 3) / 4;
  const int row = blockIdx.x / per_row;
  const int blk = (blockIdx.x % per_row) * 4 + wave;
  if (blk >= a.blocks) return;
  const int first = blk * a.block_size;
  const int end = min(a.length, first + a.block_size);
  const float* srow = a.scores + (size_t)row * a.length;
  const int cold = block_cold_count(srow, first, end, lane);
  if (cold == 0) {
    finish_warm_block(a, v, row, blk, first, end, lane);
    return;
  }
  uint4 qa[4][J];
  float wr[4][4];
  load_sketch_queries<J>(v.q_sketch + (size_t)row * kHeads * v.width, a.w + (size_t)row * kHeads, v.width, kHeads,
                         r, g, qa, wr);
  SketchKeys s;
  s.width = v.width;
  s.codes = v.sketch_codes;
  s.scale = v.sketch_scale;
  s.base = v.key_sketch + (size_t)row * v.sketch_stride * v.width * (v.sketch_codes ? 1 : 2);
  float best = -__builtin_inff();
  for (int tile = first; tile < end; tile += 16) {
    const int key = tile + r;
    const float sc = sketch_tile_score<J>(qa, wr, s, min(key, end - 1), g);
    const float out = is_cold(srow, key, end) ? sc : -__builtin_inff();
    best = fmaxf(best, out);
    if (g == 0 && key < end && v.verifier_scores) v.verifier_scores[(size_t)row * a.length + key] = out;
  }
  best = wave_max(best);
  if (lane == 0) {
    v.block_scores[(size_t)row * a.blocks + blk] = best;
    v.cold_count[(size_t)row * a.blocks + blk] = (uint8_t)cold;
  }
}

// Recorded verifier scores (trace replay): one wave per block takes the
// cold keys' scores from the recorded row instead of scoring them.
__global__ __launch_bounds__(256) void verifier_source_scan_kernel(TemporalArgs a, VerifierArgs v) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int per_row = (a.blocks + 3) / 4;
  const int row = blockIdx.x / per_row;
  const int blk = (blockIdx.x % per_row) * 4 + wave;
  if (blk >= a.blocks) return;
  const int first = blk * a.block_size;
  const int end = min(a.length, first + a.block_size);
  const float* srow = a.scores + (size_t)row * a.length;
  const float* vrow = v.vsource + (size_t)row * v.vsource_stride;
  int cold = 0;
  float best = -__builtin_inff();
  for (int key = first + lane; key - lane < end; key += 64) {
    const bool c = is_cold(srow, key, end);
    cold += __popcll(__ballot(c));
    const float s = c ? vrow[key] : -__builtin_inff();
    best = fmaxf(best, s);
    if (key < end && v.verifier_scores) v.verifier_scores[(size_t)row * a.length + key] = s;
  }
  best = wave_max(best);
  if (lane == 0) {
    v.block_scores[(size_t)row * a.blocks + blk] = cold ? best : -__builtin_inff();
    v.cold_count[(size_t)row * a.blocks + blk] = (uint8_t)cold;
  }
}

// Rescue ranking, one 1024-thread workgroup per row (blocks <= kSortN).
// Sort entries: cold blocks first (group bit), larger verifier block score,
// lower block id.
__global__ __launch_bounds__(1024) void verifier_rank_kernel(TemporalArgs a, VerifierArgs v) {
  __shared__ uint64_t xh[kSortN];
  __shared__ uint32_t xl[kSortN];
  __shared__ __align__(16) uint32_t scan_ws[16];
  const int tid = threadIdx.x;
  const int row = blockIdx.x;
  const int nb = a.blocks;
  uint64_t h[2] = {~0ull, ~0ull};
  uint32_t l[2] = {0xffffffffu, 0xffffffffu};
  uint32_t blocks_cold = 0, tokens_cold = 0, above = 0;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int b = 2 * tid + j;
    if (b >= nb) continue;
    const uint32_t n = v.cold_count[(size_t)row * nb + b];
    const float s = v.block_scores[(size_t)row * nb + b];
    blocks_cold += n ? 1u : 0u;
    tokens_cold += n;
    above += (n && s >= v.threshold) ? 1u : 0u;
    h[j] = n ? (uint64_t)(0xffffffffu - float_to_ordered(s)) : ~0ull;
    l[j] = (n ? 0u : 0x80000000u) | (uint32_t)b;
  }
  uint32_t total_blocks, total_tokens, total_above;
  block_excl_scan<16>(blocks_cold, scan_ws, total_blocks);
  __syncthreads();
  block_excl_scan<16>(tokens_cold, scan_ws, total_tokens);
  __syncthreads();
  block_excl_scan<16>(above, scan_ws, total_above);
  uint32_t rescue;
  if (v.promotion == 0) {
    const double budget = __builtin_ceil(v.fraction * (double)total_blocks);
    rescue = budget >= (double)total_blocks ? total_blocks : (uint32_t)budget;
  } else {
    rescue = total_above;
  }
  int n = 2;
  while (n < nb) n <<= 1;
  block_sort(h, l, xh, xl, n);
  uint32_t rescued_tokens = 0;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int p = 2 * tid + j;
    if (p >= nb) continue;
    const int b = (int)(l[j] & 0x7fffffffu);
    const bool take = (uint32_t)p < rescue;
    v.rescued[(size_t)row * nb + b] = take ? 1 : 0;
    if (take) rescued_tokens += v.cold_count[(size_t)row * nb + b];
    if (v.ranking) v.ranking[(size_t)row * nb + p] = (uint32_t)p < total_blocks ? b : -1;
  }
  __syncthreads();
  uint32_t total_rescued_tokens;
  block_excl_scan<16>(rescued_tokens, scan_ws, total_rescued_tokens);
  if (tid == 0) {
    int32_t* c = v.counts + (size_t)row * kCountFields;
    c[0] = (int32_t)total_tokens;
    c[1] = (int32_t)total_blocks;
    c[2] = (int32_t)rescue;
    c[3] = (int32_t)total_rescued_tokens;
  }
}

// Full scores of the rescued blocks' cold keys (one wave per block).
template <class Tag, class KF>
__global__ __launch_bounds__(256) void verifier_rescue_kernel(TemporalArgs a, VerifierArgs v) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15;
  const int g = lane >> 4;
  const int per_row = (a.blocks + 3) / 4;
  const int row = blockIdx.x / per_row;
  const int blk = (blockIdx.x % per_row) * 4 + wave;
  if (blk >= a.blocks || !v.rescued[(size_t)row * a.blocks + blk]) return;
  const int first = blk * a.block_size;
  const int end = min(a.length, first + a.block_size);
  float* srow = a.scores + (size_t)row * a.length;
  for (int u = first >> 6; u * 64 < end; ++u) {
    int tile_key[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int tile = u * 64 + 16 * t;  // blocks are whole 16-key tiles
      tile_key[t] = (tile >= first && tile < first + a.block_size) ? tile + r : (int)kFarKey;
    }
    const int key = u * 64 + lane;
    float s;
    if (a.source)  // trace replay: the recorded score
      s = (key >= first && key < end) ? a.source[(size_t)row * a.source_stride + key] : 0.f;
    else
      s = score_unit<Tag, KF>(a, row, tile_key, r, g);
    if (key >= first && key < end && srow[key] == -__builtin_inff()) {
      if constexpr (KF::kScaled)
        if (!a.source) s *= a.scales[(size_t)row * ((a.key_stride + 127) / 128) + (key >> 7)];
      srow[key] = s;
    }
  }
}

template <class Tag, class KF>
int launch_head_scan(const TemporalArgs& a, const VerifierArgs& v, dim3 grid, hipStream_t stream) {
  switch ((v.width + 15) / 16) {
    case 1: hipLaunchKernelGGL((verifier_head_scan_kernel<Tag, KF, 1>), grid, dim3(256), 0, stream, a, v); break;
    case 2: hipLaunchKernelGGL((verifier_head_scan_kernel<Tag, KF, 2>), grid, dim3(256), 0, stream, a, v); break;
    case 3: hipLaunchKernelGGL((verifier_head_scan_kernel<Tag, KF, 3>), grid, dim3(256), 0, stream, a, v); break;
    default: hipLaunchKernelGGL((verifier_head_scan_kernel<Tag, KF, 4>), grid, dim3(256), 0, stream, a, v); break;
  }
  return check_launch("verifier_head_scan_kernel");
}

template <class Tag, class KF>
int launch_verifier(TemporalArgs& a, VerifierArgs& v, int32_t path, int32_t wave, int32_t key_dtype,
                    int64_t* out_topk, hipStream_t stream) {
  if (int st = temporal_scan(a, wave, key_dtype, stream)) return st;
  const dim3 grid((unsigned)(a.rows * ((a.blocks + 3) / 4)));
  if (v.vsource) {
    hipLaunchKernelGGL(verifier_source_scan_kernel, grid, dim3(256), 0, stream, a, v);
    if (int st = check_launch("verifier_source_scan_kernel")) return st;
  } else if (path == DSA_VERIFIER_HEAD) {
    if (int st = launch_head_scan<Tag, KF>(a, v, grid, stream)) return st;
  } else {
    switch ((v.width + 31) / 32) {
      case 1: hipLaunchKernelGGL(verifier_dim_scan_kernel<1>, grid, dim3(256), 0, stream, a, v); break;
      case 2: hipLaunchKernelGGL(verifier_dim_scan_kernel<2>, grid, dim3(256), 0, stream, a, v); break;
      case 3: hipLaunchKernelGGL(verifier_dim_scan_kernel<3>, grid, dim3(256), 0, stream, a, v); break;
      default: hipLaunchKernelGGL(verifier_dim_scan_kernel<4>, grid, dim3(256), 0, stream, a, v); break;
    }
    if (int st = check_launch("verifier_dim_scan_kernel")) return st;
  }
  hipLaunchKernelGGL(verifier_rank_kernel, dim3(a.rows), dim3(1024), 0, stream, a, v);
  if (int st = check_launch("verifier_rank_kernel")) return st;
  hipLaunchKernelGGL((verifier_rescue_kernel<Tag, KF>), grid, dim3(256), 0, stream, a, v);
  if (int st = check_launch("verifier_rescue_kernel")) return st;
  return temporal_finish(a, out_topk, v.rescued, stream);
}

int check_sketch_dtype(int32_t dtype) {
  DSA_REQUIRE(dtype == DSA_DTYPE_F32 || dtype == DSA_DTYPE_F16 || dtype == DSA_DTYPE_BF16,
              "sketch rows must be fp32, fp16 or bf16 (got %d)", dtype);
  return DSA_STATUS_OK;
}

}  // namespace
}  // namespace dsa

using namespace dsa;

extern "C" int dsa_dim_sketch(const void* x, int64_t rows, int32_t dim, int32_t dtype, const int32_t* dims,
                              int32_t width, int32_t rotate, int32_t bits, float scale, void* out, int32_t out_codes,
                              void* stream) {
  DSA_REQUIRE(x && out, "null pointer argument");
  if (int st = check_sketch_dtype(dtype)) return st;
  DSA_REQUIRE(rows >= 0 && rows <= (int64_t(1) << 36), "rows %lld out of range", (long long)rows);
  DSA_REQUIRE(dim >= 1 && dim <= 128 && (dim & (dim - 1)) == 0, "dim %d must be a power of two <= 128", dim);
  DSA_REQUIRE(width >= 1 && width <= dim, "width %d outside [1, %d]", width, dim);
  DSA_REQUIRE(bits == 0 || bits == 2 || bits == 4 || bits == 8, "bits must be 0 (none), 2, 4 or 8");
  DSA_REQUIRE(bits == 0 || scale > 0.f, "quantization needs a positive scale");
  DSA_REQUIRE(!out_codes || bits, "codes need bits");
  if (rows == 0) return DSA_STATUS_OK;
  SketchArgs a;
  a.x = x;
  a.dims = dims;
  a.out = out;
  a.rows = rows;
  a.dim = dim;
  a.width = width;
  a.rotate = rotate;
  a.limit = bits ? (1 << (bits - 1)) - 1 : 0;
  a.out_codes = out_codes;
  a.scale = scale;
  a.norm = (float)std::pow((double)dim, -0.5);
  const dim3 grid((unsigned)((rows + 3) / 4));
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case DSA_DTYPE_BF16: hipLaunchKernelGGL(sketch_kernel<DSA_DTYPE_BF16>, grid, dim3(256), 0, s, a); break;
    case DSA_DTYPE_F16: hipLaunchKernelGGL(sketch_kernel<DSA_DTYPE_F16>, grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL(sketch_kernel<DSA_DTYPE_F32>, grid, dim3(256), 0, s, a); break;
  }
  return check_launch("sketch_kernel");
}

extern "C" int dsa_abs_max(const void* x, int64_t n, int32_t dtype, float* out, void* stream) {
  DSA_REQUIRE(x && out, "null pointer argument");
  if (int st = check_sketch_dtype(dtype)) return st;
  DSA_REQUIRE(n > 0, "n must be positive");
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t* o = reinterpret_cast<uint32_t*>(out);
  hipLaunchKernelGGL(zero_u32_kernel, dim3(1), dim3(1), 0, s, o);
  const unsigned grid = (unsigned)((n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024);
  switch (dtype) {
    case DSA_DTYPE_BF16: hipLaunchKernelGGL(abs_max_kernel<DSA_DTYPE_BF16>, dim3(grid), dim3(256), 0, s, x, n, o); break;
    case DSA_DTYPE_F16: hipLaunchKernelGGL(abs_max_kernel<DSA_DTYPE_F16>, dim3(grid), dim3(256), 0, s, x, n, o); break;
    default: hipLaunchKernelGGL(abs_max_kernel<DSA_DTYPE_F32>, dim3(grid), dim3(256), 0, s, x, n, o); break;
  }
  return check_launch("abs_max_kernel");
}

extern "C" int dsa_fake_quantize(const void* x, int64_t n, int32_t dtype, int32_t bits, float scale, void* values,
                                 int8_t* codes, void* stream) {
  DSA_REQUIRE(x && (values || codes), "null pointer argument");
  if (int st = check_sketch_dtype(dtype)) return st;
  DSA_REQUIRE(bits == 2 || bits == 4 || bits == 8, "bits must be one of 2, 4, 8");
  DSA_REQUIRE(scale > 0.f, "scale must be positive");
  DSA_REQUIRE(n >= 0 && n < (int64_t(1) << 40), "n out of range");
  if (n == 0) return DSA_STATUS_OK;
  const int32_t limit = (1 << (bits - 1)) - 1;
  const dim3 grid((unsigned)((n + 255) / 256));
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case DSA_DTYPE_BF16:
      hipLaunchKernelGGL(fake_quantize_kernel<DSA_DTYPE_BF16>, grid, dim3(256), 0, s, x, n, scale, limit, values, codes);
      break;
    case DSA_DTYPE_F16:
      hipLaunchKernelGGL(fake_quantize_kernel<DSA_DTYPE_F16>, grid, dim3(256), 0, s, x, n, scale, limit, values, codes);
      break;
    default:
      hipLaunchKernelGGL(fake_quantize_kernel<DSA_DTYPE_F32>, grid, dim3(256), 0, s, x, n, scale, limit, values, codes);
      break;
  }
  return check_launch("fake_quantize_kernel");
}

extern "C" int dsa_sketch_scores(const void* query_sketch, const float* weights, int64_t queries, int32_t heads,
                                 const void* key_sketch, int32_t sketch_codes, float sketch_scale, int32_t width,
                                 int64_t keys, float* out, void* stream) {
  DSA_REQUIRE(query_sketch && weights && key_sketch && out, "null pointer argument");
  DSA_REQUIRE(heads >= 1 && heads <= kHeads, "heads %d outside [1, 64]", heads);
  DSA_REQUIRE(width >= 8 && width <= 128 && width % 8 == 0, "width %d must be a multiple of 8 in [8, 128]", width);
  DSA_REQUIRE(queries >= 0 && queries <= 65535 && keys >= 0 && keys < (int64_t(1) << 31), "queries/keys out of range");
  DSA_REQUIRE(!sketch_codes || sketch_scale > 0.f, "codes need a positive scale");
  DSA_REQUIRE(reinterpret_cast<uintptr_t>(query_sketch) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(key_sketch) % (sketch_codes ? 8 : 16) == 0,
              "sketches must be 16-byte aligned (codes: 8-byte)");
  if (queries == 0 || keys == 0) return DSA_STATUS_OK;
  SketchKeys s;
  s.base = static_cast<const uint8_t*>(key_sketch);
  s.width = width;
  s.codes = sketch_codes;
  s.scale = sketch_scale;
  const dim3 grid((unsigned)((keys + 63) / 64), (unsigned)queries);
  const uint16_t* q = static_cast<const uint16_t*>(query_sketch);
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch ((width + 31) / 32) {
    case 1: hipLaunchKernelGGL(sketch_scores_kernel<1>, grid, dim3(256), 0, st, q, weights, heads, s, out, keys); break;
    case 2: hipLaunchKernelGGL(sketch_scores_kernel<2>, grid, dim3(256), 0, st, q, weights, heads, s, out, keys); break;
    case 3: hipLaunchKernelGGL(sketch_scores_kernel<3>, grid, dim3(256), 0, st, q, weights, heads, s, out, keys); break;
    default: hipLaunchKernelGGL(sketch_scores_kernel<4>, grid, dim3(256), 0, st, q, weights, heads, s, out, keys); break;
  }
  return check_launch("sketch_scores_kernel");
}

extern "C" int dsa_verifier_step(const void* queries, const float* weights, const void* keys, int64_t key_stride,
                                 const float* key_scales, const dsa_approx_policy* policy, const double* gamma_rows,
                                 int64_t prev_length, const int64_t* prev_topk, float* last_max, float* ema,
                                 float* volatility, int16_t* age, int16_t* cold_streak, int64_t state_stride,
                                 const dsa_verifier_spec* spec, const int32_t* head_ids, int64_t head_id_stride,
                                 const void* query_sketch, const void* key_sketch, int64_t sketch_stride,
                                 float* scores, float* verifier_scores, float* block_scores, uint8_t* cold_count,
                                 uint8_t* evaluated_blocks, uint8_t* rescued_blocks, int32_t* ranking,
                                 int64_t* out_topk, int32_t* qk_scored, int32_t* counts, int64_t batch,
                                 int64_t length, int64_t k, int32_t block_size, int32_t wave, int32_t key_dtype,
                                 void* workspace, int64_t workspace_bytes, void* stream) {
  DSA_REQUIRE(queries && weights && keys && policy && spec && prev_topk && last_max && ema && volatility && age &&
                  cold_streak && scores && block_scores && cold_count && evaluated_blocks && rescued_blocks &&
                  out_topk && qk_scored && counts,
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
  DSA_REQUIRE(spec->path == DSA_VERIFIER_HEAD || spec->path == DSA_VERIFIER_DIM, "verifier path %d unknown",
              spec->path);
  DSA_REQUIRE(spec->promotion == 0 || spec->promotion == 1, "promotion %d unknown", spec->promotion);
  DSA_REQUIRE(spec->rescue_fraction >= 0.0 && spec->rescue_fraction <= 1.0, "rescue_fraction outside [0, 1]");
  if (spec->path == DSA_VERIFIER_HEAD) {
    DSA_REQUIRE(head_ids, "the head path needs head ids");
    DSA_REQUIRE(spec->width >= 1 && spec->width <= kHeads, "head width %d outside [1, 64]", spec->width);
    DSA_REQUIRE(head_id_stride == 0 || head_id_stride >= spec->width, "head_id_stride < width");
  } else {
    DSA_REQUIRE(query_sketch && key_sketch, "the dim path needs query and key sketches");
    DSA_REQUIRE(spec->width >= 8 && spec->width <= 128 && spec->width % 8 == 0,
                "sketch width %d must be a multiple of 8 in [8, 128]", spec->width);
    DSA_REQUIRE(sketch_stride >= length, "sketch_stride < length");
    DSA_REQUIRE(!spec->sketch_codes || spec->sketch_scale > 0.f, "sketch codes need a positive scale");
    DSA_REQUIRE(reinterpret_cast<uintptr_t>(query_sketch) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(key_sketch) % (spec->sketch_codes ? 8 : 16) == 0,
                "sketches must be 16-byte aligned (codes: 8-byte)");
  }
  const int64_t blocks = (length + block_size - 1) / block_size;
  DSA_REQUIRE(state_stride >= blocks, "state_stride %lld < %lld blocks", (long long)state_stride, (long long)blocks);
  const TemporalWorkspace ws = temporal_layout(workspace, batch, length, k, block_size);
  if (!workspace || workspace_bytes < ws.bytes)
    return fail(DSA_STATUS_WORKSPACE_TOO_SMALL, "the verifier step needs %lld workspace bytes", (long long)ws.bytes);
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
  VerifierArgs v = {};
  v.head_ids = head_ids;
  v.id_stride = head_id_stride;
  v.width = spec->width;
  v.q_sketch = static_cast<const uint16_t*>(query_sketch);
  v.key_sketch = static_cast<const uint8_t*>(key_sketch);
  v.sketch_stride = sketch_stride;
  v.sketch_codes = spec->sketch_codes;
  v.sketch_scale = spec->sketch_scale;
  v.verifier_scores = verifier_scores;
  v.block_scores = block_scores;
  v.cold_count = cold_count;
  v.rescued = rescued_blocks;
  v.ranking = ranking;
  v.counts = counts;
  v.promotion = spec->promotion;
  v.fraction = spec->rescue_fraction;
  v.threshold = spec->promotion_threshold;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (key_dtype) {
    case DSA_DTYPE_BF16: return launch_verifier<Bf16Tag, KeysB16>(a, v, spec->path, wave, key_dtype, out_topk, s);
    case DSA_DTYPE_F16: return launch_verifier<F16Tag, KeysB16>(a, v, spec->path, wave, key_dtype, out_topk, s);
    default: return launch_verifier<Bf16Tag, KeysFP8>(a, v, spec->path, wave, key_dtype, out_topk, s);
  }
}

extern "C" int dsa_verifier_replay_step(const float* current_scores, int64_t score_stride,
                                        const float* recorded_verifier_scores, int64_t verifier_stride,
                                        const dsa_approx_policy* policy, const double* gamma_rows,
                                        int64_t prev_length, const int64_t* prev_topk, float* last_max, float* ema,
                                        float* volatility, int16_t* age, int16_t* cold_streak, int64_t state_stride,
                                        const dsa_verifier_spec* spec, float* scores, float* verifier_scores,
                                        float* block_scores, uint8_t* cold_count, uint8_t* evaluated_blocks,
                                        uint8_t* rescued_blocks, int32_t* ranking, int64_t* out_topk,
                                        int32_t* qk_scored, int32_t* counts, int64_t batch, int64_t length,
                                        int64_t k, int32_t block_size, int32_t wave, void* workspace,
                                        int64_t workspace_bytes, void* stream) {
  DSA_REQUIRE(current_scores && recorded_verifier_scores && policy && spec && prev_topk && last_max && ema &&
                  volatility && age && cold_streak && scores && block_scores && cold_count && evaluated_blocks &&
                  rescued_blocks && out_topk && qk_scored && counts,
              "null pointer argument");
  DSA_REQUIRE(score_stride >= length && verifier_stride >= length, "score rows shorter than length");
  if (int st = check_step(nullptr, nullptr, length, nullptr, prev_length, batch, length, k, block_size, wave,
                          DSA_DTYPE_BF16, workspace))
    return st;
  DSA_REQUIRE(policy->risk_model == DSA_RISK_LAST_MAX || policy->risk_model == DSA_RISK_EMA,
              "risk_model %d unknown", policy->risk_model);
  DSA_REQUIRE(policy->order >= DSA_ORDER_ADDRESS && policy->order <= DSA_ORDER_BUCKET, "order %d unknown",
              policy->order);
  DSA_REQUIRE(policy->order != DSA_ORDER_BUCKET || policy->buckets >= 1, "bucket order needs buckets >= 1");
  DSA_REQUIRE(policy->recent_window >= 0, "recent_window must be >= 0");
  DSA_REQUIRE(spec->promotion == 0 || spec->promotion == 1, "promotion %d unknown", spec->promotion);
  DSA_REQUIRE(spec->rescue_fraction >= 0.0 && spec->rescue_fraction <= 1.0, "rescue_fraction outside [0, 1]");
  const int64_t blocks = (length + block_size - 1) / block_size;
  DSA_REQUIRE(state_stride >= blocks, "state_stride %lld < %lld blocks", (long long)state_stride, (long long)blocks);
  const TemporalWorkspace ws = temporal_layout(workspace, batch, length, k, block_size);
  if (!workspace || workspace_bytes < ws.bytes)
    return fail(DSA_STATUS_WORKSPACE_TOO_SMALL, "the verifier replay step needs %lld workspace bytes",
                (long long)ws.bytes);
  TemporalArgs a = {};
  a.source = current_scores;
  a.source_stride = score_stride;
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
  a.ws = ws;
  VerifierArgs v = {};
  v.width = spec->width;
  v.verifier_scores = verifier_scores;
  v.block_scores = block_scores;
  v.cold_count = cold_count;
  v.rescued = rescued_blocks;
  v.ranking = ranking;
  v.counts = counts;
  v.promotion = spec->promotion;
  v.fraction = spec->rescue_fraction;
  v.threshold = spec->promotion_threshold;
  v.vsource = recorded_verifier_scores;
  v.vsource_stride = verifier_stride;
  return launch_verifier<Bf16Tag, KeysB16>(a, v, spec->path, wave, DSA_DTYPE_BF16, out_topk,
                                           static_cast<hipStream_t>(stream));
}
