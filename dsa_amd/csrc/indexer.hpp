// Shared MFMA tile code of the indexer scoring kernels (score.hip) and the
// temporal pruning kernels (temporal.hip).  Both compute a key's score with
// the same instructions in the same order, so a key scored by either path
// gets the same fp32 value.
#pragma once

#include "common.hpp"

namespace dsa {

// ---------------------------------------------------------------------------
// Key row formats.  `load` fetches the lane's 32-dim slice of one key of a
// 16-key tile; `step(raw, j)` yields the 8 dims of MFMA k-step j as bf16/f16.
// ---------------------------------------------------------------------------
struct KeysB16 {  // bf16 or fp16 rows, 256 B
  static constexpr int kRowBytes = 256;
  static constexpr int kRaw = 4;
  static constexpr int kBuffers = 2;  // units in flight per wave in the streaming loop
  static constexpr bool kScaled = false;
  // Natural k order: k-step j of lane group g is dims 32j + 8g .. +8, so one
  // load instruction reads 64 contiguous bytes of each of the tile's 16 rows.
  static constexpr bool kNaturalK = true;
  __device__ static __forceinline__ void load(const uint8_t* base, int key, int g,
                                              uint4 (&raw)[kRaw]) {
    const uint8_t* row = base + (size_t)key * kRowBytes + g * 16;
#pragma unroll
    for (int c = 0; c < kRaw; ++c) raw[c] = *reinterpret_cast<const uint4*>(row + 64 * c);
  }
  __device__ static __forceinline__ void load_buf(BufferRsrc rsrc, int key, int g,
                                                  uint4 (&raw)[kRaw]) {
    const uint32_t off = (uint32_t)key * kRowBytes + g * 16;
#pragma unroll
    for (int c = 0; c < kRaw; ++c) raw[c] = buffer_load_16(rsrc, off + 64 * c);
  }
  __device__ static __forceinline__ uint4 step(const uint4 (&raw)[kRaw], int j) { return raw[j]; }
  // Byte offset of the lane's slice of tile t inside a 64-key unit, and the
  // loads of that slice through a resource whose base is the unit's first key.
  __device__ static __forceinline__ uint32_t lane_offset(int t, int r, int g) {
    return (uint32_t)(16 * t + r) * kRowBytes + 16u * g;
  }
  __device__ static __forceinline__ void load_at(BufferRsrc unit, uint32_t off, uint4 (&raw)[kRaw]) {
#pragma unroll
    for (int c = 0; c < kRaw; ++c) raw[c] = buffer_load_16(unit, off + 64 * c);
  }
};

struct KeysFP8 {  // fp8 e4m3fn rows, 128 B, one fp32 scale per 128 keys
  static constexpr int kRowBytes = 128;
  static constexpr int kRaw = 2;
  static constexpr int kBuffers = 4;  // half-size units: twice as many in flight, same bytes as bf16
  static constexpr bool kScaled = true;
  // Permuted k order: k-step j of lane group g is dims 32g + 8j .. +8; a lane
  // reads 32 contiguous bytes, and two instructions cover each 128-byte row.
  static constexpr bool kNaturalK = false;
  __device__ static __forceinline__ void load(const uint8_t* base, int key, int g,
                                              uint4 (&raw)[kRaw]) {
    const uint4* p = reinterpret_cast<const uint4*>(base + (size_t)key * kRowBytes + g * 32);
    raw[0] = p[0];
    raw[1] = p[1];
  }
  __device__ static __forceinline__ void load_buf(BufferRsrc rsrc, int key, int g,
                                                  uint4 (&raw)[kRaw]) {
    const uint32_t off = (uint32_t)key * kRowBytes + g * 32;
    raw[0] = buffer_load_16(rsrc, off);
    raw[1] = buffer_load_16(rsrc, off + 16);
  }
  __device__ static __forceinline__ uint4 step(const uint4 (&raw)[kRaw], int j) {
    const uint4 v = raw[j >> 1];
    return fp8x8_to_bf16x8((j & 1) ? make_uint2(v.z, v.w) : make_uint2(v.x, v.y));
  }
  __device__ static __forceinline__ uint32_t lane_offset(int t, int r, int g) {
    return (uint32_t)(16 * t + r) * kRowBytes + 32u * g;
  }
  __device__ static __forceinline__ void load_at(BufferRsrc unit, uint32_t off, uint4 (&raw)[kRaw]) {
    raw[0] = buffer_load_16(unit, off);
    raw[1] = buffer_load_16(unit, off + 16);
  }
};

// The M head tiles' dot products with one 16-key tile: acc[m] = Q_m . K^T.
template <class Tag, int M, class KF>
__device__ __forceinline__ void tile_mfma(const uint4 (&qa)[M][4], const uint4 (&raw)[KF::kRaw], floatx4 (&acc)[M]) {
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint4 kf = KF::step(raw, j);
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = mfma_16x16x32(Tag{}, qa[m][j], kf, acc[m]);
  }
}

// w_h * ReLU(acc) summed over the M-tiles' head slots held by this lane.
template <int M>
__device__ __forceinline__ float tile_reduce(const float (&wr)[M][4], const floatx4 (&acc)[M]) {
  float v = 0.f;
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) v = fmaf(wr[m][i], relu(acc[m][i]), v);
  return v;
}

template <class Tag, int M, class KF>
__device__ __forceinline__ float tile_contrib(const uint4 (&qa)[M][4], const float (&wr)[M][4],
                                              const uint4 (&raw)[KF::kRaw]) {
  floatx4 acc[M];
  tile_mfma<Tag, M, KF>(qa, raw, acc);
  return tile_reduce<M>(wr, acc);
}

// Element offset of k-step j's 8 dims for lane group g, in the key format's
// k order (the A and B fragments must use the same one).
template <bool kNaturalK>
__device__ __forceinline__ int kstep_dims(int g, int j) {
  return kNaturalK ? 32 * j + 8 * g : 32 * g + 8 * j;
}

// A fragments of heads 16m .. 16m+15 for m < M (no gather, no padding).
template <int M, bool kNaturalK>
__device__ __forceinline__ void load_dense_head_tiles(const uint16_t* q, const float* w, int r, int g,
                                                      uint4 (&qa)[M][4], float (&wr)[M][4]) {
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const uint16_t* row = q + (16 * m + r) * kHeadDim;
#pragma unroll
    for (int j = 0; j < 4; ++j) qa[m][j] = *reinterpret_cast<const uint4*>(row + kstep_dims<kNaturalK>(g, j));
#pragma unroll
    for (int i = 0; i < 4; ++i) wr[m][i] = w[16 * m + 4 * g + i];
  }
}

// Loads the A fragments of M head tiles.  Row slot s of the stacked tiles is
// head ids[s] (or head s when ids == nullptr) for s < count, else a zero row;
// an id outside [0, 64) also gives a zero row (and weight 0).
template <int M, bool kNaturalK>
__device__ __forceinline__ void load_head_tiles(const uint16_t* q, const float* w,
                                                const int32_t* ids, int count, int r, int g,
                                                uint4 (&qa)[M][4], float (&wr)[M][4]) {
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const int slot = 16 * m + r;
    int head = slot < count ? (ids ? ids[slot] : slot) : -1;
    head = head < kHeads ? head : -1;  // an id outside [0, 64) is a zero row
#pragma unroll
    for (int j = 0; j < 4; ++j)
      qa[m][j] = head >= 0 ? *reinterpret_cast<const uint4*>(q + head * kHeadDim + kstep_dims<kNaturalK>(g, j))
                           : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ws = 16 * m + 4 * g + i;
      int wh = ws < count ? (ids ? ids[ws] : ws) : -1;
      wh = wh < kHeads ? wh : -1;
      wr[m][i] = wh >= 0 ? w[wh] : 0.f;
    }
  }
}

// Reduction of a 64-key unit: lane (r, g) holds, for each of the unit's four
// 16-key tiles t, the partial p_g = sum over its head slots of w * ReLU(q.k)
// of key (t, r).  Two exchange rounds leave lane l with the score of key l of
// the unit, summed as (p0 + p1) + (p2 + p3) for every key.
__device__ __forceinline__ float unit_reduce(const float (&s)[4], int g) {
  const bool odd = g & 1;
  const bool high = g & 2;
  float keep_a = odd ? s[1] : s[0];
  float keep_b = odd ? s[3] : s[2];
  const float send_a = odd ? s[0] : s[1];
  const float send_b = odd ? s[2] : s[3];
  keep_a += __shfl_xor(send_a, 16, kWave);
  keep_b += __shfl_xor(send_b, 16, kWave);
  float keep = high ? keep_b : keep_a;
  const float send = high ? keep_a : keep_b;
  keep += __shfl_xor(send, 32, kWave);
  return keep;
}

}  // namespace dsa
