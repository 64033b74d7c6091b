// Candidate-list epilogue shared by the scoring kernels that feed the list
// top-k (select.hip): the dense decode kernel (score.hip) and the fused
// static temporal step (temporal_fused.hip).
#pragma once

#include "common.hpp"
#include "select.hpp"
#include "waveops.hpp"

namespace dsa {

// A scoring workgroup's candidate list: thread t takes keys [t * per, t * per
// + per) of the chunk (per <= P), all read from LDS at once, and writes those
// in bins >= lbin in index order at offsets from one block scan.
template <int P, int kWaves>
__device__ __forceinline__ uint32_t emit_list(const float* chunk_scores, int per, int n_chunk, int chunk_base,
                                              uint32_t lbin, uint64_t* list, uint32_t* wsum) {
  const int i0 = (int)threadIdx.x * per;
  uint32_t key[P];
  uint32_t takes = 0;  // bit e: key e is listed
#pragma unroll
  for (int e = 0; e < P; ++e) {
    key[e] = float_to_ordered(chunk_scores[e < per ? i0 + e : i0]);
    if (e < per && i0 + e < n_chunk && (key[e] >> 20) >= lbin) takes |= 1u << e;
  }
  uint32_t listed;
  uint32_t slot = block_excl_scan<kWaves>((uint32_t)__builtin_popcount(takes), wsum, listed);
  if (takes) {
#pragma unroll
    for (int e = 0; e < P; ++e)
      if (takes & (1u << e)) list[slot++] = select_composite(key[e], (uint32_t)(chunk_base + i0 + e));
  }
  return listed;
}

// The whole epilogue, after the chunk's scores are in chunk_scores and their
// bins in hist: every key of the chunk whose bin is at least the bin of the
// chunk's quota-th largest score (all keys when the chunk has no more), in
// index order, and the list's length and lowest bin in meta[0..1].
template <int kWaves>
__device__ __forceinline__ void write_chunk_list(const uint32_t* hist, const float* chunk_scores, int chunk_keys,
                                                 int n_chunk, int chunk_base, uint32_t quota, uint64_t* list,
                                                 uint32_t* meta, uint32_t* s_bin, uint32_t* wsum) {
  constexpr int kThreads = 64 * kWaves;
  const int lane = threadIdx.x & 63;
  if (threadIdx.x < 64) {
    const Locate t = wave_locate<kSelectBins / kWave>(hist, quota, true);
    if (lane == 0) *s_bin = t.digit == kNoBin ? 0u : t.digit;
  }
  __syncthreads();
  const uint32_t lbin = *s_bin;
  uint32_t listed;
  const int per = chunk_keys / kThreads;  // keys per thread, 1..32
  switch (per) {
    case 1: listed = emit_list<1, kWaves>(chunk_scores, 1, n_chunk, chunk_base, lbin, list, wsum); break;
    case 2: listed = emit_list<2, kWaves>(chunk_scores, 2, n_chunk, chunk_base, lbin, list, wsum); break;
    case 3:
    case 4: listed = emit_list<4, kWaves>(chunk_scores, per, n_chunk, chunk_base, lbin, list, wsum); break;
    case 5: case 6: case 7:
    case 8: listed = emit_list<8, kWaves>(chunk_scores, per, n_chunk, chunk_base, lbin, list, wsum); break;
    case 9: case 10: case 11: case 12: case 13: case 14: case 15:
    case 16: listed = emit_list<16, kWaves>(chunk_scores, per, n_chunk, chunk_base, lbin, list, wsum); break;
    default: listed = emit_list<32, kWaves>(chunk_scores, per, n_chunk, chunk_base, lbin, list, wsum); break;
  }
  if (threadIdx.x == 0) {
    meta[0] = listed;
    meta[1] = lbin;
  }
}

}  // namespace dsa
