// Wave-level building blocks of the selection kernels (select.hip,
// temporal.hip): DPP scans, ballot ranks and a two-level "which bin holds
// the want-th largest" search run by a single wave.
#pragma once

#include "common.hpp"

namespace dsa {

constexpr uint32_t kNoBin = 0xffffffffu;

__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x & (kWave - 1); }

// Same XCD-aware renumbering as the scoring kernel: with a grid that is a
// multiple of 8, a row's chunks run on one XCD, whose L2 holds its scores.
__device__ __forceinline__ uint32_t logical_block() {
  const uint32_t grid = gridDim.x;
  const uint32_t b = blockIdx.x;
  return (grid % 8u == 0u) ? (b % 8u) * (grid / 8u) + b / 8u : b;
}

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
template <int kWaves>
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* ws, uint32_t& total) {
  static_assert(kWaves % 4 == 0, "wave sums are read 4 at a time");
  const uint32_t lane = lane_id();
  const uint32_t wave = threadIdx.x / kWave;
  const uint32_t incl = wave_incl_scan(v);
  if (lane == kWave - 1) ws[wave] = incl;
  __syncthreads();
  uint32_t before = 0;
  uint32_t all = 0;
#pragma unroll
  for (int q = 0; q < kWaves / 4; ++q) {
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
  uint32_t total;  // keys in all bins
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
  if (m == 0 || (none_if_fits && total <= want)) return Locate{kNoBin, 0u, 0u, total};
  const uint32_t owner = (uint32_t)__builtin_ctzll(m);
  const uint32_t above_owner = __builtin_amdgcn_readlane(above, owner);
  const uint32_t c = lane < (uint32_t)N ? bins[N * owner + lane] : 0u;
  const uint32_t incl2 = wave_incl_scan(c);
  const uint32_t above2 = above_owner + __builtin_amdgcn_readlane(incl2, kWave - 1) - incl2;
  const uint64_t m2 = __ballot(above2 < want && want <= above2 + c);
  const uint32_t j = (uint32_t)__builtin_ctzll(m2);
  return Locate{N * owner + j, want - (uint32_t)__builtin_amdgcn_readlane(above2, j),
                (uint32_t)__builtin_amdgcn_readlane(c, j), total};
}


}  // namespace dsa
