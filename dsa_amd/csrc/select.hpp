// Workspace and launch interface of the distributed decode-step top-k
// (select.hip), shared with the scoring kernel that fills its histogram.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dsa {

constexpr int kSelectBins = 4096;        // top 12 bits of the ordered score key
constexpr int kSelectChunk = 2048;       // scores per selection workgroup
constexpr int kMaxSelectChunks = 256;    // rows up to 524288 scores
constexpr int kListChunkMax = 8192;      // keys per scoring workgroup for candidate lists (LDS)
constexpr int kMaxListChunks = 256;      // candidate lists per row
constexpr int kListStageCapacity = 8192;   // list entries a selection workgroup stages in LDS

struct SelectWorkspace {
  uint32_t* hist;        // [rows][kSelectBins], zero between calls
  uint32_t* cand_count;  // [rows][chunks]: per-chunk candidate count
  uint32_t* meta;        // [rows][4]: threshold bin, rank inside it, valid count
  uint32_t* above;       // [rows][chunks]: per-chunk count above the bin
  uint64_t* cand;        // [rows][length]: chunk j's candidates at [j * kSelectChunk, ...)
                         // (candidate lists: list j at [j * chunk_keys, ...))
  uint32_t* list_meta;   // [rows][kMaxListChunks][2]: list length, lowest 12-bit bin listed
  int64_t bytes;
};

// Units of 64 keys per workgroup of the dense scoring kernel: about
// target_wgs workgroups (one per CU at 256), so that every wave streams
// several units and pays its query-block load and pipeline fill once, with
// a multiple of `waves` units (at least one per wave) in each workgroup.
inline int32_t dense_units_per_wg(int64_t sequences, int64_t length, int64_t target_wgs = 256, int32_t waves = 4) {
  const int64_t units = (length + 63) / 64;
  int64_t per = (units * sequences + target_wgs - 1) / target_wgs;
  per = per < waves ? waves : per;
  per = (per + waves - 1) / waves * waves;
  return (int32_t)per;
}

constexpr int kDecodeWaves = 4;  // waves per workgroup of the decode step's scoring kernel (8 measured slower)

// Candidate lists of the decode step.  Each scoring workgroup owns
// chunk_keys consecutive keys of one row and, when the plan is on, lists the
// keys of its chunk whose 12-bit bin is at least the bin of its quota-th
// largest score: 1.25 k / chunks + 16, a quarter again the chunk's expected
// share of the row's top-k.  The plan is on when a chunk fits the scoring workgroup's
// LDS and a row's lists (about 1.5 k entries plus a bin's worth per chunk)
// fit the selection workgroup's.  dsa_score_hist and dsa_select_topk derive
// the same plan from (rows, length, k).
struct ListPlan {
  int32_t units_per_wg;
  int32_t chunk_keys;
  int32_t chunks;  // lists per row
  int32_t quota;
  bool on;
};

inline ListPlan list_plan(int64_t rows, int64_t length, int64_t k) {
  ListPlan p;
  p.units_per_wg = dense_units_per_wg(rows, length, 256, kDecodeWaves);
  p.chunk_keys = p.units_per_wg * 64;
  p.chunks = (int32_t)((length + p.chunk_keys - 1) / p.chunk_keys);
  const int64_t quota = (5 * k + 4 * (int64_t)p.chunks - 1) / (4 * (int64_t)p.chunks) + 16;
  p.quota = (int32_t)(quota < p.chunk_keys ? quota : p.chunk_keys);
  p.on = p.chunk_keys <= kListChunkMax && p.chunks <= kMaxListChunks &&
         (3 * k) / 2 + 64 * (int64_t)p.chunks <= kListStageCapacity;
  return p;
}

// A launch that, given events, records them at the kernel's own start and
// end (the interval a profiler's kernel trace reports), else a plain launch.
template <class K, class... Args>
inline void launch_timed(K kernel, dim3 grid, dim3 block, uint32_t lds, hipStream_t stream, hipEvent_t start,
                         hipEvent_t stop, Args... args) {
  if (start || stop)
    hipExtLaunchKernelGGL(kernel, grid, block, lds, stream, start, stop, 0u, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, lds, stream, args...);
}

// (order-preserving key << 32) | ~position: distinct per row, and larger for
// the larger score, or for the lower position among equal scores.
__device__ __forceinline__ uint64_t select_composite(uint32_t key, uint32_t pos) {
  return (uint64_t(key) << 32) | (uint64_t)(~pos);
}

// Carves the workspace out of `base` (base == nullptr only measures it).
SelectWorkspace select_workspace_layout(void* base, int64_t rows, int64_t length);

// Builds the histogram of scores [rows, length] (every entry, -inf included)
// in the zeroed ws.hist, then selects their top-k.
int launch_select_scores(const float* scores, int64_t rows, int64_t length, int64_t k,
                         const SelectWorkspace& ws, int64_t* out_idx, float* out_val, hipStream_t stream);

// Selects the top-k of scores [rows, length] whose histogram is in ws.
// start/stop, when not null, are recorded by the first and last kernel at
// their own start and end (hipExtLaunchKernel).
// The exact top-k (stable ties, index order) of each row of at most
// kTopkRowsMaxLength scores, one workgroup per row; rows with skip[row] != 0
// (skip nullable) are left as they are.
constexpr int64_t kTopkRowsMaxLength = 32768;
int launch_topk_rows(const float* scores, int64_t rows, int64_t length, int64_t k, int64_t* out_idx,
                     const uint32_t* skip, hipStream_t stream);

int launch_select(const float* scores, int64_t rows, int64_t length, int64_t k,
                  const SelectWorkspace& ws, int64_t* out_idx, float* out_val,
                  hipStream_t stream, hipEvent_t start = nullptr, hipEvent_t stop = nullptr,
                  const uint32_t* skip = nullptr);  // skip[row] != 0: the row is left as it is

// Selects the top-k of scores [rows, length] from the candidate lists that
// the scoring kernel wrote to ws under `plan`.
// With count_parts, also writes count_out[row] = the sum of bits 0-30 of the
// row's count_parts[row * plan.chunks + j] over its chunks j, and, with
// flag_out, flag_out[row] = the number of those parts with bit 31 set.
int launch_select_lists(const float* scores, int64_t rows, int64_t length, int64_t k,
                        const ListPlan& plan, const SelectWorkspace& ws, int64_t* out_idx,
                        float* out_val, hipStream_t stream, hipEvent_t start = nullptr,
                        hipEvent_t stop = nullptr, const uint32_t* count_parts = nullptr,
                        int32_t* count_out = nullptr, int32_t* flag_out = nullptr);

}  // namespace dsa
