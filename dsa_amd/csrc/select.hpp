// Workspace and launch interface of the distributed decode-step top-k
// (select.hip), shared with the scoring kernel that fills its histogram.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dsa {

constexpr int kSelectBins = 4096;        // top 12 bits of the ordered score key
constexpr int kSelectChunk = 2048;       // scores per selection workgroup
constexpr int kMaxSelectChunks = 256;    // rows up to 524288 scores

struct SelectWorkspace {
  uint32_t* hist;        // [rows][kSelectBins], zero between calls
  uint32_t* cand_count;  // [rows][chunks]: per-chunk candidate count
  uint32_t* meta;        // [rows][4]: threshold bin, rank inside it, valid count
  uint32_t* above;       // [rows][chunks]: per-chunk count above the bin
  uint64_t* cand;        // [rows][length]: chunk j's candidates at [j * kSelectChunk, ...)
  int64_t bytes;
};

// Carves the workspace out of `base` (base == nullptr only measures it).
SelectWorkspace select_workspace_layout(void* base, int64_t rows, int64_t length);

// Builds the histogram of scores [rows, length] (every entry, -inf included)
// in the zeroed ws.hist, then selects their top-k.
int launch_select_scores(const float* scores, int64_t rows, int64_t length, int64_t k,
                         const SelectWorkspace& ws, int64_t* out_idx, float* out_val, hipStream_t stream);

// Selects the top-k of scores [rows, length] whose histogram is in ws.
int launch_select(const float* scores, int64_t rows, int64_t length, int64_t k,
                  const SelectWorkspace& ws, int64_t* out_idx, float* out_val,
                  hipStream_t stream);

}  // namespace dsa
