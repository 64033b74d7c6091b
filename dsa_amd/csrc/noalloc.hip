// Allocation-free decode step: the scoring + exact top-K step of
// dsa_score_topk with its workspace held in a file-scope device array, for
// callers that cannot allocate device memory (code under HIP graph capture,
// tight serving loops, harnesses that forbid hipMalloc).
//
// Every GPU that runs this entry point holds its own copy of `scratch` from the
// library's module load until the process ends.  The host only ever uses the
// array through the device address hipGetSymbolAddress returns for the
// current device (the array's name is a host-side stand-in, not a device
// address).  All calls on one GPU share that GPU's copy, so calls that overlap
// on one GPU (on different streams, or from different threads without
// ordering) race; calls ordered on one stream do not.
#include <mutex>

#include "common.hpp"
#include "dsa_amd.h"
#include "select.hpp"
#include "status.hpp"

namespace dsa {
namespace {

constexpr int64_t kScratchBytes = DSA_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Zero fill of n 16-byte words (a kernel rather than hipMemsetAsync, so that
// a caller may capture the step in a graph).
__global__ __launch_bounds__(256) void zero_words_kernel(uint4* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// Device address of this GPU's scratch array, looked up once per device with
// that device current.
int scratch_address(void** out) {
  int device = -1;
  if (int st = check_hip(hipGetDevice(&device), "hipGetDevice")) return st;
  if (device < 0 || device >= kMaxDevices)
    return fail(DSA_STATUS_INVALID_ARGUMENT, "device %d outside [0, %d)", device, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[device]) {
    void* p = nullptr;
    if (int st = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)"))
      return st;
    if (!p || reinterpret_cast<uintptr_t>(p) % 256 != 0)
      return fail(DSA_STATUS_HIP_ERROR, "scratch array has no 256-byte aligned device address");
    g_scratch_ptr[device] = p;
  }
  *out = g_scratch_ptr[device];
  return DSA_STATUS_OK;
}

}  // namespace
}  // namespace dsa

using namespace dsa;

extern "C" int dsa_score_topk_noalloc(const void* queries, const float* weights, const void* keys,
                                      const float* key_scales, float* scores, int64_t batch, int64_t length,
                                      int64_t k, int32_t key_dtype, int64_t* out_indices, float* out_values,
                                      void* stream) {
  DSA_REQUIRE(batch > 0 && batch <= 65535, "batch %lld out of range", (long long)batch);
  DSA_REQUIRE(length > 0 && length <= int64_t(kSelectChunk) * kMaxSelectChunks,
              "length %lld outside [1, %d]", (long long)length, kSelectChunk * kMaxSelectChunks);
  DSA_REQUIRE(k > 0 && k <= (int64_t(1) << 27), "k=%lld out of range", (long long)k);
  const int64_t need = dsa_score_topk_workspace_bytes(batch, length);
  if (need > kScratchBytes)
    return fail(DSA_STATUS_WORKSPACE_TOO_SMALL,
                "batch %lld x length %lld needs %lld bytes of scratch; the allocation-free decode step holds "
                "%lld (use dsa_score_topk with a caller workspace)",
                (long long)batch, (long long)length, (long long)need, (long long)kScratchBytes);
  void* ws = nullptr;
  if (int st = scratch_address(&ws)) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // The array keeps the previous call's contents.  The histogram plan needs
  // the per-row histograms (offset 0, kSelectBins words per row) at zero; the
  // candidate-list plan writes everything it reads.
  if (!list_plan(batch, length, k).on) {
    const int64_t words = batch * kSelectBins * 4 / 16;
    const int64_t blocks = (words + 255) / 256;
    hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)(blocks < 1024 ? blocks : 1024)), dim3(256), 0, s,
                       static_cast<uint4*>(ws), words);
    if (int st = check_launch("zero_words_kernel")) return st;
  }
  return dsa_score_topk(queries, weights, keys, key_scales, scores, batch, length, k, key_dtype, out_indices,
                        out_values, ws, kScratchBytes, stream);
}
