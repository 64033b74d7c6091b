// Shared device helpers for the gfx950 (CDNA4) indexer kernels.
//
// Conventions used by every kernel in this library:
//   * 64 indexer heads x 128 dims, one shared key row per token.
//   * Keys are row-major [L, 128]; a bf16/fp16 row is 256 B, an fp8 row 128 B,
//     an fp32 row 512 B.
//   * MFMA tiles are v_mfma_f32_16x16x32_{bf16,f16}: 16 heads x 16 keys per
//     tile, 32 dims per k-step, 4 k-steps per 128-dim row.
//   * Within one 16-key tile a lane owns key column (lane & 15) and the 32-dim
//     slice [32 * (lane >> 4), +32) of that key.  The k-step j of an MFMA uses
//     dims 32 * (lane >> 4) + 8 * j .. +8 for both operands, so A (queries) and
//     B (keys) agree on the dim permutation and every lane reads 64 contiguous
//     bytes of its key row.
//   * The 16x16 accumulator of a tile holds D[head = 4 * (lane >> 4) + i][key =
//     lane & 15] in element i of lane's float4.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dsa {

constexpr int kHeads = 64;
constexpr int kHeadDim = 128;
constexpr int kVerifierHeads = 8;
constexpr int kWave = 64;
constexpr int kXcds = 8;  // MI355X: 8 XCDs, workgroups dispatched round-robin

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx2 __attribute__((ext_vector_type(2)));

enum KeyDtype : int { kF32 = 0, kF16 = 1, kBF16 = 2, kFP8E4M3 = 3 };

// ---------------------------------------------------------------------------
// MFMA wrappers: one 16x16x32 product, fp32 accumulation.
// ---------------------------------------------------------------------------
struct Bf16Tag {};
struct F16Tag {};

__device__ __forceinline__ floatx4 mfma_16x16x32(Bf16Tag, uint4 a, uint4 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
__device__ __forceinline__ floatx4 mfma_16x16x32(F16Tag, uint4 a, uint4 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// fp8 e4m3fn (OCP, gfx950 native) -> bf16.  Every finite e4m3 value is exactly
// representable in bf16, so the conversion is lossless.  Two bytes are turned
// into two fp32 by the hardware converter and then truncated to bf16 (exact).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_exact(float lo, float hi) {
  return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);
}

// Converts 4 fp8 bytes packed in `v` into 4 bf16 packed in a uint2.
__device__ __forceinline__ uint2 fp8x4_to_bf16x4(uint32_t v) {
  floatx2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(v, false);
  floatx2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(v, true);
  return make_uint2(f32x2_to_bf16x2_exact(lo[0], lo[1]), f32x2_to_bf16x2_exact(hi[0], hi[1]));
}

// 8 fp8 bytes (uint2) -> 8 bf16 (uint4).
__device__ __forceinline__ uint4 fp8x8_to_bf16x8(uint2 v) {
  uint2 a = fp8x4_to_bf16x4(v.x);
  uint2 b = fp8x4_to_bf16x4(v.y);
  return make_uint4(a.x, a.y, b.x, b.y);
}

// ---------------------------------------------------------------------------
// Order-preserving float -> uint32 map used by the radix top-K.  -0.0 is folded
// onto +0.0 so that the two zeros compare equal (numpy semantics) and fall back
// to the index tie-break.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t float_to_ordered(float f) {
  uint32_t u = __float_as_uint(f);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float ordered_to_float(uint32_t o) {
  uint32_t u = (o & 0x80000000u) ? (o & 0x7fffffffu) : ~o;
  return __uint_as_float(u);
}

// ---------------------------------------------------------------------------
// Raw buffer resources (gfx9-family descriptor word 3 = 0x00020000).  Buffer
// loads past num_records return zeros and buffer stores past it are dropped by
// the hardware, so tails need neither clamped addresses nor branches.
// ---------------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t BufferRsrc;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ BufferRsrc make_buffer(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 buffer_load_16(BufferRsrc rsrc, uint32_t offset) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)offset, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void buffer_store_f32(BufferRsrc rsrc, uint32_t offset, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), rsrc, (int)offset, 0, 0);
}
__device__ __forceinline__ void buffer_store_16(BufferRsrc rsrc, uint32_t offset, uint4 v) {
  const u32x4 parts = {v.x, v.y, v.z, v.w};
  __builtin_amdgcn_raw_buffer_store_b128(parts, rsrc, (int)offset, 0, 0);
}
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void buffer_store_u64(BufferRsrc rsrc, uint32_t offset, uint64_t v) {
  const u32x2 parts = {(uint32_t)v, (uint32_t)(v >> 32)};
  __builtin_amdgcn_raw_buffer_store_b64(parts, rsrc, (int)offset, 0, 0);
}

// Kernel arguments live in the kernarg segment and are fetched by scalar loads
// that the compiler issues next to their first use, so a prologue with
// branches waits for several dependent round trips before its first vector
// load.  Naming the arguments here materialises them in SGPRs at this point:
// their loads issue together and complete in one round trip.
template <class T>
__device__ __forceinline__ void in_sgpr(const T& v) {
  asm volatile("" ::"s"(v));
}
template <class... T>
__device__ __forceinline__ void args_in_sgprs(const T&... v) {
  (in_sgpr(v), ...);
}

// ReLU as a signed-integer max on the float's bits: negative values (sign bit
// set) become +0.0, non-negative values pass unchanged.  One VALU op, where
// fmaxf(x, 0) costs two (NaN quieting).
__device__ __forceinline__ float relu(float x) {
  return __int_as_float(max(__float_as_int(x), 0));
}

// ---------------------------------------------------------------------------
// Wave-level reductions (64 lanes).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}
__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fminf(v, __shfl_xor(v, off, kWave));
  return v;
}
__device__ __forceinline__ float row16_max(float v) {
  // Max over the 16 lanes that share (lane >> 4).
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// Sum of one key's four 16-head partials held by lanes (r, r+16, r+32, r+48).
__device__ __forceinline__ float reduce_lane_groups(float v) {
  v += __shfl_xor(v, 16, kWave);
  v += __shfl_xor(v, 32, kWave);
  return v;
}

// ---------------------------------------------------------------------------
// Phase timestamps, compiled in only with -DDSA_PHASE_TRACE (the trace build
// of the library): thread 0 of workgroup `wg` stores the 100 MHz wall clock
// at mark i of a per-file log of kTraceWgs x kTraceMarks entries.
// ---------------------------------------------------------------------------
constexpr int kTraceWgs = 4096;
constexpr int kTraceMarks = 8;
#ifdef DSA_PHASE_TRACE
#define DSA_TRACE_MARK(log, wg, i)                                                         \
  do {                                                                                     \
    if (threadIdx.x == 0 && (uint32_t)(wg) < (uint32_t)kTraceWgs)                          \
      (log)[(size_t)(wg) * kTraceMarks + (i)] = wall_clock64();                            \
  } while (0)
#else
#define DSA_TRACE_MARK(log, wg, i) \
  do {                             \
  } while (0)
#endif

}  // namespace dsa
