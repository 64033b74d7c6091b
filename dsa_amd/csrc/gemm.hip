// Projections of the indexer sidecar for batches of tokens (reference
// sidecar.py:55-58 wq / wk / weights_proj, used by encode_queries and
// encode_keys, sidecar.py:74-88): out[t][f] = sum_k hidden[t][k] * W[f][k].
// (A decode step of at most 16 tokens streams the weights in project.hip.)
//
// gemm_bf16_kernel: bf16 hidden and weights, fp32 accumulation, bf16 out
// rounded once (nearest even), as a bf16 Linear stores it.  A workgroup owns
// BF features x BT tokens; its waves split them WF x WT (for wq: 256 x 256,
// eight waves of 128 features x 64 tokens).  Each k-stage of 64 stages the
// weight rows and the hidden rows in LDS (rows padded to 144 B), loaded NPF
// stages ahead into registers, and every wave runs
// v_mfma_f32_16x16x32_bf16 with 16 weight rows as the A operand and 16
// tokens as B: the accumulator of a tile then holds, per lane, four
// consecutive features of one token, stored as one 8-byte bf16x4.
// With kRope the output stage also applies the non-interleaved RoPE of the
// query heads (sidecar.py:10-28, 78-88): every 128-feature head rotates its
// first 64 dims, dim d with dim d + 32.  A wave's 64 features are one head's
// rotated or unrotated half, and dims d and d + 32 sit in the same lane (tiles
// f and f + 2), so the rotation needs no data exchange.  cos / sin come from
// rope_table_kernel, in the bf16 precision and per-op rounding of the
// encoder epilogues (sidecar.hip).
//
// gemm_f32_kernel: fp32 weights (weights_proj, which the reference runs on
// hidden.float(), and fp32 modules), hidden bf16 or fp32 widened exactly to
// fp32, v_mfma_f32_16x16x4_f32, fp32 out times an optional scale (the head
// weights' (heads * head_dim)^-0.5, one fp32 product as in the reference).
#include "common.hpp"
#include "dsa_amd.h"
#include "status.hpp"

namespace dsa {
namespace {

constexpr int kGemmBK = 64;            // k per stage (bf16)
constexpr int kGemmRow = kGemmBK + 8;  // bf16 per LDS row: 144 B against bank conflicts
constexpr uint32_t kFar = 0x80000000u; // a buffer offset past every resource: loads read 0, stores drop
constexpr int kRopeHalf = 32;          // fused RoPE: 64 rotated dims of every 128-dim head

struct GemmArgs {
  const uint16_t* hidden;  // [tokens][hidden_stride] bf16, or fp32 (gemm_f32_kernel with hidden_f32)
  int64_t hidden_stride;   // elements between tokens
  const void* weight;      // [features][kdim] bf16 or fp32
  void* out;               // [tokens][out_stride] bf16 or fp32
  int64_t out_stride;
  int32_t tokens, features, kdim;
  int32_t hidden_f32;      // gemm_f32_kernel: hidden is fp32
  float scale;             // gemm_f32_kernel: out = acc * scale
  const uint32_t* rope;    // kRope: [tokens][kRopeHalf] bf16 cos << 16 | bf16 sin
};

__device__ __forceinline__ uint32_t bf16_rne_bits(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t rounded = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  return (u & 0x7fffffffu) > 0x7f800000u ? (u >> 16) | 0x40u : rounded;  // NaN stays a (quiet) NaN
}
__device__ __forceinline__ float round_bf16f(float x) { return __uint_as_float(bf16_rne_bits(x) << 16); }

// cos / sin of position * theta^(-i / 32), i < 32, rounded to bf16: the
// rotation table of one token (the formula of the encoder epilogues).
__global__ __launch_bounds__(256) void rope_table_kernel(const int64_t* positions, int32_t tokens, float theta,
                                                         uint32_t* table) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= (int64_t)tokens * kRopeHalf) return;
  const int64_t t = e / kRopeHalf;
  const int i = (int)(e % kRopeHalf);
  const float angle = (float)positions[t] * powf(theta, -(float)i / (float)kRopeHalf);
  table[e] = (bf16_rne_bits(cosf(angle)) << 16) | bf16_rne_bits(sinf(angle));
}

template <int BF, int BT, int WF, int WT, bool kRope, int NPF>
__global__ __launch_bounds__(64 * WF * WT) void gemm_bf16_kernel(GemmArgs a) {
  constexpr int kThreads = 64 * WF * WT;
  constexpr int FW = BF / WF;  // features per wave
  constexpr int TW = BT / WT;  // tokens per wave
  constexpr int FT = FW / 16;
  constexpr int TT = TW / 16;
  constexpr int kRows = BF + BT;                  // LDS rows per stage: weights, then tokens
  // 16-byte chunks a thread stages: its first kPerW are weight rows, the
  // rest token rows, so that the buffer resource of a load is known at
  // compile time (a per-lane choice would cost a waterfall loop per load).
  constexpr int kPerW = BF * (kGemmBK / 8) / kThreads;
  constexpr int kPer = kPerW + BT * (kGemmBK / 8) / kThreads;
  static_assert(BF * (kGemmBK / 8) % kThreads == 0 && BT * (kGemmBK / 8) % kThreads == 0, "stage chunks per thread");
  static_assert(!kRope || FW == 64 || FW % 128 == 0, "a rotating wave owns half a 128-dim head or whole heads");
  __shared__ __align__(16) uint16_t lds[2][kRows][kGemmRow];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wf = wave % WF;
  const int wt = wave / WF;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int feature_tiles = (a.features + BF - 1) / BF;
  const int f0 = (int)(blockIdx.x % (uint32_t)feature_tiles) * BF;
  const int t0 = (int)(blockIdx.x / (uint32_t)feature_tiles) * BT;
  const int kdim = a.kdim;

  const BufferRsrc wr = make_buffer(a.weight, (uint32_t)a.features * (uint32_t)kdim * 2u);
  const BufferRsrc hr = make_buffer(a.hidden, (uint32_t)(((int64_t)(a.tokens - 1) * a.hidden_stride + kdim) * 2));
  // This thread's chunks of a stage: row rows_[i] (weights below BF), k
  // offset 8 * part_[i] within the stage.
  int row_of[kPer];
  uint32_t base_of[kPer];  // byte offset of the row's k = 0, or kFar for rows past the matrix
  int part_of[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int c = tid + kThreads * (i < kPerW ? i : i - kPerW);
    const int row = c / (kGemmBK / 8) + (i < kPerW ? 0 : BF);
    row_of[i] = row;
    part_of[i] = c % (kGemmBK / 8);
    if (i < kPerW) {
      const int f = f0 + row;
      base_of[i] = f < a.features ? (uint32_t)f * (uint32_t)kdim * 2u : kFar;
    } else {
      const int t = t0 + row - BF;
      base_of[i] = t < a.tokens ? (uint32_t)((int64_t)t * a.hidden_stride * 2) : kFar;
    }
  }
  // NPF stages in flight in registers (a ring), two in LDS.
  uint4 stage[NPF][kPer];
  auto load_stage = [&](int kt, uint4 (&dst)[kPer]) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int k = kt * kGemmBK + 8 * part_of[i];
      const uint32_t off = (base_of[i] == kFar || k >= kdim) ? kFar : base_of[i] + (uint32_t)k * 2u;
      dst[i] = buffer_load_16(i < kPerW ? wr : hr, off);
    }
  };
  auto store_stage = [&](int s, const uint4 (&src)[kPer]) {
#pragma unroll
    for (int i = 0; i < kPer; ++i)
      *reinterpret_cast<uint4*>(&lds[s][row_of[i]][8 * part_of[i]]) = src[i];
  };

  floatx4 acc[FT][TT];
#pragma unroll
  for (int i = 0; i < FT; ++i)
#pragma unroll
    for (int j = 0; j < TT; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int nk = (kdim + kGemmBK - 1) / kGemmBK;
  {
    uint4 first[kPer];
    load_stage(0, first);
#pragma unroll
    for (int p = 0; p < NPF; ++p) load_stage(min(1 + p, nk - 1), stage[p]);
    store_stage(0, first);
  }
  __syncthreads();
  // Iteration kt computes stage kt from LDS while stages kt + 1 .. kt + NPF
  // are in flight in registers; stage kt + 1 then goes to LDS and the loads
  // of stage kt + 1 + NPF take its registers.  Loads past the last stage
  // repeat it (unconditional, so that the compiler's waits cover exactly
  // the registers being stored).
  for (int kt0 = 0; kt0 < nk; kt0 += NPF) {
#pragma unroll
    for (int p = 0; p < NPF; ++p) {
    const int kt = kt0 + p;
    if (kt >= nk) break;
    const int cur = kt & 1;
#pragma unroll
    for (int ks = 0; ks < kGemmBK / 32; ++ks) {
      uint4 af[FT];
      uint4 bfrag[TT];
#pragma unroll
      for (int i = 0; i < FT; ++i)
        af[i] = *reinterpret_cast<const uint4*>(&lds[cur][wf * FW + 16 * i + r][32 * ks + 8 * g]);
#pragma unroll
      for (int j = 0; j < TT; ++j)
        bfrag[j] = *reinterpret_cast<const uint4*>(&lds[cur][BF + wt * TW + 16 * j + r][32 * ks + 8 * g]);
      // All of the k-step's fragment reads are issued before its MFMAs: left
      // to itself the scheduler reads one A fragment at a time, each behind
      // a wait for the previous one.
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < FT; ++i)
#pragma unroll
        for (int j = 0; j < TT; ++j) acc[i][j] = mfma_16x16x32(Bf16Tag{}, af[i], bfrag[j], acc[i][j]);
    }
    // Buffer cur ^ 1 was last read in the previous iteration, before the
    // barrier every thread has passed since.
    store_stage(cur ^ 1, stage[p]);
    load_stage(min(kt + 1 + NPF, nk - 1), stage[p]);
    __syncthreads();
    }
  }

  // Output: lane (r, g) of tile (i, j) holds features f0 + wf * FW + 16 i +
  // 4 g + e (e < 4) of token t0 + wt * TW + 16 j + r.
  const BufferRsrc outr = make_buffer(a.out, (uint32_t)(((int64_t)(a.tokens - 1) * a.out_stride + a.features) * 2));
  const int fw0 = f0 + wf * FW;
  // Tile i holds dims 16 (i % 8) .. of its head (FW = 64: the wave's first
  // tile starts at dim 0 or 64); tiles of dims 0..31 rotate with tile i + 2.
  auto rotates = [&](int i) { return (((fw0 + 16 * i) % 128) / 16) < 2; };
#pragma unroll
  for (int j = 0; j < TT; ++j) {
    const int t = t0 + wt * TW + 16 * j + r;
    float v[FT][4];
#pragma unroll
    for (int i = 0; i < FT; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) v[i][e] = round_bf16f(acc[i][j][e]);  // the projection, as bf16
    if constexpr (kRope) {
      const uint32_t* cs = a.rope + (size_t)min(t, a.tokens - 1) * kRopeHalf;
#pragma unroll
      for (int i = 0; i + 2 < FT; ++i) {
        if (!rotates(i)) continue;  // uniform across the wave
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t p = cs[16 * (i % 2) + 4 * g + e];
          const float c = __uint_as_float(p & 0xffff0000u);
          const float s = __uint_as_float(p << 16);
          const float x1 = v[i][e];
          const float x2 = v[i + 2][e];
          v[i][e] = round_bf16f(round_bf16f(x1 * c) - round_bf16f(x2 * s));
          v[i + 2][e] = round_bf16f(round_bf16f(x2 * c) + round_bf16f(x1 * s));
        }
      }
    }
#pragma unroll
    for (int i = 0; i < FT; ++i) {
      const int f = fw0 + 16 * i + 4 * g;
      const uint32_t lo = (__float_as_uint(v[i][0]) >> 16) | (__float_as_uint(v[i][1]) & 0xffff0000u);
      const uint32_t hi = (__float_as_uint(v[i][2]) >> 16) | (__float_as_uint(v[i][3]) & 0xffff0000u);
      const uint32_t off = (t < a.tokens && f < a.features) ? (uint32_t)(((int64_t)t * a.out_stride + f) * 2) : kFar;
      buffer_store_u64(outr, off, ((uint64_t)hi << 32) | lo);
    }
  }
}

// fp32 weights: a workgroup owns 64 features x 16 tokens and its four waves
// split k in four; each wave loads its MFMA operands straight from memory
// (both are read from L2 many times over, by the token tiles and the
// feature tiles).  For a chunk of 16 k, lane (r, g) loads weight row r and
// token r at k = 16 q + 4 g .. + 3 (16 and 8 or 16 bytes) and feeds element
// j to k-step j of v_mfma_f32_16x16x4_f32: both operands use that same
// order of k, so the product is the plain sum.  kAhead chunks are in flight
// per wave.  The four partial sums are added in LDS in a fixed order.
constexpr int kF32Feat = 64;
constexpr int kF32Tok = 16;
constexpr int kF32Ahead = 8;

__global__ __launch_bounds__(256) void gemm_f32_kernel(GemmArgs a) {
  __shared__ float red[4][64][17];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int feature_tiles = (a.features + kF32Feat - 1) / kF32Feat;
  const int f0 = (int)(blockIdx.x % (uint32_t)feature_tiles) * kF32Feat;
  const int t0 = (int)(blockIdx.x / (uint32_t)feature_tiles) * kF32Tok;
  const int kdim = a.kdim;
  const int chunks = (kdim + 15) / 16;
  const int per = (chunks + 3) / 4;  // chunks of this wave: [wave * per, min(chunks, wave * per + per))
  const int q0 = wave * per;
  const int q1 = min(chunks, q0 + per);
  const int hbytes = a.hidden_f32 ? 4 : 2;
  const BufferRsrc wr = make_buffer(a.weight, (uint32_t)a.features * (uint32_t)kdim * 4u);
  const BufferRsrc hr =
      make_buffer(a.hidden, (uint32_t)(((int64_t)(a.tokens - 1) * a.hidden_stride + kdim) * hbytes));
  uint32_t wbase[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int f = f0 + 16 * i + r;
    wbase[i] = f < a.features ? (uint32_t)f * (uint32_t)kdim * 4u : kFar;
  }
  const int t = t0 + r;
  const uint32_t hbase = t < a.tokens ? (uint32_t)((int64_t)t * a.hidden_stride * hbytes) : kFar;
  auto load = [&](int q, uint4 (&wv)[4], float (&hv)[4]) {
    const int k = 16 * q + 4 * g;
    const bool in = q < q1 && k < kdim;  // kdim % 4 == 0: a lane's 4 values are all in or all out
#pragma unroll
    for (int i = 0; i < 4; ++i) wv[i] = buffer_load_16(wr, in && wbase[i] != kFar ? wbase[i] + (uint32_t)k * 4u : kFar);
    const uint32_t hoff = in && hbase != kFar ? hbase + (uint32_t)k * (uint32_t)hbytes : kFar;
    if (a.hidden_f32) {
      const uint4 v = buffer_load_16(hr, hoff);
      hv[0] = __uint_as_float(v.x);
      hv[1] = __uint_as_float(v.y);
      hv[2] = __uint_as_float(v.z);
      hv[3] = __uint_as_float(v.w);
    } else {
      const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(hr, (int)hoff, 0, 0);
      hv[0] = __uint_as_float(v.x << 16);
      hv[1] = __uint_as_float(v.x & 0xffff0000u);
      hv[2] = __uint_as_float(v.y << 16);
      hv[3] = __uint_as_float(v.y & 0xffff0000u);
    }
  };
  floatx4 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  uint4 wv[kF32Ahead][4];
  float hv[kF32Ahead][4];
#pragma unroll
  for (int s = 0; s < kF32Ahead; ++s) load(q0 + s, wv[s], hv[s]);
  for (int q = q0; q < q1; q += kF32Ahead) {
#pragma unroll
    for (int s = 0; s < kF32Ahead; ++s) {
      // chunk q + s is in registers; chunks past q1 read zeros
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float b = hv[s][j];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t wbits = j == 0 ? wv[s][i].x : j == 1 ? wv[s][i].y : j == 2 ? wv[s][i].z : wv[s][i].w;
          acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(wbits), b, acc[i], 0, 0, 0);
        }
      }
      load(q + s + kF32Ahead, wv[s], hv[s]);
    }
  }
  // Lane (r, g) of tile i holds features f0 + 16 i + 4 g + e of token t0 + r.
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) red[wave][lane][4 * i + e] = acc[i][e];
  __syncthreads();
  if (wave == 0 && t < a.tokens) {
    float* out = static_cast<float*>(a.out) + (int64_t)t * a.out_stride;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int f = f0 + 16 * i + 4 * g + e;
        const float sum = ((red[0][lane][4 * i + e] + red[1][lane][4 * i + e]) + red[2][lane][4 * i + e]) +
                          red[3][lane][4 * i + e];
        if (f < a.features) out[f] = sum * a.scale;
      }
  }
}

template <int BF, int BT, int WF, int WT, bool kRope, int NPF>
int launch_bf16(const GemmArgs& a, hipStream_t stream) {
  const int64_t grid = (int64_t)((a.features + BF - 1) / BF) * ((a.tokens + BT - 1) / BT);
  if (grid > 0x7fffffffLL) return fail(DSA_STATUS_INVALID_ARGUMENT, "problem too large");
  hipLaunchKernelGGL((gemm_bf16_kernel<BF, BT, WF, WT, kRope, NPF>), dim3((unsigned)grid), dim3(64 * WF * WT), 0,
                     stream, a);
  return check_launch("gemm_bf16_kernel");
}

}  // namespace
}  // namespace dsa

using namespace dsa;

extern "C" int64_t dsa_project_gemm_workspace_bytes(int64_t tokens) {
  return tokens > 0 ? tokens * kRopeHalf * (int64_t)sizeof(uint32_t) : 0;
}

extern "C" int dsa_project_gemm(const void* hidden, int32_t hidden_dtype, int64_t hidden_stride, int64_t tokens,
                                int64_t kdim, const void* weight, int32_t weight_dtype, int64_t features, void* out,
                                int64_t out_stride, float out_scale, const int64_t* positions, float theta,
                                void* workspace, int64_t workspace_bytes, void* stream) {
  DSA_REQUIRE(hidden && weight && out, "null pointer argument");
  DSA_REQUIRE(tokens > 0 && tokens <= 0x7fffffffLL, "tokens %lld out of range", (long long)tokens);
  DSA_REQUIRE(kdim > 0 && kdim % 8 == 0, "kdim %lld must be a positive multiple of 8", (long long)kdim);
  DSA_REQUIRE(features > 0 && features % 4 == 0, "features %lld must be a positive multiple of 4",
              (long long)features);
  DSA_REQUIRE(hidden_stride >= kdim && hidden_stride % 8 == 0, "hidden_stride must be >= kdim and a multiple of 8");
  DSA_REQUIRE(out_stride >= features && out_stride % 4 == 0, "out_stride must be >= features and a multiple of 4");
  DSA_REQUIRE(reinterpret_cast<uintptr_t>(hidden) % 16 == 0 && reinterpret_cast<uintptr_t>(weight) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(out) % 16 == 0,
              "hidden, weight and out must be 16-byte aligned");
  DSA_REQUIRE(hidden_dtype == kBF16 || (hidden_dtype == kF32 && weight_dtype == kF32),
              "hidden must be bf16 (or fp32 with fp32 weights)");
  DSA_REQUIRE(weight_dtype == kBF16 || weight_dtype == kF32, "weights must be bf16 or fp32");
  const int64_t hidden_bytes = ((tokens - 1) * hidden_stride + kdim) * (hidden_dtype == kF32 ? 4 : 2);
  const int64_t out_bytes = ((tokens - 1) * out_stride + features) * (weight_dtype == kF32 ? 4 : 2);
  DSA_REQUIRE(hidden_bytes < (int64_t(1) << 31) && out_bytes < (int64_t(1) << 31) &&
                  features * kdim * (weight_dtype == kF32 ? 4 : 2) < (int64_t(1) << 31),
              "hidden, weight and out must each be below 2 GiB");
  GemmArgs a = {};
  a.hidden = static_cast<const uint16_t*>(hidden);
  a.hidden_stride = hidden_stride;
  a.weight = weight;
  a.out = out;
  a.out_stride = out_stride;
  a.tokens = (int32_t)tokens;
  a.features = (int32_t)features;
  a.kdim = (int32_t)kdim;
  a.hidden_f32 = hidden_dtype == kF32 ? 1 : 0;
  a.scale = out_scale;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (weight_dtype == kF32) {
    DSA_REQUIRE(!positions, "the fused RoPE takes bf16 weights");
    DSA_REQUIRE(kdim % 4 == 0 && hidden_stride % 4 == 0, "fp32 projections need kdim and hidden_stride divisible by 4");
    const int64_t grid = ((features + kF32Feat - 1) / kF32Feat) * ((tokens + kF32Tok - 1) / kF32Tok);
    DSA_REQUIRE(grid <= 0x7fffffffLL, "problem too large");
    hipLaunchKernelGGL(gemm_f32_kernel, dim3((unsigned)grid), dim3(256), 0, s, a);
    return check_launch("gemm_f32_kernel");
  }
  DSA_REQUIRE(out_scale == 1.f, "bf16 projections take no output scale");
  if (positions) {
    // Query projection with the fused RoPE of every 128-dim head.
    DSA_REQUIRE(features % 256 == 0, "the fused RoPE needs whole pairs of 128-dim heads (features a multiple of 256)");
    DSA_REQUIRE(workspace && workspace_bytes >= dsa_project_gemm_workspace_bytes(tokens) &&
                    reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
                "the fused RoPE needs dsa_project_gemm_workspace_bytes(tokens) bytes of 16-byte aligned workspace");
    a.rope = static_cast<const uint32_t*>(workspace);
    const int64_t entries = tokens * kRopeHalf;
    hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((entries + 255) / 256)), dim3(256), 0, s, positions,
                       (int32_t)tokens, theta, static_cast<uint32_t*>(workspace));
    if (int st = check_launch("rope_table_kernel")) return st;
    return launch_bf16<256, 256, 2, 4, true, 1>(a, s);
  }
  if (features % 256 == 0 && tokens >= 1024) return launch_bf16<256, 256, 2, 4, false, 1>(a, s);
  return launch_bf16<128, 32, 2, 2, false, 4>(a, s);
}
