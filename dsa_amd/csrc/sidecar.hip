// Sidecar encoder epilogues (reference sidecar.py:10-88).
//
// encode_keys is k_norm(wk(hidden)) then the non-interleaved RoPE on the
// first rope_dim dims; encode_queries is the RoPE on each head of
// wq(hidden), plus weights_proj(hidden) * (heads * head_dim)^-0.5.  The
// projections are plain GEMMs left to the platform BLAS; everything after
// them runs here in one pass per row, reading the projection once and
// writing the encoded row straight to its destination (for keys, a KV-cache
// row given per token), where the reference chains a LayerNorm, slices,
// six elementwise products/sums and a concatenation.
//
// Arithmetic follows torch's per-op rounding in the row's dtype: in bf16,
// cos/sin are rounded to bf16 and every product and sum of the rotation is
// rounded to bf16; in fp32 no product is fused into a sum.  LayerNorm
// computes in fp32 (biased variance, eps inside the rsqrt) and rounds once
// to the row dtype.
#include "common.hpp"
#include "status.hpp"

namespace dsa {
namespace {

constexpr int kMaxRowDim = 256;  // dims per row a wave holds (4 per lane, in two adjacent pairs)

// fp32 -> nearest-even bf16, returned as fp32 (the value a torch bf16 op stores).
__device__ __forceinline__ float round_bf16(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return x;  // NaN passes through
  u += 0x7fffu + ((u >> 16) & 1u);
  return __uint_as_float(u & 0xffff0000u);
}

__device__ __forceinline__ float load_elem(const void* p, int64_t i, bool bf16) {
  if (bf16) return __uint_as_float(uint32_t(static_cast<const uint16_t*>(p)[i]) << 16);
  return static_cast<const float*>(p)[i];
}

__device__ __forceinline__ void store_elem(void* p, int64_t i, float v, bool bf16) {
  if (bf16)
    static_cast<uint16_t*>(p)[i] = (uint16_t)(__float_as_uint(round_bf16(v)) >> 16);
  else
    static_cast<float*>(p)[i] = v;
}

struct EncodeArgs {
  const void* in;          // [tokens][heads][dim], in_dtype
  int64_t in_row_stride;   // elements between tokens
  void* out;               // [rows of out][heads][dim], out_dtype
  int64_t out_row_stride;  // elements between output rows
  const int64_t* out_rows; // nullable: output row of each token (cache append)
  int64_t out_row_limit;   // rows of the output; a token whose row is outside is not written
  const int64_t* positions;  // [tokens]
  const float* ln_weight;  // nullable (no LayerNorm) else [dim]
  const float* ln_bias;    // [dim]
  float ln_eps;
  const float* w_in;       // nullable: [tokens][heads] fp32 head weights
  float* w_out;            // [tokens][heads]
  float w_scale;
  int64_t tokens;
  int32_t heads;
  int32_t dim;
  int32_t rope_dim;
  float theta;
  int32_t in_bf16;
  int32_t out_bf16;
};

// Two adjacent elements of a row, as fp32.
__device__ __forceinline__ float2 load_pair(const void* p, int64_t i, bool bf16) {
  if (bf16) {
    const uint32_t v = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(p) + i);
    return make_float2(__uint_as_float(v << 16), __uint_as_float(v & 0xffff0000u));
  }
  return *reinterpret_cast<const float2*>(static_cast<const float*>(p) + i);
}

__device__ __forceinline__ void store_pair(void* p, int64_t i, float2 v, bool bf16) {
  if (bf16) {
    const uint32_t lo = __float_as_uint(round_bf16(v.x)) >> 16;
    const uint32_t hi = __float_as_uint(round_bf16(v.y)) & 0xffff0000u;
    *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(p) + i) = lo | hi;
  } else {
    *reinterpret_cast<float2*>(static_cast<float*>(p) + i) = v;
  }
}

// Each wave encodes G rows of one token: with one head per token (keys) the
// four waves of a workgroup take tokens 4b .. 4b + 3; with several heads the
// workgroup is (token, group of 4 G heads) and wave w takes heads
// 4 G group + w + 4 j, j < G.  A wave computes its token's rotation table
// (cos / sin of its position times each inv_freq, rounded to the row dtype)
// into its own LDS rows and issues all of its row loads before using any.
// Lane l holds dims 2l, 2l + 1, 128 + 2l, 129 + 2l of a row (pairs of
// adjacent elements are loaded and stored together).
template <int G, bool kInBf16, bool kOutBf16>
__global__ __launch_bounds__(256) void encode_rows_kernel(EncodeArgs a) {
  __shared__ float part[4][kMaxRowDim];
  __shared__ float cos_t[4][kMaxRowDim / 2];
  __shared__ float sin_t[4][kMaxRowDim / 2];
  constexpr bool in_bf16 = kInBf16;
  constexpr bool out_bf16 = kOutBf16;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const bool per_wave_token = a.heads == 1;
  const int64_t token = per_wave_token ? (int64_t)blockIdx.x * 4 + wave : (int64_t)blockIdx.x;
  if (token >= a.tokens) return;
  const int head0 = per_wave_token ? 0 : (int)blockIdx.y * 4 * G + wave;
  const int dim = a.dim;
  const int half = a.rope_dim / 2;
  auto dim_of = [&](int e) { return 128 * (e >> 1) + 2 * lane + (e & 1); };

  // Every load is issued before any is used: addresses are clamped into the
  // row (head and dim), the values past it are never stored.
  float x[G][4];
#pragma unroll
  for (int j = 0; j < G; ++j) {
    const int head = min(head0 + 4 * j, a.heads - 1);
    const int64_t in0 = token * a.in_row_stride + (int64_t)head * dim;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int d = min(128 * p + 2 * lane, dim - 2);
      const float2 v = load_pair(a.in, in0 + d, in_bf16);
      x[j][2 * p] = v.x;
      x[j][2 * p + 1] = v.y;
    }
  }
#pragma unroll
  for (int j = 0; j < G; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (dim_of(e) >= dim) x[j][e] = 0.f;

  const float pos = (float)a.positions[token];
  for (int i = lane; i < half; i += kWave) {
    // inv_freq_i = theta ^ (-i / half), angle = position * inv_freq_i (fp32).
    const float angle = pos * powf(a.theta, -(float)i / (float)half);
    const float c = cosf(angle);
    const float s = sinf(angle);
    cos_t[wave][i] = out_bf16 ? round_bf16(c) : c;
    sin_t[wave][i] = out_bf16 ? round_bf16(s) : s;
  }
  const int64_t out_row = a.out_rows ? a.out_rows[token] : token;
  const bool write = out_row >= 0 && out_row < a.out_row_limit;  // rows outside the output are skipped

#pragma unroll
  for (int j = 0; j < G; ++j) {
    const int head = head0 + 4 * j;
    if (head >= a.heads) break;
    float (&y)[4] = x[j];
    if (a.ln_weight) {
      float sum = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) sum += y[e];
      for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, kWave);
      const float mean = sum / (float)dim;
      float sq = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float c = dim_of(e) < dim ? y[e] - mean : 0.f;
        sq = fmaf(c, c, sq);
      }
      for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off, kWave);
      const float rstd = 1.f / sqrtf(sq / (float)dim + a.ln_eps);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int d = dim_of(e);
        if (d < dim) {
          const float v = __fadd_rn(__fmul_rn(__fmul_rn(y[e] - mean, rstd), a.ln_weight[d]), a.ln_bias[d]);
          y[e] = out_bf16 ? round_bf16(v) : v;
        }
      }
    } else if (out_bf16 && !in_bf16) {
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = round_bf16(y[e]);
    }

    // Rotation of the pairs (i, i + half) through this wave's LDS rows.
    if (half > 0) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (dim_of(e) < dim) part[wave][dim_of(e)] = y[e];
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int d = dim_of(e);
        if (d >= 2 * half) continue;
        const int i = d < half ? d : d - half;
        const float c = cos_t[wave][i];
        const float s = sin_t[wave][i];
        const float first = part[wave][i];
        const float second = part[wave][i + half];
        if (out_bf16) {
          y[e] = d < half ? round_bf16(round_bf16(first * c) - round_bf16(second * s))
                          : round_bf16(round_bf16(second * c) + round_bf16(first * s));
        } else {
          y[e] = d < half ? __fsub_rn(__fmul_rn(first, c), __fmul_rn(second, s))
                          : __fadd_rn(__fmul_rn(second, c), __fmul_rn(first, s));
        }
      }
      // the next row's stores to part[wave] wait until every lane has read it
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    }

    if (write) {
      const int64_t out0 = out_row * a.out_row_stride + (int64_t)head * dim;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int d = 128 * p + 2 * lane;
        if (d < dim) store_pair(a.out, out0 + d, make_float2(y[2 * p], y[2 * p + 1]), out_bf16);
      }
    }
    if (a.w_in && lane == 0) a.w_out[token * a.heads + head] = a.w_in[token * a.heads + head] * a.w_scale;
  }
}

int check_encode(const EncodeArgs& a, int32_t in_dtype, int32_t out_dtype) {
  DSA_REQUIRE(a.in && a.out && a.positions, "null pointer argument");
  DSA_REQUIRE(a.tokens >= 0 && a.heads > 0, "tokens/heads out of range");
  DSA_REQUIRE(a.dim > 0 && a.dim <= kMaxRowDim && a.dim % 2 == 0, "dim %d must be even and at most %d", a.dim,
              kMaxRowDim);
  DSA_REQUIRE(a.heads <= 4 * 65535, "too many heads");
  DSA_REQUIRE(a.tokens <= 0x7fffffffLL, "too many tokens");
  DSA_REQUIRE(a.in_row_stride % 2 == 0 && a.out_row_stride % 2 == 0, "row strides must be even");
  DSA_REQUIRE(a.rope_dim >= 0 && a.rope_dim <= a.dim && a.rope_dim % 2 == 0,
              "rope_dim must be even and no larger than dim");
  DSA_REQUIRE(in_dtype == kF32 || in_dtype == kBF16, "rows must be fp32 or bf16 (got %d)", in_dtype);
  DSA_REQUIRE(out_dtype == kF32 || out_dtype == kBF16, "outputs must be fp32 or bf16 (got %d)", out_dtype);
  return 0;
}

int launch_encode(const EncodeArgs& a, hipStream_t stream) {
  if (a.tokens == 0) return 0;
  if (a.tokens > 0x7fffffffLL) return fail(DSA_STATUS_INVALID_ARGUMENT, "too many tokens");
  // Few tokens (a decode step): one head per wave, for parallelism; many
  // (prefill): sixteen heads per wave, so a workgroup's table and launch
  // serve 64 heads.
  // One head per token: four tokens per workgroup.  Several heads: few
  // tokens (a decode step) take one head per wave for parallelism, many
  // (prefill) sixteen, so that a wave's loads and table serve 16 rows.
  const bool one = a.heads == 1;
  const bool many = !one && a.tokens >= 256;
  const dim3 grid(one ? (unsigned)((a.tokens + 3) / 4) : (unsigned)a.tokens,
                  one ? 1u : (unsigned)(many ? (a.heads + 63) / 64 : (a.heads + 3) / 4));
  auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, dim3(256), 0, stream, a); };
  const int combo = (a.in_bf16 ? 2 : 0) | (a.out_bf16 ? 1 : 0);
  switch (combo | (many ? 4 : 0)) {
    case 0: go(encode_rows_kernel<1, false, false>); break;
    case 1: go(encode_rows_kernel<1, false, true>); break;
    case 2: go(encode_rows_kernel<1, true, false>); break;
    case 3: go(encode_rows_kernel<1, true, true>); break;
    case 4: go(encode_rows_kernel<16, false, false>); break;
    case 5: go(encode_rows_kernel<16, false, true>); break;
    case 6: go(encode_rows_kernel<16, true, false>); break;
    default: go(encode_rows_kernel<16, true, true>); break;
  }
  return check_launch("encode_rows_kernel");
}

}  // namespace
}  // namespace dsa

using namespace dsa;

extern "C" int dsa_rope(const void* x, void* out, const int64_t* positions, int64_t tokens, int32_t heads,
                        int32_t dim, int32_t rope_dim, float theta, int32_t dtype, void* stream) {
  EncodeArgs a = {};
  a.in = x;
  a.in_row_stride = (int64_t)heads * dim;
  a.out = out;
  a.out_row_stride = (int64_t)heads * dim;
  a.out_row_limit = tokens;
  a.positions = positions;
  a.tokens = tokens;
  a.heads = heads;
  a.dim = dim;
  a.rope_dim = rope_dim;
  a.theta = theta;
  a.in_bf16 = a.out_bf16 = dtype == kBF16;
  if (int st = check_encode(a, dtype, dtype)) return st;
  return launch_encode(a, static_cast<hipStream_t>(stream));
}

extern "C" int dsa_encode_keys_epilogue(const void* proj, int32_t proj_dtype, int64_t proj_row_stride,
                                        const float* ln_weight, const float* ln_bias, float ln_eps,
                                        const int64_t* positions, int32_t rope_dim, float theta, void* out,
                                        int32_t out_dtype, int64_t out_row_stride, const int64_t* out_rows,
                                        int64_t out_row_limit, int64_t tokens, int32_t dim, void* stream) {
  DSA_REQUIRE(ln_weight && ln_bias, "null pointer argument");
  EncodeArgs a = {};
  a.in = proj;
  a.in_row_stride = proj_row_stride;
  a.out = out;
  a.out_row_stride = out_row_stride;
  a.out_rows = out_rows;
  a.out_row_limit = out_rows ? out_row_limit : tokens;
  a.positions = positions;
  a.ln_weight = ln_weight;
  a.ln_bias = ln_bias;
  a.ln_eps = ln_eps;
  a.tokens = tokens;
  a.heads = 1;
  a.dim = dim;
  a.rope_dim = rope_dim;
  a.theta = theta;
  a.in_bf16 = proj_dtype == kBF16;
  a.out_bf16 = out_dtype == kBF16;
  if (int st = check_encode(a, proj_dtype, out_dtype)) return st;
  DSA_REQUIRE(proj_row_stride >= dim && out_row_stride >= dim, "row strides must cover dim");
  return launch_encode(a, static_cast<hipStream_t>(stream));
}

extern "C" int dsa_encode_queries_epilogue(const void* proj, const float* proj_weights, const int64_t* positions,
                                           int32_t rope_dim, float theta, float weight_scale, void* out,
                                           float* out_weights, int64_t tokens, int32_t heads, int32_t dim,
                                           int32_t dtype, void* stream) {
  DSA_REQUIRE(proj_weights && out_weights, "null pointer argument");
  EncodeArgs a = {};
  a.in = proj;
  a.in_row_stride = (int64_t)heads * dim;
  a.out = out;
  a.out_row_stride = (int64_t)heads * dim;
  a.out_row_limit = tokens;
  a.positions = positions;
  a.w_in = proj_weights;
  a.w_out = out_weights;
  a.w_scale = weight_scale;
  a.tokens = tokens;
  a.heads = heads;
  a.dim = dim;
  a.rope_dim = rope_dim;
  a.theta = theta;
  a.in_bf16 = a.out_bf16 = dtype == kBF16;
  if (int st = check_encode(a, dtype, dtype)) return st;
  return launch_encode(a, static_cast<hipStream_t>(stream));
}
