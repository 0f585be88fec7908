// Decode-path expert kernels: fused MXFP4-dequant GEMV for gate_up (+ bias +
// clamped SwiGLU) and down (+ bias), the weighted combine, and the one-call
// MoE layer (gfx950).
//
// GEMV mapping.  A workgroup owns one 64-row tile of one active expert's
// matrix (packed row-tile layout, see klc_common.h) and all tokens routed to
// that expert.  Its 4 waves split the input groups; in each step every lane
// loads 16 bytes = 32 E2M1 codes of its own row, so a wave-wide load is 1 KiB
// of contiguous HBM.  Codes are decoded in registers with
// v_cvt_scalef32_pk_f32_fp4; the activation slice of a group is the same for
// all 64 lanes, so it is read through the scalar path and each weight is used
// by every token of the expert straight from registers.  Per group the 32
// products are summed and scaled once by 2^(e-127).  Wave partials are summed
// in wave order through LDS, then wave 0 applies bias (+ SwiGLU on the
// interleaved gate/up lane pairs) and writes fp32 results.
#include "klc_common.h"

namespace klc {

int launch_router_logits(const void* x, const void* w, const void* b, void* logits, float* x_f32, int64_t n_tok,
                         int64_t hidden, int64_t n_exp, hipStream_t stream);
int launch_topk(const void* logits, int32_t* ids, float* values, void* weights, int64_t n_tok, int64_t n_exp,
                int64_t k, hipStream_t stream);
int launch_dispatch(const int32_t* ids, int64_t n_pairs, int64_t n_exp, int32_t* offsets, int32_t* sorted,
                    int32_t* active, int32_t* n_active, hipStream_t stream);
int check_router_args(int64_t n_tok, int64_t hidden, int64_t n_exp);
int check_topk_args(int64_t n_tok, int64_t n_exp, int64_t k);
int check_dispatch_args(int64_t n_pairs, int64_t n_exp);

namespace {

constexpr int kGemvWaves = 4;                 // 4 x 16 rows = one 64-row tile per workgroup
constexpr int kGemvThreads = kGemvWaves * kWave;
constexpr int kVRows = 8;                     // activation rows (MFMA N columns) staged per pass
constexpr int kMaxSteps = 24;                 // 4-group steps per row (inputs <= 3072)

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// Expert matrices arrive through a pointer table; they live in global memory.
typedef const uint8_t __attribute__((address_space(1)))* global_u8_ptr;
typedef const u32x4 __attribute__((address_space(1)))* global_u32x4_ptr;
typedef const uint32_t __attribute__((address_space(1)))* global_u32_ptr;

// 2^(e-127) as the float32 scale operand of v_cvt_scalef32_pk_bf16_fp4; the
// conversion is exact for e = 0..254 (e = 0 is a float32 subnormal).
__device__ __forceinline__ float cvt_scale(uint32_t e) {
  return __uint_as_float(e == 0u ? 0x00400000u : (e == 255u ? 0x7f800000u : (e << 23)));
}

// Eight E2M1 codes (one dword, input order) times the scale -> 8 bf16 (MFMA A operand).
__device__ __forceinline__ bf16x8_t decode8(uint32_t word, float scale) {
  const bf16x2_t p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 0);
  const bf16x2_t p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 1);
  const bf16x2_t p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 2);
  const bf16x2_t p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 3);
  return __builtin_shufflevector(__builtin_shufflevector(p0, p1, 0, 1, 2, 3),
                                 __builtin_shufflevector(p2, p3, 0, 1, 2, 3), 0, 1, 2, 3, 4, 5, 6, 7);
}

__device__ __forceinline__ float swiglu(float gate, float up, float limit) {
  // streamed_moe_router.py:524-529; comparisons keep NaN like torch.clamp
  gate = gate > limit ? limit : gate;
  up = up > limit ? limit : (up < -limit ? -limit : up);
  const float glu = gate * (1.0f / (1.0f + expf(-(gate * 1.702f))));
  return (up + 1.0f) * glu;
}

__device__ __forceinline__ uint16_t bf16_bits_rne(float f) { return (uint16_t)f32_to_bf16_rne(f); }

// Expert GEMV on MFMA.  Workgroup = (64-row tile, active expert); wave w owns
// rows [16w, 16w + 16) of the tile over the whole input dimension.  Per
// 4-group step a lane holds the 16 code bytes of (row l % 16, group 4s + l/16)
// -- exactly the A operand of four v_mfma_f32_16x16x32_bf16 (k = 8 * (l/16) + i)
// once decoded -- and the B operand is read from the activations staged in
// LDS as bfloat16 rows (the same k mapping).  Columns are up to kVRows
// activation rows: gate_up stages one row per token (x is bfloat16, exact);
// down stages hi = bf16(g) and lo = bf16(g - hi) per token so the float32
// SwiGLU output enters the product with a 2^-17 relative residual.
template <bool kDown>
__global__ __launch_bounds__(kGemvThreads) void moe_gemv_mfma_kernel(
    const uint8_t* const* __restrict__ wptr, const uint16_t* __restrict__ bias, const void* __restrict__ act,
    float* __restrict__ out, float* __restrict__ out_raw, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ pairs, const int32_t* __restrict__ active, const int32_t* __restrict__ n_active,
    int rows, int groups, int k_top, float limit, int precision) {
  extern __shared__ uint16_t xs[];  // [kVRows][row_stride] bfloat16 bits

  const int u = blockIdx.y;
  if (u >= *n_active) return;
  const int e = active[u];
  const int pb = offsets[e];
  const int np = offsets[e + 1] - pb;
  const int tile = blockIdx.x;
  const int tiles = rows / kTileRows;
  const int g4 = (groups + 3) >> 2;             // 4-group steps
  const int in_dim = groups * 32;
  const int row_stride = g4 * 128 + 8;          // bf16 elements per staged row (zero padded)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int lr = lane & 15;                     // row within the wave's 16 (A) / column n (B, D)
  const int lq = lane >> 4;                     // k-quarter: group 4s + lq

  // ---- issue all weight loads of this lane first ----
  const global_u8_ptr mat = (global_u8_ptr)wptr[e];
  const int trow = wave * 16 + lr;              // row inside the 64-row tile
  const global_u8_ptr blk = mat + (int64_t)tile * groups * 1024 + trow * 16;
  const global_u8_ptr scl = mat + (int64_t)tiles * groups * 1024 + (int64_t)tile * g4 * 256 + trow * 4;
  u32x4 wv[kMaxSteps];
  uint32_t sv[kMaxSteps];
#pragma unroll
  for (int s = 0; s < kMaxSteps; ++s) {
    if (s < g4) {
      const int g = 4 * s + lq;
      wv[s] = g < groups ? *(global_u32x4_ptr)(blk + (int64_t)g * 1024) : u32x4{0u, 0u, 0u, 0u};
      sv[s] = *(global_u32_ptr)(scl + (int64_t)s * 256);
    }
  }

  const int tok_per_pass = kDown ? kVRows / 2 : kVRows;
  for (int tc = 0; tc < np; tc += tok_per_pass) {
    const int nt = min(tok_per_pass, np - tc);
    const int nrows = kDown ? 2 * nt : nt;
    // ---- stage activation rows (bf16) into LDS ----
    __syncthreads();  // previous pass finished reading xs
    if constexpr (!kDown) {
      const uint16_t* x = static_cast<const uint16_t*>(act);
      const int chunks = in_dim / 8;            // 16-byte chunks per row
      for (int i = threadIdx.x; i < nrows * chunks; i += kGemvThreads) {
        const int r = i / chunks, c = i - r * chunks;
        const int tok = pairs[pb + tc + r] / k_top;
        *reinterpret_cast<uint4*>(xs + r * row_stride + c * 8) =
            *reinterpret_cast<const uint4*>(x + (int64_t)tok * in_dim + c * 8);
      }
    } else {
      const float* g = static_cast<const float*>(act);
      const int chunks = in_dim / 4;            // 4 floats per thread-step
      for (int i = threadIdx.x; i < nt * chunks; i += kGemvThreads) {
        const int t = i / chunks, c = i - t * chunks;
        const float4 v = *reinterpret_cast<const float4*>(g + (int64_t)pairs[pb + tc + t] * in_dim + c * 4);
        const float f[4] = {v.x, v.y, v.z, v.w};
        uint32_t hi[2], lo[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint16_t h0 = bf16_bits_rne(f[2 * h]), h1 = bf16_bits_rne(f[2 * h + 1]);
          const uint16_t l0 = bf16_bits_rne(f[2 * h] - bf16_to_f32(h0));
          const uint16_t l1 = bf16_bits_rne(f[2 * h + 1] - bf16_to_f32(h1));
          hi[h] = (uint32_t)h0 | ((uint32_t)h1 << 16);
          lo[h] = (uint32_t)l0 | ((uint32_t)l1 << 16);
        }
        *reinterpret_cast<uint2*>(xs + (2 * t) * row_stride + c * 4) = make_uint2(hi[0], hi[1]);
        *reinterpret_cast<uint2*>(xs + (2 * t + 1) * row_stride + c * 4) = make_uint2(lo[0], lo[1]);
      }
    }
    // zero the padding beyond in_dim (its A operand is zero; keep 0 * pad finite)
    const int pad = g4 * 128 - in_dim;
    for (int i = threadIdx.x; i < nrows * pad; i += kGemvThreads) {
      const int r = i / pad;
      xs[r * row_stride + in_dim + (i - r * pad)] = 0;
    }
    __syncthreads();

    // ---- MFMA main loop ----
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const bool has_col = lr < nrows;
    const uint16_t* xrow = xs + lr * row_stride + lq * 32;
#pragma unroll
    for (int s = 0; s < kMaxSteps; ++s) {
      if (s < g4) {
        const float scale = cvt_scale((sv[s] >> (8 * lq)) & 0xffu);
        const uint32_t words[4] = {wv[s].x, wv[s].y, wv[s].z, wv[s].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const bf16x8_t a = decode8(words[j], scale);
          bf16x8_t b = {};
          if (has_col) b = *reinterpret_cast<const bf16x8_t*>(xrow + s * 128 + j * 8);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
        }
      }
    }

    // ---- epilogue: lane holds rows 4*lq + v (v = 0..3) of the wave's 16, column lr ----
    const int row0 = tile * kTileRows + wave * 16 + 4 * lq;
    float v[4] = {acc[0], acc[1], acc[2], acc[3]};
    if constexpr (!kDown) {
      if (lr < nt) {
        const int pair = pairs[pb + tc + lr];
        const int half = rows >> 1;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float gate = v[2 * h], up = v[2 * h + 1];
          if (precision == KLC_PRECISION_BF16) {
            gate = round_bf16(gate);
            up = round_bf16(up);
          }
          gate += bf16_to_f32(bias[(int64_t)e * rows + row0 + 2 * h]);
          up += bf16_to_f32(bias[(int64_t)e * rows + row0 + 2 * h + 1]);
          const float y = swiglu(gate, up, limit);
          const int64_t idx = (int64_t)pair * half + (row0 >> 1) + h;
          if (out_raw) out_raw[idx] = y;
          out[idx] = precision == KLC_PRECISION_BF16 ? round_bf16(y) : y;
        }
      }
    } else {
      // column 2t holds the hi part of token t, column 2t + 1 the lo part
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] += __shfl_xor(v[i], 1);
      if ((lr & 1) == 0 && (lr >> 1) < nt) {
        const int pair = pairs[pb + tc + (lr >> 1)];
        float o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float t = precision == KLC_PRECISION_BF16 ? round_bf16(v[i]) : v[i];
          o[i] = t + bf16_to_f32(bias[(int64_t)e * rows + row0 + i]);
        }
        *reinterpret_cast<float4*>(out + (int64_t)pair * rows + row0) = make_float4(o[0], o[1], o[2], o[3]);
      }
    }
  }
}

size_t gemv_lds_bytes(int groups) { return (size_t)kVRows * (((groups + 3) / 4) * 128 + 8) * 2; }

// out[t][h] over k slots in order; every step rounded to bfloat16.
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ eo, const uint16_t* __restrict__ w,
                                                      int k, int hidden, uint16_t* __restrict__ out) {
  const int t = blockIdx.y;
  const int h = blockIdx.x * blockDim.x + threadIdx.x;
  if (h >= hidden) return;
  float acc = 0.0f;
  for (int j = 0; j < k; ++j) {
    const int64_t p = (int64_t)t * k + j;
    const float wj = bf16_to_f32(w[p]);
    const float o = round_bf16(eo[p * hidden + h]);
    acc = round_bf16(acc + round_bf16(o * wj));
  }
  out[(int64_t)t * hidden + h] = (uint16_t)f32_to_bf16_rne(acc);
}

__global__ __launch_bounds__(256) void bias_combine_kernel(const uint16_t* __restrict__ bias,
                                                           const int32_t* __restrict__ ids,
                                                           const uint16_t* __restrict__ w, int k, int hidden,
                                                           uint16_t* __restrict__ out) {
  const int t = blockIdx.y;
  const int h = blockIdx.x * blockDim.x + threadIdx.x;
  if (h >= hidden) return;
  float acc = 0.0f;
  for (int j = 0; j < k; ++j) {
    const int64_t p = (int64_t)t * k + j;
    acc += round_bf16(bf16_to_f32(bias[(int64_t)ids[p] * hidden + h]) * bf16_to_f32(w[p]));
  }
  out[(int64_t)t * hidden + h] = (uint16_t)f32_to_bf16_rne(acc);
}

__global__ __launch_bounds__(256) void pair_norms_kernel(const float* __restrict__ gated,
                                                         const float* __restrict__ eo, int n_pairs, int inter,
                                                         int hidden, float* __restrict__ norms) {
  const int p = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (p >= n_pairs) return;
  double sg = 0.0, so = 0.0;
  for (int i = lane; i < inter; i += kWave) {
    const double v = gated[(int64_t)p * inter + i];
    sg += v * v;
  }
  for (int i = lane; i < hidden; i += kWave) {
    const double v = eo[(int64_t)p * hidden + i];
    so += v * v;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    sg += __shfl_xor(sg, off);
    so += __shfl_xor(so, off);
  }
  if (lane == 0) {
    norms[2 * p] = (float)sqrt(sg);
    norms[2 * p + 1] = (float)sqrt(so);
  }
}

int check_gemv_shapes(int64_t hidden, int64_t inter, int64_t max_active) {
  KLC_REQUIRE(hidden > 0 && inter > 0 && max_active > 0, KLC_ERR_ARGUMENT,
              "experts: bad sizes hidden=%lld inter=%lld max_active=%lld", (long long)hidden, (long long)inter,
              (long long)max_active);
  KLC_REQUIRE(hidden % 64 == 0 && inter % 32 == 0 && (2 * inter) % 64 == 0, KLC_ERR_SHAPE,
              "experts: hidden=%lld must be a multiple of 64 and inter=%lld a multiple of 32", (long long)hidden,
              (long long)inter);
  KLC_REQUIRE(max_active <= 65535 && hidden <= 32 * 4 * kMaxSteps && inter <= 32 * 4 * kMaxSteps,
              KLC_ERR_UNSUPPORTED, "experts: unsupported sizes (hidden, inter <= %d)", 32 * 4 * kMaxSteps);
  return KLC_OK;
}

int launch_gate_up(const void* const* w, const void* bias, const void* x, int64_t k, const int32_t* offsets,
                   const int32_t* pairs, const int32_t* active, const int32_t* n_active, int64_t max_active,
                   int64_t hidden, int64_t inter, float limit, int precision, float* gated, float* gated_raw,
                   hipStream_t stream) {
  const dim3 grid((unsigned)(2 * inter / kTileRows), (unsigned)max_active);
  moe_gemv_mfma_kernel<false><<<grid, kGemvThreads, gemv_lds_bytes((int)(hidden / 32)), stream>>>(
      reinterpret_cast<const uint8_t* const*>(w), static_cast<const uint16_t*>(bias), x, gated, gated_raw,
      offsets, pairs, active, n_active, (int)(2 * inter), (int)(hidden / 32), (int)k, limit, precision);
  return check_launch("moe_gemv_mfma_kernel<gate_up>");
}

int launch_down(const void* const* w, const void* bias, const float* gated, const int32_t* offsets,
                const int32_t* pairs, const int32_t* active, const int32_t* n_active, int64_t max_active,
                int64_t hidden, int64_t inter, int precision, float* eo, hipStream_t stream) {
  const dim3 grid((unsigned)(hidden / kTileRows), (unsigned)max_active);
  moe_gemv_mfma_kernel<true><<<grid, kGemvThreads, gemv_lds_bytes((int)(inter / 32)), stream>>>(
      reinterpret_cast<const uint8_t* const*>(w), static_cast<const uint16_t*>(bias), gated, eo, nullptr, offsets,
      pairs, active, n_active, (int)hidden, (int)(inter / 32), 1, 0.0f, precision);
  return check_launch("moe_gemv_mfma_kernel<down>");
}

int launch_combine(const float* eo, const void* w, int64_t n_tok, int64_t k, int64_t hidden, void* out,
                   hipStream_t stream) {
  const dim3 grid((unsigned)((hidden + 255) / 256), (unsigned)n_tok);
  combine_kernel<<<grid, 256, 0, stream>>>(eo, static_cast<const uint16_t*>(w), (int)k, (int)hidden,
                                           static_cast<uint16_t*>(out));
  return check_launch("combine_kernel");
}

inline int64_t align256(int64_t v) { return (v + 255) & ~(int64_t)255; }

struct LayerScratch {
  int64_t logits, ids, values, weights, offsets, sorted, active, n_active, gated, eo, total;
};

LayerScratch layer_scratch(int64_t n_tok, int64_t hidden, int64_t inter, int64_t n_exp, int64_t k) {
  LayerScratch s{};
  const int64_t pairs = n_tok * k;
  int64_t off = 0;
  s.logits = off;   off += align256(n_tok * n_exp * 2);
  s.ids = off;      off += align256(pairs * 4);
  s.values = off;   off += align256(pairs * 4);
  s.weights = off;  off += align256(pairs * 2);
  s.offsets = off;  off += align256((n_exp + 1) * 4);
  s.sorted = off;   off += align256(pairs * 4);
  s.active = off;   off += align256(n_exp * 4);
  s.n_active = off; off += align256(4);
  s.gated = off;    off += align256(pairs * inter * 4);
  s.eo = off;       off += align256(pairs * hidden * 4);
  s.total = off;
  return s;
}

}  // namespace
}  // namespace klc

using namespace klc;

extern "C" int klc_moe_gate_up(const void* const* w_gate_up, const void* bias, const void* x, int64_t k,
                               const int32_t* offsets, const int32_t* sorted_pairs, const int32_t* active,
                               const int32_t* n_active, int64_t max_active, int64_t hidden, int64_t inter,
                               float swiglu_limit, int precision, float* gated, float* gated_raw, void* stream) {
  KLC_REQUIRE(w_gate_up && bias && x && offsets && sorted_pairs && active && n_active && gated, KLC_ERR_ARGUMENT,
              "klc_moe_gate_up: null pointer");
  KLC_REQUIRE(k > 0, KLC_ERR_ARGUMENT, "klc_moe_gate_up: k=%lld", (long long)k);
  KLC_REQUIRE(precision == KLC_PRECISION_FP32 || precision == KLC_PRECISION_BF16, KLC_ERR_ARGUMENT,
              "klc_moe_gate_up: unknown precision %d", precision);
  const int rc = check_gemv_shapes(hidden, inter, max_active);
  if (rc) return rc;
  return launch_gate_up(w_gate_up, bias, x, k, offsets, sorted_pairs, active, n_active, max_active, hidden, inter,
                        swiglu_limit, precision, gated, gated_raw, as_stream(stream));
}

extern "C" int klc_moe_down(const void* const* w_down, const void* bias, const float* gated, const int32_t* offsets,
                            const int32_t* sorted_pairs, const int32_t* active, const int32_t* n_active,
                            int64_t max_active, int64_t hidden, int64_t inter, int precision, float* expert_out,
                            void* stream) {
  KLC_REQUIRE(w_down && bias && gated && offsets && sorted_pairs && active && n_active && expert_out,
              KLC_ERR_ARGUMENT, "klc_moe_down: null pointer");
  KLC_REQUIRE(precision == KLC_PRECISION_FP32 || precision == KLC_PRECISION_BF16, KLC_ERR_ARGUMENT,
              "klc_moe_down: unknown precision %d", precision);
  const int rc = check_gemv_shapes(hidden, inter, max_active);
  if (rc) return rc;
  return launch_down(w_down, bias, gated, offsets, sorted_pairs, active, n_active, max_active, hidden, inter,
                     precision, expert_out, as_stream(stream));
}

extern "C" int klc_moe_combine(const float* expert_out, const void* weights, int64_t n_tokens, int64_t k,
                               int64_t hidden, void* out, void* stream) {
  KLC_REQUIRE(expert_out && weights && out, KLC_ERR_ARGUMENT, "klc_moe_combine: null pointer");
  KLC_REQUIRE(n_tokens > 0 && k > 0 && hidden > 0, KLC_ERR_ARGUMENT, "klc_moe_combine: bad sizes");
  KLC_REQUIRE(n_tokens <= 65535, KLC_ERR_UNSUPPORTED, "klc_moe_combine: n_tokens=%lld > 65535", (long long)n_tokens);
  return launch_combine(expert_out, weights, n_tokens, k, hidden, out, as_stream(stream));
}

extern "C" int klc_moe_bias_combine(const void* down_bias, const int32_t* ids, const void* weights, int64_t n_tokens,
                                    int64_t k, int64_t hidden, void* out, void* stream) {
  KLC_REQUIRE(down_bias && ids && weights && out, KLC_ERR_ARGUMENT, "klc_moe_bias_combine: null pointer");
  KLC_REQUIRE(n_tokens > 0 && k > 0 && hidden > 0, KLC_ERR_ARGUMENT, "klc_moe_bias_combine: bad sizes");
  KLC_REQUIRE(n_tokens <= 65535, KLC_ERR_UNSUPPORTED, "klc_moe_bias_combine: n_tokens=%lld > 65535",
              (long long)n_tokens);
  const dim3 grid((unsigned)((hidden + 255) / 256), (unsigned)n_tokens);
  bias_combine_kernel<<<grid, 256, 0, as_stream(stream)>>>(static_cast<const uint16_t*>(down_bias), ids,
                                                           static_cast<const uint16_t*>(weights), (int)k,
                                                           (int)hidden, static_cast<uint16_t*>(out));
  return check_launch("bias_combine_kernel");
}

extern "C" int klc_moe_pair_norms(const float* gated, const float* expert_out, int64_t n_pairs, int64_t inter,
                                  int64_t hidden, float* norms, void* stream) {
  KLC_REQUIRE(gated && expert_out && norms, KLC_ERR_ARGUMENT, "klc_moe_pair_norms: null pointer");
  KLC_REQUIRE(n_pairs > 0 && inter > 0 && hidden > 0, KLC_ERR_ARGUMENT, "klc_moe_pair_norms: bad sizes");
  KLC_REQUIRE(n_pairs < ((int64_t)1 << 30), KLC_ERR_UNSUPPORTED, "klc_moe_pair_norms: too many pairs");
  pair_norms_kernel<<<(unsigned)((n_pairs + 3) / 4), 256, 0, as_stream(stream)>>>(gated, expert_out, (int)n_pairs,
                                                                                  (int)inter, (int)hidden, norms);
  return check_launch("pair_norms_kernel");
}

extern "C" int64_t klc_moe_workspace_bytes(int64_t n_tokens, int64_t hidden, int64_t inter, int64_t n_experts,
                                           int64_t k) {
  if (n_tokens <= 0 || hidden <= 0 || inter <= 0 || n_experts <= 0 || k <= 0)
    return set_error(KLC_ERR_ARGUMENT, "klc_moe_workspace_bytes: bad sizes");
  return layer_scratch(n_tokens, hidden, inter, n_experts, k).total;
}

extern "C" int klc_moe_layer(const void* x, const void* router_w, const void* router_b, const void* const* w_gate_up,
                             const void* gate_up_bias, const void* const* w_down, const void* down_bias,
                             int64_t n_tokens, int64_t hidden, int64_t inter, int64_t n_experts, int64_t k,
                             float swiglu_limit, int precision, void* workspace, int64_t workspace_bytes, void* out,
                             int32_t* ids, void* weights, void* const* events, void* stream) {
  KLC_REQUIRE(x && router_w && router_b && w_gate_up && gate_up_bias && w_down && down_bias && workspace && out,
              KLC_ERR_ARGUMENT, "klc_moe_layer: null pointer");
  KLC_REQUIRE(precision == KLC_PRECISION_FP32 || precision == KLC_PRECISION_BF16, KLC_ERR_ARGUMENT,
              "klc_moe_layer: unknown precision %d", precision);
  int rc = check_router_args(n_tokens, hidden, n_experts);
  if (rc) return rc;
  rc = check_topk_args(n_tokens, n_experts, k);
  if (rc) return rc;
  rc = check_dispatch_args(n_tokens * k, n_experts);
  if (rc) return rc;
  const int64_t max_active = n_experts < n_tokens * k ? n_experts : n_tokens * k;
  rc = check_gemv_shapes(hidden, inter, max_active);
  if (rc) return rc;
  KLC_REQUIRE(n_tokens <= 65535, KLC_ERR_UNSUPPORTED, "klc_moe_layer: n_tokens=%lld > 65535", (long long)n_tokens);
  const LayerScratch s = layer_scratch(n_tokens, hidden, inter, n_experts, k);
  KLC_REQUIRE(workspace_bytes >= s.total, KLC_ERR_ARGUMENT, "klc_moe_layer: workspace of %lld bytes < %lld needed",
              (long long)workspace_bytes, (long long)s.total);
  KLC_REQUIRE(((uintptr_t)workspace & 255) == 0, KLC_ERR_ARGUMENT, "klc_moe_layer: workspace must be 256-byte aligned");

  char* ws = static_cast<char*>(workspace);
  void* logits = ws + s.logits;
  int32_t* ids_buf = ids ? ids : reinterpret_cast<int32_t*>(ws + s.ids);
  float* values = reinterpret_cast<float*>(ws + s.values);
  void* w_buf = weights ? weights : static_cast<void*>(ws + s.weights);
  int32_t* offsets = reinterpret_cast<int32_t*>(ws + s.offsets);
  int32_t* sorted = reinterpret_cast<int32_t*>(ws + s.sorted);
  int32_t* active = reinterpret_cast<int32_t*>(ws + s.active);
  int32_t* n_active = reinterpret_cast<int32_t*>(ws + s.n_active);
  float* gated = reinterpret_cast<float*>(ws + s.gated);
  float* eo = reinterpret_cast<float*>(ws + s.eo);
  hipStream_t st = as_stream(stream);
  auto mark = [&](int i) -> int {
    if (events == nullptr) return KLC_OK;
    const hipError_t err = hipEventRecord(static_cast<hipEvent_t>(events[i]), st);
    return err == hipSuccess ? KLC_OK : set_error(KLC_ERR_HIP, "klc_moe_layer: hipEventRecord: %s", hipGetErrorString(err));
  };

  if ((rc = mark(0))) return rc;
  if ((rc = launch_router_logits(x, router_w, router_b, logits, nullptr, n_tokens, hidden, n_experts, st))) return rc;
  if ((rc = mark(1))) return rc;
  if ((rc = launch_topk(logits, ids_buf, values, w_buf, n_tokens, n_experts, k, st))) return rc;
  if ((rc = mark(2))) return rc;
  if ((rc = launch_dispatch(ids_buf, n_tokens * k, n_experts, offsets, sorted, active, n_active, st))) return rc;
  if ((rc = mark(3))) return rc;
  if ((rc = launch_gate_up(w_gate_up, gate_up_bias, x, k, offsets, sorted, active, n_active, max_active, hidden,
                           inter, swiglu_limit, precision, gated, nullptr, st)))
    return rc;
  if ((rc = mark(4))) return rc;
  if ((rc = launch_down(w_down, down_bias, gated, offsets, sorted, active, n_active, max_active, hidden, inter,
                        precision, eo, st)))
    return rc;
  if ((rc = mark(5))) return rc;
  if ((rc = launch_combine(eo, w_buf, n_tokens, k, hidden, out, st))) return rc;
  return mark(6);
}
