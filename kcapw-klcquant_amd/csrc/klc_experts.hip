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

constexpr int kGemvWaves = 4;
constexpr int kGemvThreads = kGemvWaves * kWave;
constexpr int kGemvTok = 4;   // tokens per pass over the weights
constexpr int kGemvBatch = 24;  // groups loaded per batch per wave (<= 96 VGPRs)

// The activations are read-only for the whole kernel and every lane of a wave
// reads the same slice, so they are addressed through the constant address
// space, which lets the compiler fetch them with scalar loads into SGPRs.
typedef const float __attribute__((address_space(4)))* const_f32_ptr;
// Expert matrices arrive through a pointer table; they live in global memory.
typedef const uint8_t __attribute__((address_space(1)))* global_u8_ptr;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef const u32x4 __attribute__((address_space(1)))* global_u32x4_ptr;
typedef const uint32_t __attribute__((address_space(1)))* global_u32_ptr;

// Decodes one 16-byte chunk (32 codes, input order) to float32.
__device__ __forceinline__ void decode_chunk(const u32x4& v, float* wf) {
  const uint32_t words[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float2 a = fp4x2_to_f32<0>(words[q]);
    float2 b = fp4x2_to_f32<1>(words[q]);
    float2 c = fp4x2_to_f32<2>(words[q]);
    float2 d = fp4x2_to_f32<3>(words[q]);
    wf[q * 8 + 0] = a.x; wf[q * 8 + 1] = a.y;
    wf[q * 8 + 2] = b.x; wf[q * 8 + 3] = b.y;
    wf[q * 8 + 4] = c.x; wf[q * 8 + 5] = c.y;
    wf[q * 8 + 6] = d.x; wf[q * 8 + 7] = d.y;
  }
}

__device__ __forceinline__ float swiglu(float gate, float up, float limit) {
  // streamed_moe_router.py:524-529; comparisons keep NaN like torch.clamp
  gate = gate > limit ? limit : gate;
  up = up > limit ? limit : (up < -limit ? -limit : up);
  const float glu = gate * (1.0f / (1.0f + expf(-(gate * 1.702f))));
  return (up + 1.0f) * glu;
}

template <bool kGateUp>
__global__ __launch_bounds__(kGemvThreads) void moe_gemv_kernel(
    const uint8_t* const* __restrict__ wptr, const uint16_t* __restrict__ bias, const float* __restrict__ act,
    float* __restrict__ out, float* __restrict__ out_raw, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ pairs, const int32_t* __restrict__ active, const int32_t* __restrict__ n_active,
    int rows, int groups, int k_top, float limit, int precision) {
  __shared__ float red[kGemvWaves][kGemvTok][kWave];

  const int u = blockIdx.y;
  if (u >= *n_active) return;
  const int e = active[u];
  const int pb = offsets[e];
  const int np = offsets[e + 1] - pb;
  const int tile = blockIdx.x;
  const int tiles = rows / kTileRows;
  const int g4 = (groups + 3) >> 2;
  const int in_dim = groups * 32;
  // wave index made provably uniform so group addressing stays scalar
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int g_lo = wave * groups / kGemvWaves;
  const int g_hi = (wave + 1) * groups / kGemvWaves;

  const global_u8_ptr mat = (global_u8_ptr)wptr[e];
  const global_u8_ptr blk = mat + (int64_t)tile * groups * 1024 + lane * 16;
  const global_u8_ptr scl = mat + (int64_t)tiles * groups * 1024 + (int64_t)tile * g4 * 256 + lane * 4;
  const int row = tile * kTileRows + lane;
  const float bias_v = bf16_to_f32(bias[(int64_t)e * rows + row]);

  for (int tc = 0; tc < np; tc += kGemvTok) {
    const int nt = min(kGemvTok, np - tc);
    const float* xrow[kGemvTok];
#pragma unroll
    for (int j = 0; j < kGemvTok; ++j) {
      const int pair = pairs[pb + tc + min(j, nt - 1)];
      const int src = kGateUp ? pair / k_top : pair;
      xrow[j] = act + (int64_t)src * in_dim;
    }
    float acc[kGemvTok];
#pragma unroll
    for (int j = 0; j < kGemvTok; ++j) acc[j] = 0.0f;

    for (int gb = g_lo; gb < g_hi; gb += kGemvBatch) {
      const int ng = min(kGemvBatch, g_hi - gb);
      u32x4 wv[kGemvBatch];
#pragma unroll
      for (int i = 0; i < kGemvBatch; ++i)
        if (i < ng) wv[i] = *(global_u32x4_ptr)(blk + (int64_t)(gb + i) * 1024);
#pragma unroll
      for (int i = 0; i < kGemvBatch; ++i) {
        if (i < ng) {
          const int g = gb + i;
          const uint32_t sw = *(global_u32_ptr)(scl + (int64_t)(g >> 2) * 256);
          const float s = e8m0_to_f32((sw >> ((g & 3) * 8)) & 0xffu);
          float wf[32];
          decode_chunk(wv[i], wf);
#pragma unroll
          for (int j = 0; j < kGemvTok; ++j) {
            if (j < nt) {
              const const_f32_ptr xr = (const_f32_ptr)(xrow[j] + g * 32);
              float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
              for (int q = 0; q < 32; q += 2) {
                a0 = fmaf(wf[q], xr[q], a0);
                a1 = fmaf(wf[q + 1], xr[q + 1], a1);
              }
              acc[j] = fmaf(a0 + a1, s, acc[j]);
            }
          }
        }
      }
    }

#pragma unroll
    for (int j = 0; j < kGemvTok; ++j) red[wave][j][lane] = acc[j];
    __syncthreads();
    if (wave == 0) {
      for (int j = 0; j < nt; ++j) {
        float v = red[0][j][lane];
#pragma unroll
        for (int w = 1; w < kGemvWaves; ++w) v += red[w][j][lane];
        if (precision == KLC_PRECISION_BF16) v = round_bf16(v);
        v += bias_v;
        const int pair = pairs[pb + tc + j];
        if constexpr (kGateUp) {
          const float up = __shfl_xor(v, 1);
          if ((lane & 1) == 0) {
            const float y = swiglu(v, up, limit);
            const int64_t idx = (int64_t)pair * (rows >> 1) + (row >> 1);
            if (out_raw) out_raw[idx] = y;
            out[idx] = precision == KLC_PRECISION_BF16 ? round_bf16(y) : y;
          }
        } else {
          out[(int64_t)pair * rows + row] = v;
        }
      }
    }
    __syncthreads();
  }
}

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
  KLC_REQUIRE(max_active <= 65535 && hidden < (1 << 24) && inter < (1 << 24), KLC_ERR_UNSUPPORTED,
              "experts: unsupported sizes");
  return KLC_OK;
}

int launch_gate_up(const void* const* w, const void* bias, const float* x_f32, int64_t k, const int32_t* offsets,
                   const int32_t* pairs, const int32_t* active, const int32_t* n_active, int64_t max_active,
                   int64_t hidden, int64_t inter, float limit, int precision, float* gated, float* gated_raw,
                   hipStream_t stream) {
  const dim3 grid((unsigned)(2 * inter / kTileRows), (unsigned)max_active);
  moe_gemv_kernel<true><<<grid, kGemvThreads, 0, stream>>>(
      reinterpret_cast<const uint8_t* const*>(w), static_cast<const uint16_t*>(bias), x_f32, gated, gated_raw,
      offsets, pairs, active, n_active, (int)(2 * inter), (int)(hidden / 32), (int)k, limit, precision);
  return check_launch("moe_gemv_kernel<gate_up>");
}

int launch_down(const void* const* w, const void* bias, const float* gated, const int32_t* offsets,
                const int32_t* pairs, const int32_t* active, const int32_t* n_active, int64_t max_active,
                int64_t hidden, int64_t inter, int precision, float* eo, hipStream_t stream) {
  const dim3 grid((unsigned)(hidden / kTileRows), (unsigned)max_active);
  moe_gemv_kernel<false><<<grid, kGemvThreads, 0, stream>>>(
      reinterpret_cast<const uint8_t* const*>(w), static_cast<const uint16_t*>(bias), gated, eo, nullptr, offsets,
      pairs, active, n_active, (int)hidden, (int)(inter / 32), 1, 0.0f, precision);
  return check_launch("moe_gemv_kernel<down>");
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
  int64_t logits, x_f32, ids, values, weights, offsets, sorted, active, n_active, gated, eo, total;
};

LayerScratch layer_scratch(int64_t n_tok, int64_t hidden, int64_t inter, int64_t n_exp, int64_t k) {
  LayerScratch s{};
  const int64_t pairs = n_tok * k;
  int64_t off = 0;
  s.logits = off;   off += align256(n_tok * n_exp * 2);
  s.x_f32 = off;    off += align256(n_tok * hidden * 4);
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

extern "C" int klc_moe_gate_up(const void* const* w_gate_up, const void* bias, const float* x_f32, int64_t k,
                               const int32_t* offsets, const int32_t* sorted_pairs, const int32_t* active,
                               const int32_t* n_active, int64_t max_active, int64_t hidden, int64_t inter,
                               float swiglu_limit, int precision, float* gated, float* gated_raw, void* stream) {
  KLC_REQUIRE(w_gate_up && bias && x_f32 && offsets && sorted_pairs && active && n_active && gated, KLC_ERR_ARGUMENT,
              "klc_moe_gate_up: null pointer");
  KLC_REQUIRE(k > 0, KLC_ERR_ARGUMENT, "klc_moe_gate_up: k=%lld", (long long)k);
  KLC_REQUIRE(precision == KLC_PRECISION_FP32 || precision == KLC_PRECISION_BF16, KLC_ERR_ARGUMENT,
              "klc_moe_gate_up: unknown precision %d", precision);
  const int rc = check_gemv_shapes(hidden, inter, max_active);
  if (rc) return rc;
  return launch_gate_up(w_gate_up, bias, x_f32, k, offsets, sorted_pairs, active, n_active, max_active, hidden, inter,
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
  float* x_f32 = reinterpret_cast<float*>(ws + s.x_f32);
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
  if ((rc = launch_router_logits(x, router_w, router_b, logits, x_f32, n_tokens, hidden, n_experts, st))) return rc;
  if ((rc = mark(1))) return rc;
  if ((rc = launch_topk(logits, ids_buf, values, w_buf, n_tokens, n_experts, k, st))) return rc;
  if ((rc = mark(2))) return rc;
  if ((rc = launch_dispatch(ids_buf, n_tokens * k, n_experts, offsets, sorted, active, n_active, st))) return rc;
  if ((rc = mark(3))) return rc;
  if ((rc = launch_gate_up(w_gate_up, gate_up_bias, x_f32, k, offsets, sorted, active, n_active, max_active, hidden,
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
