// Prefill path: expert-grouped GEMM on MFMA (gfx950).
//
// For batches that give experts many tokens, each expert's weights are read
// once per 64-token unit and multiplied into all of the unit's tokens:
// a workgroup owns one GEMM unit (up to 64 tokens of one expert, from the
// dispatch) and 256 output rows (4 waves, each one 64-row packed tile, i.e.
// 4 row blocks of 16).  Per 128-deep k step every wave decodes its A chunks
// (MXFP4 -> bfloat16 with v_cvt_scalef32_pk_bf16_fp4, exact) and multiplies
// them with v_mfma_f32_16x16x32_bf16 into each 16-token column block of B,
// which the workgroup stages in LDS (double buffered; global loads issued two
// steps ahead) from the token rows.  A chunks stream from HBM two steps ahead.  The products are exact and the
// sums run in float32, like the decode GEMVs, so both paths meet the same
// tolerance; gate_up reads the bfloat16 hidden state as is, down reads the
// float32 SwiGLU output as hi + lo bfloat16 planes (relative residual 2^-17).
//
// (The scaled FP4 MFMA, v_mfma_scale_f32_16x16x128_f8f6f4 with FP8 hi/lo
// activations, takes the weights in their own format but forms its
// 128-term sums with less than float32 precision: measured on gfx950 it
// misses exact sums by up to 4e-5 of the sum of |terms|, which at 2880-deep
// rows exceeds the 1e-2 absolute tolerance on small outputs.)
//
// Operand layouts (v_mfma_f32_16x16x32_bf16): A lane l = row l % 16,
// k = 8 (l / 16) + i; B lane l = column l % 16, same k; D lane l register v =
// row 4 (l / 16) + v, column l % 16.  A step of 4 MX groups is four MFMAs:
// MFMA j takes dword j of every lane's 16-byte chunk (group 4s + l/16), so
// its k set is {128 s + 32 q + 8 j + i}; the B lane (column n, q) reads those
// 8 activations of its token.
#include "klc_common.h"

namespace klc {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kGemmThreads = 256;
constexpr int kGemmWaves = 4;
constexpr int kGemmRows = kGemmWaves * kTileRows;   // 256 output rows per workgroup
constexpr int kGemmCb = kUnitTokensGemm / 16;       // 8 column blocks of 16 tokens
constexpr int kRowBytes = 128 * 2 + 16;             // one token's 128 bfloat16 of a step, padded (bank spread)
constexpr int kPlaneBytes = kUnitTokensGemm * kRowBytes;
constexpr int kPieces = kUnitTokensGemm * 16 / kGemmThreads;  // 16-byte pieces per thread per plane and step
constexpr int kXcds = 8;  // accelerator complex dies of an MI355X, each with its own L2

__device__ __forceinline__ float swiglu(float gate, float up, float limit) {
  // streamed_moe_router.py:524-529; comparisons keep NaN like torch.clamp
  gate = gate > limit ? limit : gate;
  up = up > limit ? limit : (up < -limit ? -limit : up);
  const float glu = gate * (1.0f / (1.0f + expf(-(gate * 1.702f))));
  return (up + 1.0f) * glu;
}

// One GEMM unit x one 256-row tile.  gate_up: act = bfloat16 hidden state
// [n_tok][in], one plane; writes the down input as hi/lo bfloat16 planes
// [2][pairs][in_down] (and float32 SwiGLU output to out_raw if set).  down:
// act = those planes (rows by pair); writes float32 expert outputs.
template <bool kDown>
__global__ __launch_bounds__(kGemmThreads) void moe_gemm_kernel(
    const uint8_t* const* __restrict__ wptr, const uint16_t* __restrict__ bias, const uint16_t* __restrict__ act,
    int64_t act_plane, float* __restrict__ out, uint16_t* __restrict__ out_split, int64_t out_plane,
    float* __restrict__ out_raw, const int32_t* __restrict__ offsets, const int32_t* __restrict__ pairs,
    const int32_t* __restrict__ units, const int32_t* __restrict__ n_units, int rows, int groups, int k_top,
    float limit, int precision, int row_wgs, int units_per_xcd) {
  constexpr int kPlanes = kDown ? 2 : 1;
  constexpr int kStage = kPlanes * kPlaneBytes;
  extern __shared__ __align__(16) uint8_t stage[];  // 2 x kStage

  // XCD-aware order: workgroups are handed to the 8 XCDs round-robin, so XCD
  // x = blockIdx.x % 8 runs units x, x + 8, ...; all row tiles of a unit run on
  // one XCD, which reads the unit's activation rows into its own L2 once.
  const int xcd = blockIdx.x % kXcds;
  const int j = blockIdx.x / kXcds;
  const int u = xcd + kXcds * (j / row_wgs);
  const int row_wg = j % row_wgs;
  if (j >= units_per_xcd * row_wgs || u >= *n_units) return;
  const int32_t unit = units[u];
  const int e = unit_expert(unit);
  const int pb = offsets[e];
  const int tc = unit_pass(unit) * kUnitTokensGemm;
  const int nt = min(kUnitTokensGemm, offsets[e + 1] - pb - tc);
  const int ncb = (nt + 15) >> 4;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int lr = lane & 15;
  const int lq = lane >> 4;
  const int tiles = rows / kTileRows;
  const int tile = row_wg * kGemmWaves + wave;
  const bool wave_live = tile < tiles;
  const int in_dim = groups * 32;
  const int steps = (groups + 3) >> 2;

  // ---- staging: thread moves pieces (plane, token c = (tid >> 4) + 16 i, 8 values at 8 o), o = tid & 15 ----
  const int so = tid & 15;
  int64_t src_row[kPieces];
#pragma unroll
  for (int i = 0; i < kPieces; ++i) {
    const int c = min((tid >> 4) + 16 * i, nt - 1);
    const int p = pairs[pb + tc + c];
    src_row[i] = (int64_t)(kDown ? p : p / k_top) * in_dim;
  }
  auto stage_load = [&](int s, u32x4_t* pv) {
    const int kc = min(s * 128 + so * 8, in_dim - 8);
#pragma unroll
    for (int i = 0; i < kPieces * kPlanes; ++i)
      pv[i] = *reinterpret_cast<const u32x4_t*>(act + (i / kPieces) * act_plane + src_row[i % kPieces] + kc);
  };
  auto stage_store = [&](int s, int buf, const u32x4_t* pv) {
    uint8_t* base = stage + buf * kStage;
    const bool k_ok = s * 128 + so * 8 < in_dim;
#pragma unroll
    for (int i = 0; i < kPieces * kPlanes; ++i) {
      const int c = (tid >> 4) + 16 * (i % kPieces);
      const u32x4_t z = {0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4_t*>(base + (i / kPieces) * kPlaneBytes + c * kRowBytes + so * 16) =
          (k_ok && c < nt) ? pv[i] : z;
    }
  };

  // ---- A stream: the wave's 64-row tile, 4 row blocks, two steps ahead ----
  const int wtile = wave_live ? tile : 0;
  const __amdgpu_buffer_rsrc_t wbuf = __builtin_amdgcn_make_buffer_rsrc(
      (void*)wptr[e], (short)0, (int)packed_matrix_bytes(rows, groups), kBufferWord3);
  const uint32_t tile_off = (uint32_t)wtile * (uint32_t)groups * 1024u;
  const int rec = (int)packed_scale_record(groups);
  const uint32_t scale_base = (uint32_t)packed_block_bytes(rows, groups);
  auto a_load = [&](int s, u32x4_t* a, uint32_t* sw) {
    const bool ok = 4 * s + lq < groups;
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const uint32_t v = ok ? (uint32_t)(lq * 1024 + (rb * 16 + lr) * 16) : kOutOfRange;
      a[rb] = __builtin_amdgcn_raw_buffer_load_b128(wbuf, v, tile_off + 4096u * s, 0);
      const uint32_t r = (uint32_t)((wtile * kTileRows + rb * 16 + lr) * 4 + lq);
      sw[rb] = __builtin_amdgcn_raw_buffer_load_b32(wbuf, r * (uint32_t)rec + (uint32_t)(s & ~3), scale_base, 0);
    }
  };

  f32x4_t acc[4][kGemmCb];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
#pragma unroll
    for (int cb = 0; cb < kGemmCb; ++cb) acc[rb][cb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // activation staging: two register sets, loads issued two steps ahead;
  // LDS double buffered
  u32x4_t pva[kPieces * kPlanes], pvb[kPieces * kPlanes];
  u32x4_t a_cur[4], a_nxt[4];
  uint32_t s_cur[4], s_nxt[4];
  stage_load(0, pva);
  a_load(0, a_cur, s_cur);
  if (steps > 1) a_load(1, a_nxt, s_nxt);
  if (steps > 1) stage_load(1, pvb);
  stage_store(0, 0, pva);
  __syncthreads();

  // one k step: stage s + 2 is loaded into `ld` (free since stage s was
  // stored), stage s + 1 (loaded a step ago, in `st`) goes to LDS
  auto step = [&](int s, u32x4_t* ld, const u32x4_t* st) {
    const int buf = s & 1;
    if (s + 2 < steps) stage_load(s + 2, ld);
    if (wave_live) {
      // per quarter j of the step: decode the 4 row blocks' A operands, then
      // multiply them into every column block (row blocks innermost, so
      // consecutive MFMAs update different accumulators)
      const bool live = 4 * s + lq < groups;
      float scale[4];
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) scale[rb] = cvt_scale_operand((s_cur[rb] >> (8 * (s & 3))) & 0xffu, live);
      const uint8_t* base = stage + buf * kStage + lr * kRowBytes + lq * 64;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bf16x8_t a[4];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) a[rb] = decode8(a_cur[rb][j], scale[rb]);
#pragma unroll
        for (int cb = 0; cb < kGemmCb; ++cb) {
          if (cb < ncb) {
#pragma unroll
            for (int pl = 0; pl < kPlanes; ++pl) {
              const bf16x8_t b =
                  *reinterpret_cast<const bf16x8_t*>(base + pl * kPlaneBytes + cb * 16 * kRowBytes + j * 16);
#pragma unroll
              for (int rb = 0; rb < 4; ++rb)
                acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[rb], b, acc[rb][cb], 0, 0, 0);
            }
          }
        }
      }
    }
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      a_cur[rb] = a_nxt[rb];
      s_cur[rb] = s_nxt[rb];
    }
    if (s + 2 < steps) a_load(s + 2, a_nxt, s_nxt);
    if (s + 1 < steps) stage_store(s + 1, buf ^ 1, st);
    __syncthreads();
  };
  for (int s = 0; s < steps; s += 2) {
    step(s, pva, pvb);
    if (s + 1 < steps) step(s + 1, pvb, pva);
  }

  if (!wave_live) return;
  // ---- epilogue: lane holds rows rb * 16 + 4 lq + v of the tile, token column cb * 16 + lr ----
#pragma unroll
  for (int cb = 0; cb < kGemmCb; ++cb) {
    if (cb >= ncb) continue;
    const int c = cb * 16 + lr;
    if (c >= nt) continue;
    const int p = pairs[pb + tc + c];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const int row0 = tile * kTileRows + rb * 16 + 4 * lq;
      const f32x4_t v4 = acc[rb][cb];
      if constexpr (!kDown) {
        const int half = rows >> 1;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float gate = v4[2 * h], up = v4[2 * h + 1];
          if (precision == KLC_PRECISION_BF16) {
            gate = round_bf16(gate);
            up = round_bf16(up);
          }
          gate += bf16_to_f32(bias[(int64_t)e * rows + row0 + 2 * h]);
          up += bf16_to_f32(bias[(int64_t)e * rows + row0 + 2 * h + 1]);
          const float y = swiglu(gate, up, limit);
          const int64_t idx = (int64_t)p * half + (row0 >> 1) + h;
          if (out_raw) out_raw[idx] = y;
          const uint32_t hi = f32_to_bf16_rne(y);
          const uint32_t lo = precision == KLC_PRECISION_BF16 ? 0u : f32_to_bf16_rne(y - bf16_to_f32(hi));
          out_split[idx] = (uint16_t)hi;
          out_split[out_plane + idx] = (uint16_t)lo;
        }
      } else {
        float o[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float t = precision == KLC_PRECISION_BF16 ? round_bf16(v4[v]) : v4[v];
          o[v] = t + bf16_to_f32(bias[(int64_t)e * rows + row0 + v]);
        }
        *reinterpret_cast<float4*>(out + (int64_t)p * rows + row0) = make_float4(o[0], o[1], o[2], o[3]);
      }
    }
  }
}

}  // namespace

int launch_gemm_gate_up(const void* const* w, const void* bias, const void* x, int64_t n_tok, int64_t k,
                        int64_t n_exp, const int32_t* offsets, const int32_t* pairs, const int32_t* units,
                        int64_t hidden, int64_t inter, float limit, int precision, void* gated_split,
                        float* gated_raw, hipStream_t stream) {
  const int64_t n_pairs = n_tok * k;
  const int64_t rows = 2 * inter;
  const int row_wgs = (int)((rows + kGemmRows - 1) / kGemmRows);
  const int per_xcd = (int)((units_capacity(n_pairs, n_exp, kUnitTokensGemm) + kXcds - 1) / kXcds);
  const dim3 grid((unsigned)(kXcds * per_xcd * row_wgs));
  moe_gemm_kernel<false><<<grid, kGemmThreads, 2 * kPlaneBytes, stream>>>(
      reinterpret_cast<const uint8_t* const*>(w), static_cast<const uint16_t*>(bias), static_cast<const uint16_t*>(x),
      0, nullptr, static_cast<uint16_t*>(gated_split), n_pairs * inter, gated_raw, offsets, pairs,
      units + units_offset_gemm(n_pairs, n_exp), units + 2, (int)rows, (int)(hidden / 32), (int)k, limit, precision,
      row_wgs, per_xcd);
  return check_launch("moe_gemm_kernel<gate_up>");
}

int launch_gemm_down(const void* const* w, const void* bias, const void* gated_split, int64_t n_pairs, int64_t n_exp,
                     const int32_t* offsets, const int32_t* pairs, const int32_t* units, int64_t hidden, int64_t inter,
                     int precision, float* eo, hipStream_t stream) {
  const int row_wgs = (int)((hidden + kGemmRows - 1) / kGemmRows);
  const int per_xcd = (int)((units_capacity(n_pairs, n_exp, kUnitTokensGemm) + kXcds - 1) / kXcds);
  const dim3 grid((unsigned)(kXcds * per_xcd * row_wgs));
  moe_gemm_kernel<true><<<grid, kGemmThreads, 2 * 2 * kPlaneBytes, stream>>>(
      reinterpret_cast<const uint8_t* const*>(w), static_cast<const uint16_t*>(bias),
      static_cast<const uint16_t*>(gated_split), n_pairs * inter, eo, nullptr, 0, nullptr, offsets, pairs,
      units + units_offset_gemm(n_pairs, n_exp), units + 2, (int)hidden, (int)(inter / 32), 1, 0.0f, precision,
      row_wgs, per_xcd);
  return check_launch("moe_gemm_kernel<down>");
}

int check_gemv_shapes(int64_t hidden, int64_t inter, int64_t n_pairs, int64_t n_exp);

}  // namespace klc

using namespace klc;

extern "C" int klc_moe_gemm_gate_up(const void* const* w_gate_up, const void* bias, const void* x, int64_t n_tokens,
                                    int64_t k, int64_t n_experts, const int32_t* offsets, const int32_t* sorted_pairs,
                                    const int32_t* units, int64_t hidden, int64_t inter, float swiglu_limit,
                                    int precision, void* gated_split, float* gated_raw, void* stream) {
  KLC_REQUIRE(w_gate_up && bias && x && offsets && sorted_pairs && units && gated_split, KLC_ERR_ARGUMENT,
              "klc_moe_gemm_gate_up: null pointer");
  KLC_REQUIRE(n_tokens > 0 && k > 0, KLC_ERR_ARGUMENT, "klc_moe_gemm_gate_up: n_tokens=%lld k=%lld",
              (long long)n_tokens, (long long)k);
  KLC_REQUIRE(precision == KLC_PRECISION_FP32 || precision == KLC_PRECISION_BF16, KLC_ERR_ARGUMENT,
              "klc_moe_gemm_gate_up: unknown precision %d", precision);
  const int rc = check_gemv_shapes(hidden, inter, n_tokens * k, n_experts);
  if (rc) return rc;
  return launch_gemm_gate_up(w_gate_up, bias, x, n_tokens, k, n_experts, offsets, sorted_pairs, units, hidden, inter,
                             swiglu_limit, precision, gated_split, gated_raw, as_stream(stream));
}

extern "C" int klc_moe_gemm_down(const void* const* w_down, const void* bias, const void* gated_split, int64_t n_pairs,
                                 int64_t n_experts, const int32_t* offsets, const int32_t* sorted_pairs,
                                 const int32_t* units, int64_t hidden, int64_t inter, int precision,
                                 float* expert_out, void* stream) {
  KLC_REQUIRE(w_down && bias && gated_split && offsets && sorted_pairs && units && expert_out, KLC_ERR_ARGUMENT,
              "klc_moe_gemm_down: null pointer");
  KLC_REQUIRE(n_pairs > 0, KLC_ERR_ARGUMENT, "klc_moe_gemm_down: n_pairs=%lld", (long long)n_pairs);
  KLC_REQUIRE(precision == KLC_PRECISION_FP32 || precision == KLC_PRECISION_BF16, KLC_ERR_ARGUMENT,
              "klc_moe_gemm_down: unknown precision %d", precision);
  const int rc = check_gemv_shapes(hidden, inter, n_pairs, n_experts);
  if (rc) return rc;
  return launch_gemm_down(w_down, bias, gated_split, n_pairs, n_experts, offsets, sorted_pairs, units, hidden, inter,
                          precision, expert_out, as_stream(stream));
}
