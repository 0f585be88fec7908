// Decode-path expert kernels: fused MXFP4-dequant GEMV for gate_up (+ bias +
// clamped SwiGLU) and down (+ bias), the weighted combine, and the one-call
// MoE layer (gfx950).
//
// GEMV mapping.  Tokens are grouped by expert (klc_moe_dispatch), and one
// workgroup streams a run of consecutive 64-row tiles of one active expert's
// packed matrix (row-tile layout, klc_common.h) for all tokens routed to that
// expert.  Codes are decoded in registers by v_cvt_scalef32_pk_bf16_fp4 (E2M1
// times the E8M0 scale, exact) straight into the A operand of
// v_mfma_f32_16x16x32_bf16; the B operand is the tokens' activation rows,
// staged once in LDS.  A workgroup serves one work unit: up to 8 (gate_up)
// or 4 (down) of the expert's tokens, so each weight byte is read from HBM
// once per unit however many of its tokens share it; an expert with more
// tokens has several units, run by separate workgroups side by side (see
// klc_common.h).  gate_up applies bias and the
// clamped SwiGLU on interleaved row pairs in registers and writes the down
// input; down applies bias and writes float32 expert outputs.
#include <functional>
#include <mutex>

#include "klc_common.h"
#include "klc_gemv.h"

namespace klc {

int launch_router_logits(const void* x, const void* w, const void* b, void* logits, float* x_f32, int64_t n_tok,
                         int64_t hidden, int64_t n_exp, hipStream_t stream);
// host_ids / host_weights (optional): copies of the selection in a host
// record, pinned host memory mapped into the device
int launch_topk(const void* logits, int32_t* ids, float* values, void* weights, int64_t n_tok, int64_t n_exp,
                int64_t k, hipStream_t stream, int32_t* host_ids = nullptr, void* host_weights = nullptr);
int launch_dispatch(const int32_t* ids, int64_t n_pairs, int64_t n_exp, int32_t* offsets, int32_t* sorted,
                    int32_t* active, int32_t* n_active, int32_t* units, hipStream_t stream);
int launch_router_decode(const void* x, const void* w, const void* b, void* logits, int64_t n_tok, int64_t hidden,
                         int64_t n_exp, int64_t k, int32_t* ids, float* values, void* weights, int32_t* offsets,
                         int32_t* sorted, int32_t* active, int32_t* n_active, int32_t* units, uint32_t* counters,
                         double* partials, hipStream_t stream, int32_t* host_ids = nullptr,
                         void* host_weights = nullptr, uint32_t* host_tag = nullptr, uint32_t tag_value = 0);
int64_t decode_router_counters(int64_t n_tok, int64_t n_exp);
int64_t decode_router_partial_bytes(int64_t n_tok, int64_t hidden, int64_t n_exp);
int check_router_args(int64_t n_tok, int64_t hidden, int64_t n_exp);
int launch_gemm_gate_up(const void* const* w, const void* bias, const void* x, int64_t n_tok, int64_t k,
                        int64_t n_exp, const int32_t* offsets, const int32_t* pairs, const int32_t* units,
                        int64_t hidden, int64_t inter, float limit, int precision, void* gated_split,
                        float* gated_raw, hipStream_t stream);
int launch_gemm_down(const void* const* w, const void* bias, const void* gated_split, int64_t n_pairs, int64_t n_exp,
                     const int32_t* offsets, const int32_t* pairs, const int32_t* units, int64_t hidden, int64_t inter,
                     int precision, float* eo, hipStream_t stream);
int check_topk_args(int64_t n_tok, int64_t n_exp, int64_t k);
int check_dispatch_args(int64_t n_pairs, int64_t n_exp);
bool fused_decode_supported(int64_t n_tok, int64_t hidden, int64_t inter, int64_t n_exp, int64_t k, const void* out,
                            const void* residual);
int64_t fused_decode_scratch_bytes(int64_t n_tok, int64_t hidden, int64_t inter, int64_t n_exp, int64_t k);
int64_t fused_decode_status_offset(int64_t n_tok, int64_t hidden, int64_t inter, int64_t n_exp, int64_t k);
int launch_moe_decode_fused(const void* x, const void* router_w, const void* router_b, const void* const* w_gate_up,
                            const void* gate_up_bias, const void* const* w_down, const void* down_bias,
                            int64_t n_tok, int64_t hidden, int64_t inter, int64_t n_exp, int64_t k, float limit,
                            int precision, char* fused_ws, void* logits, int32_t* ids, float* values, void* weights,
                            void* gated, float* eo, void* out, const void* residual, hipStream_t stream);

namespace {

template <bool kDown, int kSteps>
__global__ __launch_bounds__(kGemvThreads) void moe_gemv_mfma_kernel(
    const uint8_t* const* __restrict__ wptr, const uint16_t* __restrict__ bias, const uint16_t* __restrict__ act,
    int64_t act_plane, float* __restrict__ out, uint16_t* __restrict__ out_split, int64_t out_plane,
    float* __restrict__ out_raw, const int32_t* __restrict__ offsets, const int32_t* __restrict__ pairs,
    const int32_t* __restrict__ units, const int32_t* __restrict__ n_units, int rows, int groups, int k_top,
    float limit, int precision, int tpw) {
  extern __shared__ __align__(16) uint16_t xs[];  // [kVRows][row_stride] bfloat16 bits

  // Start-up: each load is issued as soon as its address is known, so the
  // weight stream starts after two dependent levels (unit count and unit;
  // the expert's offsets and matrix pointer) instead of one per value.
  const int tiles = rows / kTileRows;
  const int tile0 = blockIdx.x * tpw;
  const int ntile = min(tpw, tiles - tile0);
  if (ntile <= 0) return;
  const int u = blockIdx.y;
  const int n_u = *n_units;
  const int32_t unit = units[u];  // u < the unit capacity: always readable
  // both loads are issued before the branch waits (the compiler would
  // otherwise sink the unit's load below it)
  asm volatile("" ::"s"(unit), "s"(n_u));
  if (u >= n_u) return;
  const int e = unit_expert(unit);
  const int pb = offsets[e];
  const int pe = offsets[e + 1];
  const uint8_t* const wmat = wptr[e];
  const int tok_per_pass = kDown ? kUnitTokensDown : kUnitTokensGateUp;
  const int tc = unit_pass(unit) * tok_per_pass;  // first token of this unit
  const int nt = min(tok_per_pass, pe - pb - tc);
  gemv_unit<kDown, kSteps, false>(wmat, bias, e, act, act_plane, out, out_split, out_plane, out_raw, pairs + pb + tc,
                                  nt, rows, groups, k_top, limit, precision, tile0, ntile, xs, NoWait{});
}


template <bool kDown>
using GemvKernel = void (*)(const uint8_t* const*, const uint16_t*, const uint16_t*, int64_t, float*, uint16_t*,
                            int64_t, float*, const int32_t*, const int32_t*, const int32_t*, const int32_t*, int, int,
                            int, float, int, int);

template <bool kDown>
GemvKernel<kDown> gemv_kernel_for(int steps) {
  switch (steps) {
    case 1: return moe_gemv_mfma_kernel<kDown, 1>;
    case 2: return moe_gemv_mfma_kernel<kDown, 2>;
    case 3: return moe_gemv_mfma_kernel<kDown, 3>;
    case 4: return moe_gemv_mfma_kernel<kDown, 4>;
    case 6: return moe_gemv_mfma_kernel<kDown, 6>;
    case 8: return moe_gemv_mfma_kernel<kDown, 8>;
    case 16: return moe_gemv_mfma_kernel<kDown, 16>;
    case 24: return moe_gemv_mfma_kernel<kDown, 24>;
    default: return nullptr;
  }
}


// Tiles each workgroup streams: the unit capacity's tiles spread over about
// `target` workgroups (768 are resident at once: 3 per CU), at most 2
// (gate_up) or 3 (down) tiles each, so workgroups that finish early are
// replaced and the tail stays short; one tile per workgroup when few units
// exist.  max_units is an upper bound of the units.  Every workgroup start
// stages up to 8 activation rows and waits for a chain of index loads, so
// one tile per workgroup is much slower at batches of 4 and more.  Measured
// (120B shape): the targets 720 / 240 reach the 2 / 3 tile limits from
// batch 4 on (batch 4 62.4 -> 59.1 us, 8 91.2 -> 86.3 us, 16 137.4 ->
// 128.7 us against targets 6144 / 2304, which reached them only near batch
// 64); 3 gate_up tiles per workgroup, or 4 down tiles, were slower.
constexpr int64_t kGemvWorkgroupsUp = 720, kGemvMaxTilesUp = 2;
constexpr int64_t kGemvWorkgroupsDown = 240, kGemvMaxTilesDown = 3;

int tiles_per_workgroup(int tiles, int64_t max_units, int64_t target, int64_t max_tpw) {
  int64_t tpw = (int64_t)tiles * max_units / target;
  if (tpw > max_tpw) tpw = max_tpw;
  if (tpw < 1) tpw = 1;
  if (tpw > tiles) tpw = tiles;
  return (int)tpw;
}


// out[t][h] over k slots in order; every step rounded to bfloat16; then, if
// residual is given, out = bf16(residual + out) (the stacked decode's
// hidden += moe_out).
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ eo, const uint16_t* __restrict__ w,
                                                      const uint16_t* residual, int k, int hidden,
                                                      uint16_t* out) {  // out may alias residual
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
  if (residual != nullptr) acc = bf16_to_f32(residual[(int64_t)t * hidden + h]) + acc;
  out[(int64_t)t * hidden + h] = (uint16_t)f32_to_bf16_rne(acc);
}

// The same combine, 4 consecutive outputs per thread, for hidden % 4 == 0
// and 16-byte aligned expert outputs (8-byte aligned out/residual): every
// slot's 16-byte load is issued before the first is used, so a token costs
// one memory round trip instead of one per slot.  Same operations, same
// order, per output.
constexpr int kCombineMaxK = 4;  // slots whose loads are in flight together (top-4)
__global__ __launch_bounds__(256) void combine4_kernel(const float* __restrict__ eo, const uint16_t* __restrict__ w,
                                                       const uint16_t* residual, int k, int hidden,
                                                       uint16_t* out) {  // out may alias residual
  const int t = blockIdx.y;
  const int h = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (h >= hidden) return;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int j0 = 0; j0 < k; j0 += kCombineMaxK) {
    float4 v[kCombineMaxK];
    float wj[kCombineMaxK];
#pragma unroll
    for (int q = 0; q < kCombineMaxK; ++q) {
      const int64_t p = (int64_t)t * k + min(j0 + q, k - 1);
      wj[q] = bf16_to_f32(w[p]);
      v[q] = *reinterpret_cast<const float4*>(eo + p * hidden + h);
    }
#pragma unroll
    for (int q = 0; q < kCombineMaxK; ++q) {
      if (j0 + q < k) {
        const float o[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = round_bf16(acc[i] + round_bf16(round_bf16(o[i]) * wj[q]));
      }
    }
  }
  if (residual != nullptr) {
    const uint2 r = *reinterpret_cast<const uint2*>(residual + (int64_t)t * hidden + h);
    acc[0] = bf16_to_f32(r.x & 0xffffu) + acc[0];
    acc[1] = bf16_to_f32(r.x >> 16) + acc[1];
    acc[2] = bf16_to_f32(r.y & 0xffffu) + acc[2];
    acc[3] = bf16_to_f32(r.y >> 16) + acc[3];
  }
  const uint2 o = make_uint2(f32_to_bf16_rne(acc[0]) | (f32_to_bf16_rne(acc[1]) << 16),
                             f32_to_bf16_rne(acc[2]) | (f32_to_bf16_rne(acc[3]) << 16));
  *reinterpret_cast<uint2*>(out + (int64_t)t * hidden + h) = o;
}

// ---- one token (decode batch of 1): no dispatch ---------------------------
//
// The token's k <= 4 experts come straight from the router's ids; its pair
// for slot j is j.  gate_up runs the GEMV unit body with unit j = slot j.
// down and the combine run as one launch: workgroup b owns output rows
// [16 b, 16 b + 16) and wave j computes them for slot j (expert ids[j], the
// pair's hi/lo rows staged by the wave itself), with the same operations in
// the same order as the multi-launch GEMV (an MFMA output column depends on
// its own B column only), so the expert outputs are bit-identical; the k
// slots' rows then meet in LDS and 16 threads combine them in slot order
// with the combine kernel's roundings.

// pair index of slot j of the token (unit j's only pair)
__device__ const int32_t kSlotPairs[kCombineMaxK] = {0, 1, 2, 3};

template <int kSteps>
__global__ __launch_bounds__(kGemvThreads) void gate_up_single_kernel(
    const uint8_t* const* __restrict__ wptr, const uint16_t* __restrict__ bias, const uint16_t* __restrict__ x,
    uint16_t* __restrict__ out_split, int64_t out_plane, float* __restrict__ out_raw, const int32_t* __restrict__ ids,
    int rows, int groups, int k_top, float limit, int precision, int tpw) {
  extern __shared__ __align__(16) uint16_t xs[];
  const int tiles = rows / kTileRows;
  const int tile0 = blockIdx.x * tpw;
  const int ntile = min(tpw, tiles - tile0);
  if (ntile <= 0) return;
  const int u = blockIdx.y;  // slot u < k_top
  const int e = ids[u];
  gemv_unit<false, kSteps, false>(wptr[e], bias, e, x, 0, nullptr, out_split, out_plane, out_raw, kSlotPairs + u, 1,
                                  rows, groups, k_top, limit, precision, tile0, ntile, xs, NoWait{});
}

template <int kSteps>
__global__ __launch_bounds__(kGemvThreads) void down_combine_single_kernel(
    const uint8_t* const* __restrict__ wptr, const uint16_t* __restrict__ bias, const uint16_t* __restrict__ act,
    int64_t act_plane, const int32_t* __restrict__ ids, const uint16_t* __restrict__ wts, int k,
    float* __restrict__ eo, const uint16_t* residual, uint16_t* out, int rows, int groups, int precision) {
  // [kVRows][row_stride] staged rows (slot j: rows 2 j and 2 j + 1), then [4][16] float32 outputs
  extern __shared__ __align__(16) uint16_t xs[];
  constexpr int kR = kRing < kSteps ? kRing : kSteps;
  constexpr int row_stride = gemv_row_stride(kSteps);
  constexpr int kRowChunks = gemv_row_chunks(kSteps);
  constexpr int kBlocks = kRowChunks / 64;
  constexpr int kRecWords = (kSteps + 7) / 8 * 2;
  float* comb = reinterpret_cast<float*>(xs + kVRows * row_stride);
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, lr = lane & 15, lq = lane >> 4;
  const int r0 = blockIdx.x * 16;  // first output row of the workgroup
  const bool live = wave < k;
  const int e = ids[live ? wave : 0];
  const int cpr = groups * 4, in_dim = groups * 32;
  const int g4 = (groups + 3) >> 2;
  // the combine's operands, loaded first and converted only when used (a
  // conversion here would wait for the loads before the weight stream starts)
  uint32_t wj_bits[kCombineMaxK];
#pragma unroll
  for (int j = 0; j < kCombineMaxK; ++j) wj_bits[j] = wts[min(j, k - 1)];
  // branch-free: a null residual is an empty buffer (out-of-range reads are 0)
  const __amdgpu_buffer_rsrc_t rsbuf = __builtin_amdgcn_make_buffer_rsrc(
      (void*)residual, (short)0, residual != nullptr ? rows * 2 : 0, kBufferWord3);
  const uint32_t res_bits = __builtin_amdgcn_raw_buffer_load_b16(rsbuf, (uint32_t)(r0 + (tid & 15)) * 2u, 0, 0);
  // ---- the wave's 16 rows of expert e: scale words and bias (before the
  //      rows' DMA: only the ring's loads come between it and its wait) ----
  const int trow = (r0 & (kTileRows - 1)) + lr;  // row inside its 64-row tile
  const __amdgpu_buffer_rsrc_t wbuf = __builtin_amdgcn_make_buffer_rsrc(
      (void*)wptr[e], (short)0, live ? (int)packed_matrix_bytes(rows, groups) : 0, kBufferWord3);
  const uint32_t tb = (uint32_t)(r0 / kTileRows) * (uint32_t)groups * 1024u;
  const uint32_t voff = (uint32_t)(lq * 1024 + trow * 16);
  const uint32_t voff_tail = 4 * (g4 - 1) + lq < groups ? voff : kOutOfRange;
  auto chunk = [&](int t) -> u32x4_t {
    const uint32_t v = t >= g4 ? kOutOfRange : (t == g4 - 1 ? voff_tail : voff);
    return __builtin_amdgcn_raw_buffer_load_b128(wbuf, v, tb + 4096u * t, kStreamPolicy);
  };
  const uint32_t scale_base = (uint32_t)packed_block_bytes(rows, groups);
  const int rec = ((groups + 3) / 4 + 7) / 8 * 8;
  uint32_t sc[kRecWords];
#pragma unroll
  for (int i = 0; i < kRecWords / 2; ++i) {
    const uint32_t off = (uint32_t)packed_scale_word(groups, r0 + lr, min(i, rec / 8 - 1), lq);
    const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(wbuf, off, scale_base, kStreamPolicy);
    sc[2 * i] = v.x;
    sc[2 * i + 1] = v.y;
  }
  const u32x2_t bias4 = *reinterpret_cast<const u32x2_t*>(bias + (int64_t)e * rows + r0 + 4 * lq);
  __builtin_amdgcn_sched_barrier(0);
  // ---- the wave's hi and lo rows of pair `wave` by LDS-DMA (out of range
  //      for a slot past k), then the pad chunks zeroed ----
#pragma unroll
  for (int m = 0; m < 2 * kBlocks; ++m) {
    const int pl = m / kBlocks, b = m - pl * kBlocks;
    const uint16_t* row = act + pl * act_plane + (int64_t)(live ? wave : 0) * in_dim;
    const __amdgpu_buffer_rsrc_t rbuf =
        __builtin_amdgcn_make_buffer_rsrc((void*)row, (short)0, live ? cpr * 16 : 0, kBufferWord3);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rbuf, (__attribute__((address_space(3))) void*)(xs + (2 * wave + pl) * row_stride + b * 512), 16,
        (uint32_t)((b * 64 + lane) * 16), 0, 0, 0);
  }
  for (int c = cpr + lane; c < kRowChunks; c += kWave) {
    *reinterpret_cast<u32x4_t*>(xs + (2 * wave) * row_stride + c * 8) = u32x4_t{0u, 0u, 0u, 0u};
    *reinterpret_cast<u32x4_t*>(xs + (2 * wave + 1) * row_stride + c * 8) = u32x4_t{0u, 0u, 0u, 0u};
  }
  __builtin_amdgcn_sched_barrier(0);
  u32x4_t ring[kR];
#pragma unroll
  for (int t = 0; t < kR; ++t) ring[t] = chunk(t);
  __builtin_amdgcn_sched_barrier(0);
  // the rows have landed (the ring's loads after them stay in flight); the
  // barrier and the workgroup-scope acquire keep the LDS reads below the wait
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(kR));
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");

  // B: column 0 the hi row, columns 1..15 the lo row (only columns 0 and 1 are used)
  const uint16_t* xrow = xs + (2 * wave + min(lr, 1)) * row_stride + lq * 32;
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
  bf16x8_t bcur[4], bnext[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) bcur[j] = *reinterpret_cast<const bf16x8_t*>(xrow + j * 8);
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" : "+v"(ring[s % kR]));
    const u32x4_t w = ring[s % kR];
    ring[s % kR] = chunk(s + kR);
    if (s + 1 < kSteps) {
#pragma unroll
      for (int j = 0; j < 4; ++j) bnext[j] = *reinterpret_cast<const bf16x8_t*>(xrow + (s + 1) * 128 + j * 8);
    }
    const int eb = (int)((sc[s >> 2] >> (8 * (s & 3))) & 0xffu);
    const float scale = __builtin_amdgcn_ldexpf(1.0f, eb - 127);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(decode8(w[j], scale), bcur[j], acc, 0, 0, 0);
    if (s + 1 < kSteps) {
#pragma unroll
      for (int j = 0; j < 4; ++j) bcur[j] = bnext[j];
    }
  }
  // ---- epilogue: hi + lo (columns 0 and 1), bias, this slot's expert output ----
  float v[4] = {acc[0], acc[1], acc[2], acc[3]};
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] += __shfl_xor(v[i], 1);
  if (live && lr == 0) {
    const float bias_row[4] = {bf16_to_f32(bias4.x & 0xffffu), bf16_to_f32(bias4.x >> 16),
                               bf16_to_f32(bias4.y & 0xffffu), bf16_to_f32(bias4.y >> 16)};
    float o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (precision == KLC_PRECISION_BF16 ? round_bf16(v[i]) : v[i]) + bias_row[i];
    *reinterpret_cast<float4*>(eo + (int64_t)wave * rows + r0 + 4 * lq) = make_float4(o[0], o[1], o[2], o[3]);
    *reinterpret_cast<float4*>(comb + wave * 16 + 4 * lq) = make_float4(o[0], o[1], o[2], o[3]);
  }
  __syncthreads();
  // ---- combine: the slots in order, every step rounded to bfloat16 ----
  if (tid < 16) {
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < kCombineMaxK; ++j)
      if (j < k) a = round_bf16(a + round_bf16(round_bf16(comb[j * 16 + tid]) * bf16_to_f32(wj_bits[j])));
    if (residual != nullptr) a = bf16_to_f32(res_bits) + a;
    out[r0 + tid] = (uint16_t)f32_to_bf16_rne(a);
  }
}

using GateUpSingleKernel = void (*)(const uint8_t* const*, const uint16_t*, const uint16_t*, uint16_t*, int64_t,
                                   float*, const int32_t*, int, int, int, float, int, int);
using DownCombineSingleKernel = void (*)(const uint8_t* const*, const uint16_t*, const uint16_t*, int64_t,
                                         const int32_t*, const uint16_t*, int, float*, const uint16_t*, uint16_t*,
                                         int, int, int);

template <typename K, template <int> class Pick>
K single_kernel_for(int steps) {
  switch (steps) {
    case 1: return Pick<1>::fn;
    case 2: return Pick<2>::fn;
    case 3: return Pick<3>::fn;
    case 4: return Pick<4>::fn;
    case 6: return Pick<6>::fn;
    case 8: return Pick<8>::fn;
    case 16: return Pick<16>::fn;
    case 24: return Pick<24>::fn;
    default: return nullptr;
  }
}
template <int kSteps>
struct PickGateUpSingle {
  static constexpr GateUpSingleKernel fn = gate_up_single_kernel<kSteps>;
};
template <int kSteps>
struct PickDownCombineSingle {
  static constexpr DownCombineSingleKernel fn = down_combine_single_kernel<kSteps>;
};

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

// Sum of squares (float64) of this thread's elements of row[0 .. n): with
// 16-byte aligned rows and n % 4 == 0, float4 chunks tid, tid + 256, ...,
// four of them loaded before any is summed; else elements tid, tid + 256, ...
__device__ __forceinline__ double row_sum_squares(const float* __restrict__ row, int n, bool vec) {
  double s = 0.0;
  if (vec) {
    const float4* r4 = reinterpret_cast<const float4*>(row);
    const int n4 = n >> 2;
    for (int c0 = 0; c0 < n4; c0 += 4 * 256) {
      float4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int c = c0 + u * 256 + (int)threadIdx.x;
        v[u] = c < n4 ? r4[c] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const double a = v[u].x, b = v[u].y, c = v[u].z, d = v[u].w;
        s += a * a;
        s += b * b;
        s += c * c;
        s += d * d;
      }
    }
  } else {
    for (int i = threadIdx.x; i < n; i += 256) {
      const double v = row[i];
      s += v * v;
    }
  }
  return s;
}

// One workgroup per pair: its 256 threads read the pair's SwiGLU row and
// expert-output row with all loads in flight at once, then reduce in a
// fixed order (wave butterflies, then the four waves in order), so the
// norms are the same on every run.
__global__ __launch_bounds__(256) void pair_norms_kernel(const float* __restrict__ gated,
                                                         const float* __restrict__ eo, int inter, int hidden,
                                                         bool vec_g, bool vec_o, float* __restrict__ norms) {
  __shared__ double red[2][4];
  const int64_t p = blockIdx.x;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  double sg = row_sum_squares(gated + p * inter, inter, vec_g);
  double so = row_sum_squares(eo + p * hidden, hidden, vec_o);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    sg += __shfl_xor(sg, off);
    so += __shfl_xor(so, off);
  }
  if (lane == 0) {
    red[0][wave] = sg;
    red[1][wave] = so;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    norms[2 * p] = (float)sqrt(((red[0][0] + red[0][1]) + red[0][2]) + red[0][3]);
    norms[2 * p + 1] = (float)sqrt(((red[1][0] + red[1][1]) + red[1][2]) + red[1][3]);
  }
}

}  // namespace

int check_gemv_shapes(int64_t hidden, int64_t inter, int64_t n_pairs, int64_t n_exp) {
  KLC_REQUIRE(hidden > 0 && inter > 0 && n_pairs > 0 && n_exp > 0, KLC_ERR_ARGUMENT,
              "experts: bad sizes hidden=%lld inter=%lld n_pairs=%lld n_experts=%lld", (long long)hidden,
              (long long)inter, (long long)n_pairs, (long long)n_exp);
  const int rc = check_dispatch_args(n_pairs, n_exp);
  if (rc) return rc;
  KLC_REQUIRE(hidden % 64 == 0 && inter % 32 == 0 && (2 * inter) % 64 == 0, KLC_ERR_SHAPE,
              "experts: hidden=%lld must be a multiple of 64 and inter=%lld a multiple of 32", (long long)hidden,
              (long long)inter);
  KLC_REQUIRE(hidden <= 32 * 4 * kMaxSteps && inter <= 32 * 4 * kMaxSteps, KLC_ERR_UNSUPPORTED,
              "experts: unsupported sizes (hidden, inter <= %d)", 32 * 4 * kMaxSteps);
  return KLC_OK;
}

// The decode GEMVs run one grid row per work unit (a grid dimension holds
// at most 65535); the grouped GEMM has no such limit.
int check_gemv_grid(int64_t n_pairs, int64_t n_exp) {
  KLC_REQUIRE(units_capacity(n_pairs, n_exp, kUnitTokensDown) <= 65535, KLC_ERR_UNSUPPORTED,
              "experts: %lld pairs over %lld experts exceed the decode GEMVs' 65535 work units (use the grouped "
              "GEMM)", (long long)n_pairs, (long long)n_exp);
  return KLC_OK;
}

namespace {

int launch_gate_up(const void* const* w, const void* bias, const void* x, int64_t n_tok, int64_t k, int64_t n_exp,
                   const int32_t* offsets, const int32_t* pairs, const int32_t* units, int64_t hidden, int64_t inter,
                   float limit, int precision, void* gated_split, float* gated_raw, hipStream_t stream) {
  const int tiles = (int)(2 * inter / kTileRows);
  const int64_t cap = units_capacity(n_tok * k, n_exp, kUnitTokensGateUp);
  const int tpw = tiles_per_workgroup(tiles, cap, kGemvWorkgroupsUp, kGemvMaxTilesUp);
  const dim3 grid((unsigned)((tiles + tpw - 1) / tpw), (unsigned)cap);
  const int steps = gemv_steps((int)(hidden / 32));
  gemv_kernel_for<false>(steps)<<<grid, kGemvThreads, gemv_lds_bytes(steps), stream>>>(
      reinterpret_cast<const uint8_t* const*>(w), static_cast<const uint16_t*>(bias),
      static_cast<const uint16_t*>(x), 0, nullptr, static_cast<uint16_t*>(gated_split), n_tok * k * inter,
      gated_raw, offsets, pairs, units + kUnitHeader, units, (int)(2 * inter), (int)(hidden / 32), (int)k, limit,
      precision,
      tpw);
  return check_launch("moe_gemv_mfma_kernel<gate_up>");
}

int launch_down(const void* const* w, const void* bias, const void* gated_split, int64_t n_pairs, int64_t n_exp,
                const int32_t* offsets, const int32_t* pairs, const int32_t* units, int64_t hidden, int64_t inter,
                int precision, float* eo, hipStream_t stream) {
  const int tiles = (int)(hidden / kTileRows);
  const int64_t cap = units_capacity(n_pairs, n_exp, kUnitTokensDown);
  const int tpw = tiles_per_workgroup(tiles, cap, kGemvWorkgroupsDown, kGemvMaxTilesDown);
  const dim3 grid((unsigned)((tiles + tpw - 1) / tpw), (unsigned)cap);
  const int32_t* list = units + units_offset_down(n_pairs, n_exp);
  const int steps = gemv_steps((int)(inter / 32));
  gemv_kernel_for<true>(steps)<<<grid, kGemvThreads, gemv_lds_bytes(steps), stream>>>(
      reinterpret_cast<const uint8_t* const*>(w), static_cast<const uint16_t*>(bias),
      static_cast<const uint16_t*>(gated_split), n_pairs * inter, eo, nullptr, 0, nullptr, offsets, pairs, list,
      units + 1, (int)hidden, (int)(inter / 32), 1, 0.0f, precision, tpw);
  return check_launch("moe_gemv_mfma_kernel<down>");
}

// One token's gate_up GEMV, one grid row per slot of its top-k (ids).
int launch_gate_up_single(const void* const* w, const void* bias, const void* x, const int32_t* ids, int64_t k,
                          int64_t hidden, int64_t inter, float limit, int precision, void* gated_split,
                          float* gated_raw, hipStream_t stream) {
  const int tiles = (int)(2 * inter / kTileRows);
  const int tpw = tiles_per_workgroup(tiles, k, kGemvWorkgroupsUp, kGemvMaxTilesUp);
  const int steps = gemv_steps((int)(hidden / 32));
  single_kernel_for<GateUpSingleKernel, PickGateUpSingle>(steps)<<<
      dim3((unsigned)((tiles + tpw - 1) / tpw), (unsigned)k), kGemvThreads, gemv_lds_bytes(steps), stream>>>(
      reinterpret_cast<const uint8_t* const*>(w), static_cast<const uint16_t*>(bias), static_cast<const uint16_t*>(x),
      static_cast<uint16_t*>(gated_split), k * inter, gated_raw, ids, (int)(2 * inter), (int)(hidden / 32), (int)k,
      limit, precision, tpw);
  return check_launch("gate_up_single_kernel");
}

// One token's down GEMV for its k <= 4 slots and the combine, one workgroup per 16 output rows.
int launch_down_combine_single(const void* const* w, const void* bias, const void* gated_split, const int32_t* ids,
                               const void* weights, int64_t k, int64_t hidden, int64_t inter, int precision,
                               float* eo, const void* residual, void* out, hipStream_t stream) {
  const int steps = gemv_steps((int)(inter / 32));
  single_kernel_for<DownCombineSingleKernel, PickDownCombineSingle>(steps)<<<
      (unsigned)(hidden / 16), kGemvThreads, gemv_lds_bytes(steps) + 4 * 16 * sizeof(float), stream>>>(
      reinterpret_cast<const uint8_t* const*>(w), static_cast<const uint16_t*>(bias),
      static_cast<const uint16_t*>(gated_split), k * inter, ids, static_cast<const uint16_t*>(weights), (int)k, eo,
      static_cast<const uint16_t*>(residual), static_cast<uint16_t*>(out), (int)hidden, (int)(inter / 32),
      precision);
  return check_launch("down_combine_single_kernel");
}

int launch_combine(const float* eo, const void* w, const void* residual, int64_t n_tok, int64_t k, int64_t hidden,
                   void* out, hipStream_t stream) {
  const bool vec = hidden % 4 == 0 && ((uintptr_t)eo & 15) == 0 && ((uintptr_t)out & 7) == 0 &&
                   ((uintptr_t)residual & 7) == 0;
  if (vec) {
    const dim3 grid((unsigned)((hidden / 4 + 255) / 256), (unsigned)n_tok);
    combine4_kernel<<<grid, 256, 0, stream>>>(eo, static_cast<const uint16_t*>(w),
                                              static_cast<const uint16_t*>(residual), (int)k, (int)hidden,
                                              static_cast<uint16_t*>(out));
    return check_launch("combine4_kernel");
  }
  const dim3 grid((unsigned)((hidden + 255) / 256), (unsigned)n_tok);
  combine_kernel<<<grid, 256, 0, stream>>>(eo, static_cast<const uint16_t*>(w),
                                           static_cast<const uint16_t*>(residual), (int)k, (int)hidden,
                                           static_cast<uint16_t*>(out));
  return check_launch("combine_kernel");
}

inline int64_t align256(int64_t v) { return (v + 255) & ~(int64_t)255; }

// Batches up to this size route in one launch (router_decode_kernel); its
// completion counters live in the workspace's first kCounterBytes.
constexpr int64_t kDecodeRouterTokens = 128;
constexpr int64_t kCounterBytes = 1024;
// Batches up to this size can run as one launch (klc_decode.hip).
constexpr int64_t kFusedDecodeTokens = 16;

// The expert path klc_moe_layer takes for `path` (KLC_PATH_*).  AUTO picks
// the multi-launch layer: the one-launch layer (KLC_PATH_FUSED) measured
// 36.6 us against 35.6 us at batch 1 and 104 us against 93 us at batch 8
// (gpt-oss-120B shape), so it runs only when asked for, on a batch it takes
// and a stream that is not capturing a graph.
int resolve_layer_path(int path, int64_t n_tok, int64_t hidden, int64_t inter, int64_t n_exp, int64_t k,
                       const void* out, const void* residual, hipStream_t stream) {
  if (path == KLC_PATH_GEMV || path == KLC_PATH_GEMM) return path;
  if (path == KLC_PATH_FUSED) {
    bool fused = fused_decode_supported(n_tok, hidden, inter, n_exp, k, out, residual);
    if (fused) {
      hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
      if (hipStreamIsCapturing(stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) fused = false;
    }
    return fused ? KLC_PATH_FUSED : -1;
  }
  return n_tok * k >= 8 * n_exp ? KLC_PATH_GEMM : KLC_PATH_GEMV;
}


struct LayerScratch {
  int64_t counters, partials, logits, ids, values, weights, offsets, sorted, active, n_active, units, gated, eo, fused,
      total;
};

LayerScratch layer_scratch(int64_t n_tok, int64_t hidden, int64_t inter, int64_t n_exp, int64_t k) {
  LayerScratch s{};
  const int64_t pairs = n_tok * k;
  int64_t off = 0;
  s.counters = off; off += kCounterBytes;  // self-resetting completion counters (zero before first use)
  s.partials = off; off += align256(n_tok <= kDecodeRouterTokens ? decode_router_partial_bytes(n_tok, hidden, n_exp) : 0);
  s.logits = off;   off += align256(n_tok * n_exp * 2);
  s.ids = off;      off += align256(pairs * 4);
  s.values = off;   off += align256(pairs * 4);
  s.weights = off;  off += align256(pairs * 2);
  s.offsets = off;  off += align256((n_exp + 1) * 4);
  s.sorted = off;   off += align256(pairs * 4);
  s.active = off;   off += align256(n_exp * 4);
  s.n_active = off; off += align256(4);
  s.units = off;    off += align256(units_size(pairs, n_exp) * 4);
  s.gated = off;    off += align256(pairs * inter * 4);  // hi and lo bf16 planes
  s.eo = off;       off += align256(pairs * hidden * 4);
  // the one-launch decode layer's epoch-tagged logits and item flags
  s.fused = off;    off += n_tok <= kFusedDecodeTokens ? fused_decode_scratch_bytes(n_tok, hidden, inter, n_exp, k) : 0;
  s.total = off;
  return s;
}

}  // namespace
}  // namespace klc

using namespace klc;

extern "C" int klc_moe_gate_up(const void* const* w_gate_up, const void* bias, const void* x, int64_t n_tokens,
                               int64_t k, int64_t n_experts, const int32_t* offsets, const int32_t* sorted_pairs,
                               const int32_t* units, int64_t hidden, int64_t inter, float swiglu_limit,
                               int precision, void* gated_split, float* gated_raw, void* stream) {
  KLC_REQUIRE(w_gate_up && bias && x && offsets && sorted_pairs && units && gated_split, KLC_ERR_ARGUMENT,
              "klc_moe_gate_up: null pointer");
  KLC_REQUIRE(n_tokens > 0 && k > 0, KLC_ERR_ARGUMENT, "klc_moe_gate_up: n_tokens=%lld k=%lld", (long long)n_tokens,
              (long long)k);
  KLC_REQUIRE(precision == KLC_PRECISION_FP32 || precision == KLC_PRECISION_BF16, KLC_ERR_ARGUMENT,
              "klc_moe_gate_up: unknown precision %d", precision);
  const int rc = check_gemv_shapes(hidden, inter, n_tokens * k, n_experts);
  if (rc) return rc;
  const int rc2 = check_gemv_grid(n_tokens * k, n_experts);
  if (rc2) return rc2;
  return launch_gate_up(w_gate_up, bias, x, n_tokens, k, n_experts, offsets, sorted_pairs, units, hidden, inter,
                        swiglu_limit, precision, gated_split, gated_raw, as_stream(stream));
}

extern "C" int klc_moe_down(const void* const* w_down, const void* bias, const void* gated_split, int64_t n_pairs,
                            int64_t n_experts, const int32_t* offsets, const int32_t* sorted_pairs,
                            const int32_t* units, int64_t hidden, int64_t inter, int precision, float* expert_out,
                            void* stream) {
  KLC_REQUIRE(w_down && bias && gated_split && offsets && sorted_pairs && units && expert_out, KLC_ERR_ARGUMENT,
              "klc_moe_down: null pointer");
  KLC_REQUIRE(n_pairs > 0, KLC_ERR_ARGUMENT, "klc_moe_down: n_pairs=%lld", (long long)n_pairs);
  KLC_REQUIRE(precision == KLC_PRECISION_FP32 || precision == KLC_PRECISION_BF16, KLC_ERR_ARGUMENT,
              "klc_moe_down: unknown precision %d", precision);
  const int rc = check_gemv_shapes(hidden, inter, n_pairs, n_experts);
  if (rc) return rc;
  const int rc2 = check_gemv_grid(n_pairs, n_experts);
  if (rc2) return rc2;
  return launch_down(w_down, bias, gated_split, n_pairs, n_experts, offsets, sorted_pairs, units, hidden, inter,
                     precision, expert_out, as_stream(stream));
}

extern "C" int klc_moe_combine(const float* expert_out, const void* weights, const void* residual,
                               int64_t n_tokens, int64_t k, int64_t hidden, void* out, void* stream) {
  KLC_REQUIRE(expert_out && weights && out, KLC_ERR_ARGUMENT, "klc_moe_combine: null pointer");
  KLC_REQUIRE(n_tokens > 0 && k > 0 && hidden > 0, KLC_ERR_ARGUMENT, "klc_moe_combine: bad sizes");
  KLC_REQUIRE(n_tokens <= KLC_LAYER_MAX_TOKENS, KLC_ERR_UNSUPPORTED, "klc_moe_combine: n_tokens=%lld > 65535", (long long)n_tokens);
  return launch_combine(expert_out, weights, residual, n_tokens, k, hidden, out, as_stream(stream));
}

extern "C" int klc_moe_bias_combine(const void* down_bias, const int32_t* ids, const void* weights, int64_t n_tokens,
                                    int64_t k, int64_t hidden, void* out, void* stream) {
  KLC_REQUIRE(down_bias && ids && weights && out, KLC_ERR_ARGUMENT, "klc_moe_bias_combine: null pointer");
  KLC_REQUIRE(n_tokens > 0 && k > 0 && hidden > 0, KLC_ERR_ARGUMENT, "klc_moe_bias_combine: bad sizes");
  KLC_REQUIRE(n_tokens <= KLC_LAYER_MAX_TOKENS, KLC_ERR_UNSUPPORTED, "klc_moe_bias_combine: n_tokens=%lld > 65535",
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
  KLC_REQUIRE(inter < ((int64_t)1 << 30) && hidden < ((int64_t)1 << 30), KLC_ERR_UNSUPPORTED,
              "klc_moe_pair_norms: rows too long");
  const bool vec_g = inter % 4 == 0 && ((uintptr_t)gated & 15) == 0;
  const bool vec_o = hidden % 4 == 0 && ((uintptr_t)expert_out & 15) == 0;
  pair_norms_kernel<<<(unsigned)n_pairs, 256, 0, as_stream(stream)>>>(gated, expert_out, (int)inter, (int)hidden,
                                                                      vec_g, vec_o, norms);
  return check_launch("pair_norms_kernel");
}

extern "C" int64_t klc_moe_workspace_bytes(int64_t n_tokens, int64_t hidden, int64_t inter, int64_t n_experts,
                                           int64_t k) {
  if (n_tokens <= 0 || hidden <= 0 || inter <= 0 || n_experts <= 0 || k <= 0)
    return set_error(KLC_ERR_ARGUMENT, "klc_moe_workspace_bytes: bad sizes");
  return layer_scratch(n_tokens, hidden, inter, n_experts, k).total;
}

extern "C" int klc_moe_layer_path(int64_t n_tokens, int64_t hidden, int64_t inter, int64_t n_experts, int64_t k,
                                  int path, void* stream) {
  KLC_REQUIRE(n_tokens > 0 && hidden > 0 && inter > 0 && n_experts > 0 && k > 0, KLC_ERR_ARGUMENT,
              "klc_moe_layer_path: bad sizes");
  KLC_REQUIRE(path == KLC_PATH_AUTO || path == KLC_PATH_GEMV || path == KLC_PATH_GEMM || path == KLC_PATH_FUSED,
              KLC_ERR_ARGUMENT, "klc_moe_layer_path: unknown path %d", path);
  const int route = resolve_layer_path(path, n_tokens, hidden, inter, n_experts, k, nullptr, nullptr, as_stream(stream));
  KLC_REQUIRE(route >= 0, KLC_ERR_UNSUPPORTED, "klc_moe_layer_path: KLC_PATH_FUSED does not take this batch");
  return route;
}

extern "C" int64_t klc_moe_layer_status_offset(int64_t n_tokens, int64_t hidden, int64_t inter, int64_t n_experts,
                                               int64_t k) {
  KLC_REQUIRE(n_tokens > 0 && hidden > 0 && inter > 0 && n_experts > 0 && k > 0, KLC_ERR_ARGUMENT,
              "klc_moe_layer_status_offset: bad sizes");
  if (n_tokens > kFusedDecodeTokens) return -1;
  return layer_scratch(n_tokens, hidden, inter, n_experts, k).fused +
         fused_decode_status_offset(n_tokens, hidden, inter, n_experts, k);
}

namespace klc {
namespace {

// Argument checks shared by klc_moe_layer and klc_moe_layer_static_scratch
// (everything but the scratch memory); `fn` names the entry point.
int check_layer_args(const char* fn, const void* x, const void* router_w, const void* router_b,
                     const void* const* w_gate_up, const void* gate_up_bias, const void* const* w_down,
                     const void* down_bias, const void* out, int64_t n_tokens, int64_t hidden, int64_t inter,
                     int64_t n_experts, int64_t k, int precision, int path) {
  KLC_REQUIRE(x && router_w && router_b && w_gate_up && gate_up_bias && w_down && down_bias && out,
              KLC_ERR_ARGUMENT, "%s: null pointer", fn);
  KLC_REQUIRE(precision == KLC_PRECISION_FP32 || precision == KLC_PRECISION_BF16, KLC_ERR_ARGUMENT,
              "%s: unknown precision %d", fn, precision);
  KLC_REQUIRE(path == KLC_PATH_AUTO || path == KLC_PATH_GEMV || path == KLC_PATH_GEMM || path == KLC_PATH_FUSED,
              KLC_ERR_ARGUMENT, "%s: unknown path %d", fn, path);
  int rc = check_router_args(n_tokens, hidden, n_experts);
  if (rc) return rc;
  rc = check_topk_args(n_tokens, n_experts, k);
  if (rc) return rc;
  rc = check_gemv_shapes(hidden, inter, n_tokens * k, n_experts);
  if (rc) return rc;
  KLC_REQUIRE(n_tokens <= KLC_LAYER_MAX_TOKENS, KLC_ERR_UNSUPPORTED, "%s: n_tokens=%lld > 65535", fn, (long long)n_tokens);
  return KLC_OK;
}

// Host copy of a route call's record (klc_moe_route_readback): pinned host
// memory mapped into the device (`rec`, the record's device address).  The
// kernel that selects the experts writes ids and weights there as well; the
// record's tag word then receives `tag` (from the one-token router itself,
// else from write_tag_kernel after the selecting kernel), and the norms
// kernel writes the norms.  Record layout (4-byte words): ids (pairs), bf16
// weights (pairs, padded to a word), norms (float32, 2 * pairs), tag.
struct Readback {
  char* rec;
  int64_t pairs;
  uint32_t tag;
  int32_t* ids() const { return reinterpret_cast<int32_t*>(rec); }
  void* weights() const { return rec + 4 * pairs; }
  float* norms() const { return reinterpret_cast<float*>(rec + 4 * (pairs + (pairs + 1) / 2)); }
  uint32_t* tag_word() const { return reinterpret_cast<uint32_t*>(rec + 4 * (3 * pairs + (pairs + 1) / 2)); }
};

__global__ __launch_bounds__(64) void write_tag_kernel(uint32_t* tag_word, uint32_t tag) {
  // the selecting kernel has finished (stream order) and fenced its host stores
  if (threadIdx.x == 0) __hip_atomic_store(tag_word, tag, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

int write_tag(const Readback* rb, hipStream_t st) {
  if (rb == nullptr) return KLC_OK;
  write_tag_kernel<<<1, 64, 0, st>>>(rb->tag_word(), rb->tag);
  return check_launch("write_tag_kernel");
}

// The layer's launches on scratch memory `ws` (layer_scratch layout, counters
// zero on entry and left zero).  router_w == NULL: ids / weights already hold
// the selection (klc_moe_experts), and the layer starts at the dispatch.
// rb != NULL (with router_w): the selecting kernel also writes the
// selection to the host record, followed by its tag (the caller passes the
// record's norms as `norms`).
int run_moe_layer(const void* x, const void* router_w, const void* router_b, const void* const* w_gate_up,
                  const void* gate_up_bias, const void* const* w_down, const void* down_bias, int64_t n_tokens,
                  int64_t hidden, int64_t inter, int64_t n_experts, int64_t k, float swiglu_limit, int precision,
                  int path, char* ws, void* out, const void* residual, int32_t* ids, void* weights,
                  float* gated_raw, float* norms, void* const* events, void* stream,
                  const Readback* rb = nullptr) {
  int rc = KLC_OK;
  const LayerScratch s = layer_scratch(n_tokens, hidden, inter, n_experts, k);
  void* logits = ws + s.logits;
  int32_t* ids_buf = ids ? ids : reinterpret_cast<int32_t*>(ws + s.ids);
  float* values = reinterpret_cast<float*>(ws + s.values);
  void* w_buf = weights ? weights : static_cast<void*>(ws + s.weights);
  int32_t* offsets = reinterpret_cast<int32_t*>(ws + s.offsets);
  int32_t* sorted = reinterpret_cast<int32_t*>(ws + s.sorted);
  int32_t* active = reinterpret_cast<int32_t*>(ws + s.active);
  int32_t* n_active = reinterpret_cast<int32_t*>(ws + s.n_active);
  int32_t* units = reinterpret_cast<int32_t*>(ws + s.units);
  void* gated = ws + s.gated;
  float* eo = reinterpret_cast<float*>(ws + s.eo);
  uint32_t* counters = reinterpret_cast<uint32_t*>(ws + s.counters);
  hipStream_t st = as_stream(stream);
  auto mark = [&](int i) -> int {
    if (events == nullptr) return KLC_OK;
    const hipError_t err = hipEventRecord(static_cast<hipEvent_t>(events[i]), st);
    return err == hipSuccess ? KLC_OK : set_error(KLC_ERR_HIP, "klc_moe_layer: hipEventRecord: %s", hipGetErrorString(err));
  };

  const int route = resolve_layer_path(path, n_tokens, hidden, inter, n_experts, k, out, residual, st);
  KLC_REQUIRE(route >= 0, KLC_ERR_UNSUPPORTED,
              "klc_moe_layer: KLC_PATH_FUSED does not take n_tokens=%lld, n_experts=%lld, k=%lld (at most 16 tokens, "
              "64 pairs, 256 experts, k <= 16, 8-byte aligned out/residual, no graph capture)",
              (long long)n_tokens, (long long)n_experts, (long long)k);
  // one token routed here, by the GEMVs: the single-token kernels
  const bool single = route == KLC_PATH_GEMV && router_w != nullptr && n_tokens == 1 && k <= kCombineMaxK;
  if ((rc = mark(0))) return rc;
  if (route == KLC_PATH_FUSED) {
    // the whole layer in one launch; the remaining events follow it back to back
    if ((rc = launch_moe_decode_fused(x, router_w, router_b, w_gate_up, gate_up_bias, w_down, down_bias, n_tokens,
                                      hidden, inter, n_experts, k, swiglu_limit, precision, ws + s.fused, logits,
                                      ids_buf, values, w_buf, gated, eo, out, residual, st)))
      return rc;
    for (int i = 1; i < KLC_LAYER_EVENTS; ++i)
      if ((rc = mark(i))) return rc;
    return KLC_OK;
  }
  if (router_w == nullptr) {
    // the selection is given (ids / weights hold it): dispatch only
    if ((rc = mark(1))) return rc;
    if ((rc = mark(2))) return rc;
    if ((rc = launch_dispatch(ids_buf, n_tokens * k, n_experts, offsets, sorted, active, n_active, units, st)))
      return rc;
  } else if (single) {
    // one token: logits and top-k in one launch, no dispatch (the expert
    // kernels take the token's slots from the ids)
    if ((rc = launch_router_decode(x, router_w, router_b, logits, 1, hidden, n_experts, k, ids_buf, values, w_buf,
                                   nullptr, nullptr, nullptr, nullptr, nullptr, counters,
                                   reinterpret_cast<double*>(ws + s.partials), st, rb ? rb->ids() : nullptr,
                                   rb ? rb->weights() : nullptr, rb ? rb->tag_word() : nullptr,
                                   rb ? rb->tag : 0u)))
      return rc;
    if (!router_decode_one_wave(1, n_experts) && (rc = write_tag(rb, st))) return rc;
    if ((rc = mark(1))) return rc;
    if ((rc = mark(2))) return rc;
  } else if (n_tokens <= kDecodeRouterTokens) {
    // decode batches: logits, top-k and dispatch in one launch
    KLC_REQUIRE(decode_router_counters(n_tokens, n_experts) * 4 <= kCounterBytes, KLC_ERR_UNSUPPORTED,
                "klc_moe_layer: %lld experts need more completion counters than the workspace holds",
                (long long)n_experts);
    if ((rc = launch_router_decode(x, router_w, router_b, logits, n_tokens, hidden, n_experts, k, ids_buf, values,
                                   w_buf, offsets, sorted, active, n_active, units, counters,
                                   reinterpret_cast<double*>(ws + s.partials), st, rb ? rb->ids() : nullptr,
                                   rb ? rb->weights() : nullptr)))
      return rc;
    if ((rc = write_tag(rb, st))) return rc;
    if ((rc = mark(1))) return rc;
    if ((rc = mark(2))) return rc;
  } else {
    if ((rc = launch_router_logits(x, router_w, router_b, logits, nullptr, n_tokens, hidden, n_experts, st)))
      return rc;
    if ((rc = mark(1))) return rc;
    if ((rc = launch_topk(logits, ids_buf, values, w_buf, n_tokens, n_experts, k, st, rb ? rb->ids() : nullptr,
                          rb ? rb->weights() : nullptr)))
      return rc;
    if ((rc = write_tag(rb, st))) return rc;
    if ((rc = mark(2))) return rc;
    if ((rc = launch_dispatch(ids_buf, n_tokens * k, n_experts, offsets, sorted, active, n_active, units, st)))
      return rc;
  }
  if ((rc = mark(3))) return rc;
  if (single) {
    if ((rc = launch_gate_up_single(w_gate_up, gate_up_bias, x, ids_buf, k, hidden, inter, swiglu_limit, precision,
                                    gated, gated_raw, st)))
      return rc;
    if ((rc = mark(4))) return rc;
    if ((rc = launch_down_combine_single(w_down, down_bias, gated, ids_buf, w_buf, k, hidden, inter, precision, eo,
                                         residual, out, st)))
      return rc;
    if ((rc = mark(5))) return rc;
    if ((rc = mark(6))) return rc;
    if (norms == nullptr) return KLC_OK;
    return klc_moe_pair_norms(gated_raw, eo, k, inter, hidden, norms, st);
  }
  const bool gemm = route == KLC_PATH_GEMM;
  if (!gemm && (rc = check_gemv_grid(n_tokens * k, n_experts))) return rc;
  if (gemm) {
    if ((rc = launch_gemm_gate_up(w_gate_up, gate_up_bias, x, n_tokens, k, n_experts, offsets, sorted, units, hidden,
                                  inter, swiglu_limit, precision, gated, gated_raw, st)))
      return rc;
    if ((rc = mark(4))) return rc;
    if ((rc = launch_gemm_down(w_down, down_bias, gated, n_tokens * k, n_experts, offsets, sorted, units, hidden,
                               inter, precision, eo, st)))
      return rc;
  } else {
    if ((rc = launch_gate_up(w_gate_up, gate_up_bias, x, n_tokens, k, n_experts, offsets, sorted, units, hidden,
                             inter, swiglu_limit, precision, gated, gated_raw, st)))
      return rc;
    if ((rc = mark(4))) return rc;
    if ((rc = launch_down(w_down, down_bias, gated, n_tokens * k, n_experts, offsets, sorted, units, hidden, inter,
                          precision, eo, st)))
      return rc;
  }
  if ((rc = mark(5))) return rc;
  if ((rc = launch_combine(eo, w_buf, residual, n_tokens, k, hidden, out, st))) return rc;
  if ((rc = mark(6))) return rc;
  if (norms == nullptr) return KLC_OK;
  return klc_moe_pair_norms(gated_raw, eo, n_tokens * k, inter, hidden, norms, st);
}

__global__ __launch_bounds__(256) void clear_words_kernel(uint32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// Scratch memory of klc_moe_layer_static_scratch: one array per GPU, held by
// the process from the library's load on.  Host code never passes `scratch`
// itself to a kernel (on the host it names a host-side stand-in): the
// device address comes from hipGetSymbolAddress, once per device.
static __device__ __align__(256) char scratch[KLC_STATIC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices];

// Device address of the current device's `scratch`, looked up (and its
// completion counters cleared on `stream`) on the first call on that device.
int static_scratch_address(const char* fn, hipStream_t stream, char** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  KLC_REQUIRE(err == hipSuccess, KLC_ERR_HIP, "%s: hipGetDevice: %s", fn, hipGetErrorString(err));
  KLC_REQUIRE(dev >= 0 && dev < kMaxDevices, KLC_ERR_UNSUPPORTED, "%s: device %d >= %d", fn, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    KLC_REQUIRE(err == hipSuccess && ptr != nullptr, KLC_ERR_HIP, "%s: hipGetSymbolAddress(scratch): %s", fn,
                hipGetErrorString(err));
    // the array starts zeroed; the counters are cleared once more, by a kernel
    // (not a memset, so that a caller capturing this call in a graph records
    // no memset node), and every launch leaves them zero
    clear_words_kernel<<<(kCounterBytes / 4 + 255) / 256, 256, 0, stream>>>(static_cast<uint32_t*>(ptr),
                                                                             (int)(kCounterBytes / 4));
    const int rc = check_launch("clear_words_kernel");
    if (rc) return rc;
    g_scratch_ptr[dev] = ptr;
  }
  *out = static_cast<char*>(g_scratch_ptr[dev]);
  return KLC_OK;
}

}  // namespace
}  // namespace klc

extern "C" int klc_moe_layer(const void* x, const void* router_w, const void* router_b, const void* const* w_gate_up,
                             const void* gate_up_bias, const void* const* w_down, const void* down_bias,
                             int64_t n_tokens, int64_t hidden, int64_t inter, int64_t n_experts, int64_t k,
                             float swiglu_limit, int precision, int path, void* workspace, int64_t workspace_bytes,
                             void* out, const void* residual, int32_t* ids, void* weights, void* const* events,
                             void* stream) {
  int rc = check_layer_args("klc_moe_layer", x, router_w, router_b, w_gate_up, gate_up_bias, w_down, down_bias, out,
                            n_tokens, hidden, inter, n_experts, k, precision, path);
  if (rc) return rc;
  KLC_REQUIRE(workspace != nullptr, KLC_ERR_ARGUMENT, "klc_moe_layer: null pointer");
  const LayerScratch s = layer_scratch(n_tokens, hidden, inter, n_experts, k);
  KLC_REQUIRE(workspace_bytes >= s.total, KLC_ERR_ARGUMENT, "klc_moe_layer: workspace of %lld bytes < %lld needed",
              (long long)workspace_bytes, (long long)s.total);
  KLC_REQUIRE(((uintptr_t)workspace & 255) == 0, KLC_ERR_ARGUMENT, "klc_moe_layer: workspace must be 256-byte aligned");
  return run_moe_layer(x, router_w, router_b, w_gate_up, gate_up_bias, w_down, down_bias, n_tokens, hidden, inter,
                       n_experts, k, swiglu_limit, precision, path, static_cast<char*>(workspace), out, residual, ids,
                       weights, nullptr, nullptr, events, stream);
}

namespace klc {
namespace {

int route_layer(const char* fn, const void* x, const void* router_w, const void* router_b,
                const void* const* w_gate_up, const void* gate_up_bias, const void* const* w_down,
                const void* down_bias, int64_t n_tokens, int64_t hidden, int64_t inter, int64_t n_experts, int64_t k,
                float swiglu_limit, int precision, int path, void* workspace, int64_t workspace_bytes, void* out,
                int32_t* ids, void* weights, float* gated, float* norms, void* stream, const Readback* rb) {
  int rc = check_layer_args(fn, x, router_w, router_b, w_gate_up, gate_up_bias, w_down, down_bias, out, n_tokens,
                            hidden, inter, n_experts, k, precision, path);
  if (rc) return rc;
  KLC_REQUIRE(workspace && ids && weights && gated && norms, KLC_ERR_ARGUMENT, "%s: null pointer", fn);
  KLC_REQUIRE(path != KLC_PATH_FUSED, KLC_ERR_UNSUPPORTED,
              "%s: the one-launch layer keeps no float32 SwiGLU outputs for the norms", fn);
  const LayerScratch s = layer_scratch(n_tokens, hidden, inter, n_experts, k);
  KLC_REQUIRE(workspace_bytes >= s.total, KLC_ERR_ARGUMENT, "%s: workspace of %lld bytes < %lld needed", fn,
              (long long)workspace_bytes, (long long)s.total);
  KLC_REQUIRE(((uintptr_t)workspace & 255) == 0, KLC_ERR_ARGUMENT, "%s: workspace must be 256-byte aligned", fn);
  return run_moe_layer(x, router_w, router_b, w_gate_up, gate_up_bias, w_down, down_bias, n_tokens, hidden, inter,
                       n_experts, k, swiglu_limit, precision, path, static_cast<char*>(workspace), out, nullptr, ids,
                       weights, gated, norms, nullptr, stream, rb);
}

}  // namespace
}  // namespace klc

extern "C" int klc_moe_route(const void* x, const void* router_w, const void* router_b, const void* const* w_gate_up,
                             const void* gate_up_bias, const void* const* w_down, const void* down_bias,
                             int64_t n_tokens, int64_t hidden, int64_t inter, int64_t n_experts, int64_t k,
                             float swiglu_limit, int precision, int path, void* workspace, int64_t workspace_bytes,
                             void* out, int32_t* ids, void* weights, float* gated, float* norms, void* stream) {
  return route_layer("klc_moe_route", x, router_w, router_b, w_gate_up, gate_up_bias, w_down, down_bias, n_tokens,
                     hidden, inter, n_experts, k, swiglu_limit, precision, path, workspace, workspace_bytes, out, ids,
                     weights, gated, norms, stream, nullptr);
}

extern "C" int klc_moe_route_readback(const void* x, const void* router_w, const void* router_b,
                                      const void* const* w_gate_up, const void* gate_up_bias,
                                      const void* const* w_down, const void* down_bias, int64_t n_tokens,
                                      int64_t hidden, int64_t inter, int64_t n_experts, int64_t k,
                                      float swiglu_limit, int precision, int path, void* workspace,
                                      int64_t workspace_bytes, void* out, int32_t* ids, void* weights, float* gated,
                                      void* host_record, uint32_t tag, void* stream) {
  const char* fn = "klc_moe_route_readback";
  KLC_REQUIRE(host_record != nullptr, KLC_ERR_ARGUMENT, "%s: null host record", fn);
  KLC_REQUIRE(tag != 0u, KLC_ERR_ARGUMENT, "%s: tag 0 (the caller clears the tag word to 0)", fn);
  KLC_REQUIRE(n_tokens > 0 && k > 0 && n_tokens * k <= KLC_DISPATCH_MAX_PAIRS, KLC_ERR_ARGUMENT,
              "%s: n_tokens=%lld k=%lld", fn, (long long)n_tokens, (long long)k);
  // the record must be host memory the runtime maps into the device; its
  // device address comes from the runtime (pageable memory is refused)
  hipPointerAttribute_t attr{};
  const hipError_t err = hipPointerGetAttributes(&attr, host_record);
  KLC_REQUIRE(err == hipSuccess && attr.type == hipMemoryTypeHost && attr.devicePointer != nullptr,
              KLC_ERR_ARGUMENT, "%s: host_record is not pinned host memory mapped into the device (%s)", fn,
              hipGetErrorString(err));
  const Readback rb{static_cast<char*>(attr.devicePointer), n_tokens * k, tag};
  return route_layer(fn, x, router_w, router_b, w_gate_up, gate_up_bias, w_down, down_bias, n_tokens, hidden, inter,
                     n_experts, k, swiglu_limit, precision, path, workspace, workspace_bytes, out, ids, weights, gated,
                     rb.norms(), stream, &rb);
}

extern "C" int klc_moe_experts(const void* x, const int32_t* ids, const void* weights, const void* const* w_gate_up,
                               const void* gate_up_bias, const void* const* w_down, const void* down_bias,
                               int64_t n_tokens, int64_t hidden, int64_t inter, int64_t n_experts, int64_t k,
                               float swiglu_limit, int precision, int path, void* workspace, int64_t workspace_bytes,
                               void* out, float* gated, float* norms, void* stream) {
  const char* fn = "klc_moe_experts";
  KLC_REQUIRE(x && ids && weights && w_gate_up && gate_up_bias && w_down && down_bias && out && workspace,
              KLC_ERR_ARGUMENT, "%s: null pointer", fn);
  KLC_REQUIRE((gated == nullptr) == (norms == nullptr), KLC_ERR_ARGUMENT, "%s: gated and norms go together", fn);
  KLC_REQUIRE(precision == KLC_PRECISION_FP32 || precision == KLC_PRECISION_BF16, KLC_ERR_ARGUMENT,
              "%s: unknown precision %d", fn, precision);
  KLC_REQUIRE(path == KLC_PATH_AUTO || path == KLC_PATH_GEMV || path == KLC_PATH_GEMM, KLC_ERR_UNSUPPORTED,
              "%s: path %d (AUTO, GEMV or GEMM; the one-launch layer routes by itself)", fn, path);
  KLC_REQUIRE(n_tokens > 0 && k > 0 && k <= n_experts, KLC_ERR_ARGUMENT, "%s: n_tokens=%lld k=%lld n_experts=%lld",
              fn, (long long)n_tokens, (long long)k, (long long)n_experts);
  KLC_REQUIRE(n_tokens <= KLC_LAYER_MAX_TOKENS, KLC_ERR_UNSUPPORTED, "%s: n_tokens=%lld > 65535", fn,
              (long long)n_tokens);
  int rc = check_gemv_shapes(hidden, inter, n_tokens * k, n_experts);
  if (rc) return rc;
  const LayerScratch s = layer_scratch(n_tokens, hidden, inter, n_experts, k);
  KLC_REQUIRE(workspace_bytes >= s.total, KLC_ERR_ARGUMENT, "%s: workspace of %lld bytes < %lld needed", fn,
              (long long)workspace_bytes, (long long)s.total);
  KLC_REQUIRE(((uintptr_t)workspace & 255) == 0, KLC_ERR_ARGUMENT, "%s: workspace must be 256-byte aligned", fn);
  return run_moe_layer(x, nullptr, nullptr, w_gate_up, gate_up_bias, w_down, down_bias, n_tokens, hidden, inter,
                       n_experts, k, swiglu_limit, precision, path, static_cast<char*>(workspace), out, nullptr,
                       const_cast<int32_t*>(ids), const_cast<void*>(weights), gated, norms, nullptr, stream);
}

extern "C" int klc_moe_select(const void* x, const void* router_w, const void* router_b, int64_t n_tokens,
                              int64_t hidden, int64_t n_experts, int64_t k, void* workspace, int64_t workspace_bytes,
                              int32_t* ids, void* weights, void* stream) {
  const char* fn = "klc_moe_select";
  KLC_REQUIRE(x && router_w && router_b && workspace && ids && weights, KLC_ERR_ARGUMENT, "%s: null pointer", fn);
  int rc = check_router_args(n_tokens, hidden, n_experts);
  if (rc) return rc;
  if ((rc = check_topk_args(n_tokens, n_experts, k))) return rc;
  if ((rc = check_dispatch_args(n_tokens * k, n_experts))) return rc;
  KLC_REQUIRE(n_tokens <= KLC_LAYER_MAX_TOKENS, KLC_ERR_UNSUPPORTED, "%s: n_tokens=%lld > 65535", fn,
              (long long)n_tokens);
  // the routing regions of the layer workspace come before the expert
  // regions, so their offsets do not depend on the intermediate size
  const LayerScratch s = layer_scratch(n_tokens, hidden, 32, n_experts, k);
  KLC_REQUIRE(workspace_bytes >= s.gated, KLC_ERR_ARGUMENT, "%s: workspace of %lld bytes < %lld needed", fn,
              (long long)workspace_bytes, (long long)s.gated);
  KLC_REQUIRE(((uintptr_t)workspace & 255) == 0, KLC_ERR_ARGUMENT, "%s: workspace must be 256-byte aligned", fn);
  char* ws = static_cast<char*>(workspace);
  float* values = reinterpret_cast<float*>(ws + s.values);
  hipStream_t st = as_stream(stream);
  if (n_tokens <= kDecodeRouterTokens) {
    KLC_REQUIRE(decode_router_counters(n_tokens, n_experts) * 4 <= kCounterBytes, KLC_ERR_UNSUPPORTED,
                "%s: %lld experts need more completion counters than the workspace holds", fn, (long long)n_experts);
    // routing only: the expert half (klc_moe_experts) builds its own dispatch
    return launch_router_decode(x, router_w, router_b, ws + s.logits, n_tokens, hidden, n_experts, k, ids, values,
                                weights, nullptr, nullptr, nullptr, nullptr, nullptr,
                                reinterpret_cast<uint32_t*>(ws + s.counters),
                                reinterpret_cast<double*>(ws + s.partials), st);
  }
  if ((rc = launch_router_logits(x, router_w, router_b, ws + s.logits, nullptr, n_tokens, hidden, n_experts, st)))
    return rc;
  return launch_topk(ws + s.logits, ids, values, weights, n_tokens, n_experts, k, st);
}

extern "C" int klc_moe_layer_static_scratch(const void* x, const void* router_w, const void* router_b,
                                            const void* const* w_gate_up, const void* gate_up_bias,
                                            const void* const* w_down, const void* down_bias, int64_t n_tokens,
                                            int64_t hidden, int64_t inter, int64_t n_experts, int64_t k,
                                            float swiglu_limit, int precision, int path, void* out,
                                            const void* residual, int32_t* ids, void* weights, void* const* events,
                                            void* stream) {
  const char* fn = "klc_moe_layer_static_scratch";
  int rc = check_layer_args(fn, x, router_w, router_b, w_gate_up, gate_up_bias, w_down, down_bias, out, n_tokens,
                            hidden, inter, n_experts, k, precision, path);
  if (rc) return rc;
  const LayerScratch s = layer_scratch(n_tokens, hidden, inter, n_experts, k);
  KLC_REQUIRE(s.total <= (int64_t)KLC_STATIC_SCRATCH_BYTES, KLC_ERR_UNSUPPORTED,
              "%s: the layer needs %lld bytes of scratch for n_tokens=%lld, more than the %lld bytes of the "
              "library's static scratch (use klc_moe_layer with a workspace)", fn, (long long)s.total,
              (long long)n_tokens, (long long)KLC_STATIC_SCRATCH_BYTES);
  char* ws = nullptr;
  if ((rc = static_scratch_address(fn, as_stream(stream), &ws))) return rc;
  return run_moe_layer(x, router_w, router_b, w_gate_up, gate_up_bias, w_down, down_bias, n_tokens, hidden, inter,
                       n_experts, k, swiglu_limit, precision, path, ws, out, residual, ids, weights, nullptr, nullptr,
                       events, stream);
}
