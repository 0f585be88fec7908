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
#include <mutex>

#include "klc_common.h"

namespace klc {

int launch_router_logits(const void* x, const void* w, const void* b, void* logits, float* x_f32, int64_t n_tok,
                         int64_t hidden, int64_t n_exp, hipStream_t stream);
int launch_topk(const void* logits, int32_t* ids, float* values, void* weights, int64_t n_tok, int64_t n_exp,
                int64_t k, hipStream_t stream);
int launch_dispatch(const int32_t* ids, int64_t n_pairs, int64_t n_exp, int32_t* offsets, int32_t* sorted,
                    int32_t* active, int32_t* n_active, int32_t* units, hipStream_t stream);
int launch_router_decode(const void* x, const void* w, const void* b, void* logits, int64_t n_tok, int64_t hidden,
                         int64_t n_exp, int64_t k, int32_t* ids, float* values, void* weights, int32_t* offsets,
                         int32_t* sorted, int32_t* active, int32_t* n_active, int32_t* units, uint32_t* counters,
                         double* partials, hipStream_t stream);
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

namespace {

constexpr int kGemvWaves = 4;                 // 4 x 16 rows = one 64-row tile per workgroup
constexpr int kGemvThreads = kGemvWaves * kWave;
constexpr int kVRows = 8;                     // activation rows (MFMA N columns) staged per unit
constexpr int kMaxSteps = 24;                 // 4-group steps per row (inputs <= 3072)

typedef float f32x4_t __attribute__((ext_vector_type(4)));


__device__ __forceinline__ float swiglu(float gate, float up, float limit) {
  // streamed_moe_router.py:524-529; comparisons keep NaN like torch.clamp
  gate = gate > limit ? limit : gate;
  up = up > limit ? limit : (up < -limit ? -limit : up);
  const float glu = gate * (1.0f / (1.0f + expf(-(gate * 1.702f))));
  return (up + 1.0f) * glu;
}

// Expert GEMV on MFMA.  A workgroup streams `tpw` consecutive 64-row tiles of
// one active expert; wave w owns rows [16w, 16w + 16) of each tile over the
// whole input dimension.  Per 4-group step a lane holds the 16 code bytes of
// (row l % 16, group 4s + l/16) -- the A operand of four
// v_mfma_f32_16x16x32_bf16 (k = 8 * (l/16) + i) once decoded -- and reads the
// matching B operand from activation rows staged once in LDS as bfloat16.
//
// Weight chunks stream through a ring of kRing registers: step s's slot is
// refilled with the chunk kRing steps ahead (in this tile or the next) right
// after it is consumed, so every wave keeps kRing KiB of HBM reads in flight
// across tile boundaries.  kSteps is a template constant and every load is
// unconditional straight-line code, which lets the compiler wait for exactly
// one chunk per step (vector loads retire in order).  Past the last tile the
// refills are out-of-range buffer loads (they return 0 and touch no memory).
// The activation-row loads are issued before the ring prologue, so waiting
// for them (the oldest loads) does not wait for any weight chunk.
//
// Columns are up to kVRows activation rows.  gate_up stages one row per token
// (the bfloat16 hidden state, exact).  down stages two rows per token, the hi
// and lo bfloat16 planes written by gate_up (hi = bf16(y), lo = bf16(y - hi)),
// so the float32 SwiGLU output enters the product with a 2^-17 residual.  A
// unit therefore holds 4 tokens in down and 8 in gate_up.
constexpr int kRing = 8;  // every compiled kSteps >= kRing is a multiple of it (slot s % kRing is step s of any tile)

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
  const int in_dim = groups * 32;
  const int cpr = groups * 4;                   // 16-byte activation chunks per row
  const int row_stride = kSteps * 128 + 8;      // bf16 elements per staged row (zero padded)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int lr = lane & 15;                     // row within the wave's 16 (A) / column n (B, D)
  const int lq = lane >> 4;                     // k-quarter: groups 4s + lq
  constexpr int kLoads = (kVRows * kSteps * 16 + kGemvThreads - 1) / kGemvThreads;  // staging chunks per thread
  constexpr int kR = kRing < kSteps ? kRing : kSteps;
  static_assert(kSteps % kR == 0, "the ring must divide the step count");
  static_assert(kUnitTokensGateUp <= kVRows && 2 * kUnitTokensDown <= kVRows, "a unit's rows fit one pass");
  const int trow = wave * 16 + lr;              // row inside a 64-row tile
  const int rec = ((groups + 3) / 4 + 7) / 8 * 8;
  const uint32_t tile_bytes = (uint32_t)groups * 1024u;
  // the expert matrix as a buffer: weight chunks and scale records are read
  // with a per-lane VGPR offset and a uniform (SGPR) step offset
  const __amdgpu_buffer_rsrc_t wbuf = __builtin_amdgcn_make_buffer_rsrc(
      (void*)wmat, (short)0, (int)packed_matrix_bytes(rows, groups), kBufferWord3);
  // chunk of step t in a tile = tile offset + 4096 t + voff.  kSteps is a
  // multiple of the ring size and may exceed the real step count g4: lanes
  // whose group 4t + lq is past the last group read out of range (0, no
  // memory traffic) and decode with scale 0.
  const int g4 = (groups + 3) >> 2;
  const uint32_t voff = (uint32_t)(lq * 1024 + trow * 16);
  const uint32_t voff_tail = 4 * (g4 - 1) + lq < groups ? voff : kOutOfRange;  // step g4 - 1
  auto chunk = [&](uint32_t tile_off, int t, bool valid) -> u32x4_t {
    const uint32_t v = !valid || t >= g4 ? kOutOfRange : (t == g4 - 1 ? voff_tail : voff);
    return __builtin_amdgcn_raw_buffer_load_b128(wbuf, v, tile_off + 4096u * t, kStreamPolicy);
  };
  const uint32_t scale_base = (uint32_t)packed_block_bytes(rows, groups);

  {
    const int nrows = kDown ? 2 * nt : nt;

    // ---- 1. the unit's pairs: one vector load, issued before the weight
    //      stream so that waiting for it does not wait for any weight chunk.
    //      Lane r < kVRows holds staged row r's pair; the lane's output pair
    //      (the same for every tile) comes in the same round trip. ----
    const int rr_l = min(lane & (kVRows - 1), nrows - 1);
    const int pair_l = pairs[pb + tc + (kDown ? rr_l >> 1 : rr_l)];
    const int out_col = kDown ? lr >> 1 : lr;  // the lane's token within the unit
    const int out_pair = pairs[pb + tc + min(out_col, nt - 1)];

    // ---- 2. scale record of the first tile, the first tile's bias, then the
    //      ring prologue ----
    // the lane's scales of a tile: 8-byte word i holds steps 8i .. 8i + 7 of
    // (row, quarter); a wave's load of word i is 512 contiguous bytes
    constexpr int kRecWords = (kSteps + 7) / 8 * 2;
    auto load_rec = [&](int tile, uint32_t* dst) {
#pragma unroll
      for (int i = 0; i < kRecWords / 2; ++i) {
        const uint32_t off = (uint32_t)packed_scale_word(groups, tile * kTileRows + trow, min(i, rec / 8 - 1), lq);
        const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(wbuf, off, scale_base, kStreamPolicy);
        dst[2 * i] = v.x;
        dst[2 * i + 1] = v.y;
      }
    };
    // Epilogue operands are loaded ahead too: the bias of the lane's 4 rows
    // one tile ahead, next to the scale record.  A load issued in the
    // epilogue itself would be the youngest in flight, and waiting for it
    // would drain the weight ring.
    auto load_bias = [&](int tile) -> u32x2_t {
      const int64_t row = (int64_t)e * rows + tile * kTileRows + wave * 16 + 4 * lq;
      return *reinterpret_cast<const u32x2_t*>(bias + row);
    };
    uint32_t sc[kRecWords], sc_next[kRecWords];
    load_rec(tile0, sc);
    u32x2_t bias_cur = load_bias(tile0), bias_next = bias_cur;
    uint32_t tb = (uint32_t)tile0 * tile_bytes;
    u32x4_t ring[kR];
    __builtin_amdgcn_sched_barrier(0);  // the ring goes out before the rows' loads
#pragma unroll
    for (int t = 0; t < kR; ++t) ring[t] = chunk(tb, t, true);
    __builtin_amdgcn_sched_barrier(0);

    // ---- 3. activation-row loads (row sources read back from the pairs) ----
    int src[kVRows];
    {
      const int src_l = kDown ? pair_l : pair_l / k_top;
#pragma unroll
      for (int r = 0; r < kVRows; ++r) src[r] = __builtin_amdgcn_readlane(src_l, r);
    }
    u32x4_t xv[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int id = min((int)threadIdx.x + i * kGemvThreads, nrows * cpr - 1);
      const int r = id / cpr;
      const int c = id - r * cpr;
      int srow = src[0];
#pragma unroll
      for (int q = 1; q < kVRows; ++q) srow = r == q ? src[q] : srow;
      const uint16_t* p = act + (kDown ? (r & 1) * act_plane : 0) + (int64_t)srow * in_dim + c * 8;
      xv[i] = *reinterpret_cast<const u32x4_t*>(p);
    }

    // ---- 4. activation rows into LDS ----
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int id = (int)threadIdx.x + i * kGemvThreads;
      const int r = id / cpr;
      const int c = id - r * cpr;
      // ids past the staged rows land in row 0's spare 16-byte slot, which nothing reads
      const int dst = id < nrows * cpr ? r * row_stride + c * 8 : row_stride - 8;
      *reinterpret_cast<u32x4_t*>(xs + dst) = xv[i];
    }
    {
      const int pad = kSteps * 128 - in_dim;  // zero: its A operand is zero, keep 0 * pad finite
      for (int i = threadIdx.x; i < nrows * pad; i += kGemvThreads) {
        const int r = i / pad;
        xs[r * row_stride + in_dim + (i - r * pad)] = 0;
      }
    }
    __syncthreads();

    // B operand rows: column n = lr reads staged row min(n, kVRows - 1) without
    // masking; columns past the live rows produce outputs nobody stores (an
    // MFMA output column depends only on its own B column)
    const uint16_t* xrow = xs + min(lr, kVRows - 1) * row_stride + lq * 32;
    for (int ti = 0; ti < ntile; ++ti) {
      const int tile = tile0 + ti;
      // refills past this tile read the next one; past the last tile they read
      // out of range (0, no memory traffic) at a valid tile offset
      const bool has_next = ti + 1 < ntile;
      const uint32_t nb = has_next ? tb + tile_bytes : tb;
      // the next tile's scale record is issued before the first refill that
      // reads the next tile, so waiting for it never waits for a ring load
      const int next_tile = has_next ? tile + 1 : tile;
      if constexpr (kSteps <= kR) {
        load_rec(next_tile, sc_next);
        bias_next = load_bias(next_tile);
      }

      f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
      // B operands are read one step ahead of their MFMAs (LDS latency)
      bf16x8_t bcur[4], bnext[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) bcur[j] = *reinterpret_cast<const bf16x8_t*>(xrow + j * 8);
#pragma unroll
      for (int s = 0; s < kSteps; ++s) {
        __builtin_amdgcn_sched_barrier(0);  // keep each step's decode next to its MFMAs
        if constexpr (kSteps > kR) {
          if (s == kSteps - kR) {
            load_rec(next_tile, sc_next);
            bias_next = load_bias(next_tile);
          }
        }
        // an empty asm "modifying" the chunk pins each step's decode right
        // here, so decoded operands (16 registers per step) are never
        // computed early and kept live across steps
        asm volatile("" : "+v"(ring[s % kR]));
        const u32x4_t w = ring[s % kR];
        {
          const int t = s + kR;  // refill: kR steps ahead
          ring[s % kR] = t < kSteps ? chunk(tb, t, true) : chunk(nb, t - kSteps, has_next);
        }
        if (s + 1 < kSteps) {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            bnext[j] = *reinterpret_cast<const bf16x8_t*>(xrow + (s + 1) * 128 + j * 8);
        }
        // 2^(e-127) as float32 bits (e = 0: the subnormal 2^-127; e = 255: inf,
        // which the conversion reads as the MX NaN scale); a lane past the
        // last group uses scale 0 (finite E2M1 values times 0 are +-0)
        const uint32_t eb = (sc[s >> 2] >> (8 * (s & 3))) & 0xffu;
        uint32_t sbits = eb == 0u ? 0x00400000u : (eb << 23);
        sbits = 4 * s + lq < groups ? sbits : 0u;
        const float scale = __uint_as_float(sbits);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const bf16x8_t a = decode8(w[j], scale);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bcur[j], acc, 0, 0, 0);
        }
        if (s + 1 < kSteps) {
#pragma unroll
          for (int j = 0; j < 4; ++j) bcur[j] = bnext[j];
        }
      }
      tb = nb;
#pragma unroll
      for (int i = 0; i < kRecWords; ++i) sc[i] = sc_next[i];
      // bias of rows row0 .. row0 + 3 as bfloat16 bits, low half first
      const float bias_row[4] = {bf16_to_f32(bias_cur.x & 0xffffu), bf16_to_f32(bias_cur.x >> 16),
                                 bf16_to_f32(bias_cur.y & 0xffffu), bf16_to_f32(bias_cur.y >> 16)};
      bias_cur = bias_next;

      // ---- epilogue: lane holds rows 4*lq + v (v = 0..3) of the wave's 16, column lr ----
      const int row0 = tile * kTileRows + wave * 16 + 4 * lq;
      float v[4] = {acc[0], acc[1], acc[2], acc[3]};
      if constexpr (!kDown) {
        if (lr < nt) {
          const int pair = out_pair;
          const int half = rows >> 1;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            float gate = v[2 * h], up = v[2 * h + 1];
            if (precision == KLC_PRECISION_BF16) {
              gate = round_bf16(gate);
              up = round_bf16(up);
            }
            gate += bias_row[2 * h];
            up += bias_row[2 * h + 1];
            const float y = swiglu(gate, up, limit);
            const int64_t idx = (int64_t)pair * half + (row0 >> 1) + h;
            if (out_raw) out_raw[idx] = y;
            // down input: hi/lo bfloat16 planes (lo = 0 when the reference rounds to bf16)
            const uint32_t hi = f32_to_bf16_rne(y);
            const uint32_t lo = precision == KLC_PRECISION_BF16 ? 0u : f32_to_bf16_rne(y - bf16_to_f32(hi));
            out_split[idx] = (uint16_t)hi;
            out_split[out_plane + idx] = (uint16_t)lo;
          }
        }
      } else {
        // column 2t holds the hi part of token t, column 2t + 1 the lo part
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] += __shfl_xor(v[i], 1);
        if ((lr & 1) == 0 && (lr >> 1) < nt) {
          const int pair = out_pair;
          float o[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float t = precision == KLC_PRECISION_BF16 ? round_bf16(v[i]) : v[i];
            o[i] = t + bias_row[i];
          }
          *reinterpret_cast<float4*>(out + (int64_t)pair * rows + row0) = make_float4(o[0], o[1], o[2], o[3]);
        }
      }
    }
  }
}

// Step counts with a compiled kernel; other shapes round up (the extra steps
// read out of range and decode to zero).  Each is <= kRing or a multiple of it.
constexpr int kStepSizes[] = {1, 2, 3, 4, 6, 8, 16, 24};

int gemv_steps(int groups) {
  const int g4 = (groups + 3) / 4;
  for (int s : kStepSizes)
    if (s >= g4) return s;
  return -1;
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

size_t gemv_lds_bytes(int steps) { return (size_t)kVRows * (steps * 128 + 8) * 2; }

// Tiles each workgroup streams: the unit capacity's tiles spread over about
// `target` workgroups (768 are resident at once: 3 per CU), so workgroups
// that finish early are replaced and the tail stays short; one tile per
// workgroup when few units exist.  max_units is an upper bound of the units.
// Measured at batches 64 and 128 (120B shape): gate_up is fastest with 2
// tiles per workgroup, down with 3 -- one tile per workgroup is much slower
// for both, since every workgroup start stages 8 activation rows and waits
// for a chain of index loads.
constexpr int64_t kGemvWorkgroupsUp = 6144, kGemvMaxTilesUp = 2;
constexpr int64_t kGemvWorkgroupsDown = 2304, kGemvMaxTilesDown = 3;

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
  KLC_REQUIRE(units_capacity(n_pairs, n_exp, kUnitTokensDown) <= 65535 && hidden <= 32 * 4 * kMaxSteps &&
                  inter <= 32 * 4 * kMaxSteps,
              KLC_ERR_UNSUPPORTED, "experts: unsupported sizes (hidden, inter <= %d, <= 65535 work units)",
              32 * 4 * kMaxSteps);
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

// The grouped GEMM pays off once experts see several MFMA column blocks of
// tokens; below about 8 tokens per expert the GEMV streams the same weights
// with less overhead.
bool use_gemm_path(int64_t n_pairs, int64_t n_exp) { return n_pairs >= 8 * n_exp; }

struct LayerScratch {
  int64_t counters, partials, logits, ids, values, weights, offsets, sorted, active, n_active, units, gated, eo, total;
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
  KLC_REQUIRE(path == KLC_PATH_AUTO || path == KLC_PATH_GEMV || path == KLC_PATH_GEMM, KLC_ERR_ARGUMENT,
              "%s: unknown path %d", fn, path);
  int rc = check_router_args(n_tokens, hidden, n_experts);
  if (rc) return rc;
  rc = check_topk_args(n_tokens, n_experts, k);
  if (rc) return rc;
  rc = check_gemv_shapes(hidden, inter, n_tokens * k, n_experts);
  if (rc) return rc;
  KLC_REQUIRE(n_tokens <= KLC_LAYER_MAX_TOKENS, KLC_ERR_UNSUPPORTED, "%s: n_tokens=%lld > 65535", fn, (long long)n_tokens);
  return KLC_OK;
}

// The layer's launches on scratch memory `ws` (layer_scratch layout, counters
// zero on entry and left zero).
int run_moe_layer(const void* x, const void* router_w, const void* router_b, const void* const* w_gate_up,
                  const void* gate_up_bias, const void* const* w_down, const void* down_bias, int64_t n_tokens,
                  int64_t hidden, int64_t inter, int64_t n_experts, int64_t k, float swiglu_limit, int precision,
                  int path, char* ws, void* out, const void* residual, int32_t* ids, void* weights,
                  void* const* events, void* stream) {
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

  if ((rc = mark(0))) return rc;
  if (n_tokens <= kDecodeRouterTokens) {
    // decode batches: logits, top-k and dispatch in one launch
    KLC_REQUIRE(decode_router_counters(n_tokens, n_experts) * 4 <= kCounterBytes, KLC_ERR_UNSUPPORTED,
                "klc_moe_layer: %lld experts need more completion counters than the workspace holds",
                (long long)n_experts);
    if ((rc = launch_router_decode(x, router_w, router_b, logits, n_tokens, hidden, n_experts, k, ids_buf, values,
                                   w_buf, offsets, sorted, active, n_active, units, counters,
                                   reinterpret_cast<double*>(ws + s.partials), st)))
      return rc;
    if ((rc = mark(1))) return rc;
    if ((rc = mark(2))) return rc;
  } else {
    if ((rc = launch_router_logits(x, router_w, router_b, logits, nullptr, n_tokens, hidden, n_experts, st)))
      return rc;
    if ((rc = mark(1))) return rc;
    if ((rc = launch_topk(logits, ids_buf, values, w_buf, n_tokens, n_experts, k, st))) return rc;
    if ((rc = mark(2))) return rc;
    if ((rc = launch_dispatch(ids_buf, n_tokens * k, n_experts, offsets, sorted, active, n_active, units, st)))
      return rc;
  }
  if ((rc = mark(3))) return rc;
  const bool gemm = path == KLC_PATH_GEMM || (path == KLC_PATH_AUTO && use_gemm_path(n_tokens * k, n_experts));
  if (gemm) {
    if ((rc = launch_gemm_gate_up(w_gate_up, gate_up_bias, x, n_tokens, k, n_experts, offsets, sorted, units, hidden,
                                  inter, swiglu_limit, precision, gated, nullptr, st)))
      return rc;
    if ((rc = mark(4))) return rc;
    if ((rc = launch_gemm_down(w_down, down_bias, gated, n_tokens * k, n_experts, offsets, sorted, units, hidden,
                               inter, precision, eo, st)))
      return rc;
  } else {
    if ((rc = launch_gate_up(w_gate_up, gate_up_bias, x, n_tokens, k, n_experts, offsets, sorted, units, hidden,
                             inter, swiglu_limit, precision, gated, nullptr, st)))
      return rc;
    if ((rc = mark(4))) return rc;
    if ((rc = launch_down(w_down, down_bias, gated, n_tokens * k, n_experts, offsets, sorted, units, hidden, inter,
                          precision, eo, st)))
      return rc;
  }
  if ((rc = mark(5))) return rc;
  if ((rc = launch_combine(eo, w_buf, residual, n_tokens, k, hidden, out, st))) return rc;
  return mark(6);
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
                       weights, events, stream);
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
                       n_experts, k, swiglu_limit, precision, path, ws, out, residual, ids, weights, events, stream);
}
