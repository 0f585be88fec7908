// Decode-path expert GEMV (gfx950): one work unit's pass over consecutive
// 64-row tiles of one packed MXFP4 expert matrix.  Shared by the standalone
// GEMV kernels (klc_experts.hip) and the fused small-batch decode layer
// (klc_decode.hip).
//
// Mapping.  Wave w of the 256-thread workgroup owns rows [16w, 16w + 16) of
// each tile over the whole input dimension.  Per 4-group step a lane holds
// the 16 code bytes of (row l % 16, group 4s + l/16) -- the A operand of four
// v_mfma_f32_16x16x32_bf16 (k = 8 * (l/16) + i) once decoded by
// v_cvt_scalef32_pk_bf16_fp4 (E2M1 times the E8M0 scale, exact) -- and reads
// the matching B operand from activation rows staged once in LDS as bfloat16.
//
// Weight chunks stream through a ring of kRing registers: step s's slot is
// refilled with the chunk kRing steps ahead (in this tile or the next) right
// after it is consumed, so every wave keeps kRing KiB of HBM reads in flight
// across tile boundaries.  kSteps is a template constant and every load is
// unconditional straight-line code, which lets the compiler wait for exactly
// one chunk per step (vector loads retire in order).  Past the last tile the
// refills are out-of-range buffer loads (they return 0 and touch no memory).
// The activation rows go to LDS by buffer-to-LDS DMA issued before the ring
// prologue, so waiting for them (the oldest loads) waits for no weight chunk
// (the fused layer, whose down items wait for their inputs after starting
// their weight stream, stages them through registers after the ring).
//
// Columns are up to kVRows activation rows.  gate_up stages one row per token
// (the bfloat16 hidden state, exact).  down stages two rows per token, the hi
// and lo bfloat16 planes written by gate_up (hi = bf16(y), lo = bf16(y - hi)),
// so the float32 SwiGLU output enters the product with a 2^-17 residual.  A
// unit therefore holds 4 tokens in down and 8 in gate_up.
#pragma once

#include "klc_common.h"

namespace klc {
namespace {

constexpr int kGemvWaves = 4;                 // 4 x 16 rows = one 64-row tile per workgroup
constexpr int kGemvThreads = kGemvWaves * kWave;
constexpr int kVRows = 8;                     // activation rows (MFMA N columns) staged per unit
constexpr int kMaxSteps = 24;                 // 4-group steps per row (inputs <= 3072)
constexpr int kRing = 8;  // every compiled kSteps >= kRing is a multiple of it (slot s % kRing is step s of any tile)

typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float swiglu(float gate, float up, float limit) {
  // streamed_moe_router.py:524-529; comparisons keep NaN like torch.clamp
  gate = gate > limit ? limit : gate;
  up = up > limit ? limit : (up < -limit ? -limit : up);
  const float glu = gate * (1.0f / (1.0f + expf(-(gate * 1.702f))));
  return (up + 1.0f) * glu;
}

// Staged activation rows in LDS: each row holds its 16-byte chunks rounded
// up to whole 64-chunk blocks (one wave-wide LDS-DMA load fills one block)
// plus one spare chunk, so consecutive rows start 16 bytes apart modulo 256
// and the B reads of the 8 rows at one offset hit different banks.
__host__ __device__ constexpr int gemv_row_chunks(int steps) { return (steps * 16 + 63) / 64 * 64; }
__host__ __device__ constexpr int gemv_row_stride(int steps) { return (gemv_row_chunks(steps) + 1) * 8; }  // bf16
__host__ __device__ constexpr size_t gemv_lds_bytes(int steps) { return (size_t)kVRows * gemv_row_stride(steps) * 2; }

// Step counts with a compiled kernel; other shapes round up (the extra steps
// read out of range and decode to zero).  Each is <= kRing or a multiple of it.
constexpr int kStepSizes[] = {1, 2, 3, 4, 6, 8, 16, 24};

inline int gemv_steps(int groups) {
  const int g4 = (groups + 3) / 4;
  for (int s : kStepSizes)
    if (s >= g4) return s;
  return -1;
}

struct NoWait {
  __device__ void operator()() const {}
};

// One unit's pass over tiles [tile0, tile0 + ntile) of expert matrix `wmat`
// (packed row-tile layout, `rows` x `groups`).  unit_pairs[0 .. nt) are the
// unit's (token, slot) pairs in expert-sorted order; `e` is the expert (for
// its bias rows).  gate_up (kDown false) reads the tokens' rows of `act`
// ([tokens][in] bfloat16) and writes the SwiGLU output as hi/lo bfloat16
// planes (out_split, planes out_plane elements apart) and optionally as
// float32 (out_raw); down reads the pairs' hi/lo rows of `act` (planes
// act_plane apart) and writes float32 outputs (out, [pairs][rows]).
//
// kFused: the fused decode layer's form.  Outputs are stored at agent scope
// (the consumers run on other XCDs of the same launch), down reads its input
// rows at agent scope, out_raw is not written, and wait_inputs() is called
// after the weight ring's prologue and before the input rows are read (down
// waits there for the gate_up workgroups that produce them).  xs: the
// workgroup's gemv_lds_bytes(kSteps) bytes of LDS, 16-byte aligned.
template <bool kDown, int kSteps, bool kFused, int kRingDepth = kRing, typename WaitFn = NoWait>
__device__ __forceinline__ void gemv_unit(const uint8_t* __restrict__ wmat, const uint16_t* __restrict__ bias, int e,
                                          const uint16_t* __restrict__ act, int64_t act_plane, float* __restrict__ out,
                                          uint16_t* __restrict__ out_split, int64_t out_plane,
                                          float* __restrict__ out_raw, const int32_t* unit_pairs, int nt, int rows,
                                          int groups, int k_top, float limit, int precision, int tile0, int ntile,
                                          uint16_t* xs, WaitFn wait_inputs) {
  // the thread index, opaque to the compiler: everything derived from it is
  // computed here rather than hoisted out of a caller's loop over units
  // (which would keep those values live across the whole loop)
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int in_dim = groups * 32;
  const int cpr = groups * 4;                   // 16-byte activation chunks per row
  constexpr int row_stride = gemv_row_stride(kSteps);  // bf16 elements per staged row (zero padded)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int lr = lane & 15;                     // row within the wave's 16 (A) / column n (B, D)
  const int lq = lane >> 4;                     // k-quarter: groups 4s + lq
  constexpr int kLoads = (kVRows * kSteps * 16 + kGemvThreads - 1) / kGemvThreads;  // staging chunks per thread
  constexpr int kR = kRingDepth < kSteps ? kRingDepth : kSteps;
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
  // memory traffic); their scale byte is record padding (0), so they decode
  // to 0 * 2^-127 = 0.
  const int g4 = (groups + 3) >> 2;
  const uint32_t voff = (uint32_t)(lq * 1024 + trow * 16);
  const uint32_t voff_tail = 4 * (g4 - 1) + lq < groups ? voff : kOutOfRange;  // step g4 - 1
  auto chunk = [&](uint32_t tile_off, int t, bool valid) -> u32x4_t {
    const uint32_t v = !valid || t >= g4 ? kOutOfRange : (t == g4 - 1 ? voff_tail : voff);
    return __builtin_amdgcn_raw_buffer_load_b128(wbuf, v, tile_off + 4096u * t, kStreamPolicy);
  };
  const uint32_t scale_base = (uint32_t)packed_block_bytes(rows, groups);

  const int nrows = kDown ? 2 * nt : nt;
  const int out_col = kDown ? lr >> 1 : lr;  // the lane's token within the unit
  // Lane r < kVRows holds staged row r's pair; every lane its output pair
  // (the same for every tile); one vector load each, issued together.
  const int rr_l = min(lane & (kVRows - 1), nrows - 1);
  const int pair_l = unit_pairs[kDown ? rr_l >> 1 : rr_l];
  const int out_pair = unit_pairs[min(out_col, nt - 1)];

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
  u32x2_t bias_cur, bias_next;
  uint32_t tb = (uint32_t)tile0 * tile_bytes;
  u32x4_t ring[kR];

  if constexpr (!kFused) {
    // scale record and bias of the first tile first: the only loads issued
    // between the rows' DMA and the wait for it are then the ring's, whose
    // count is fixed (a load the compiler moved past the wait, as it may
    // move one whose only use is in a later block, would be counted wrongly)
    load_rec(tile0, sc);
    bias_cur = load_bias(tile0);
    bias_next = bias_cur;
    __builtin_amdgcn_sched_barrier(0);
    // ---- activation rows by LDS-DMA, before any weight chunk: waiting for
    //      them then waits for no weight chunk.  Row r's
    //      64-chunk block b is one wave-wide buffer load into LDS (lane l
    //      writes chunk 64 b + l); chunks past the row and rows past the
    //      unit's are out of range (no memory traffic).  The pad chunks of
    //      live rows are also zeroed by ds_write: their A operand is zero,
    //      and 0 * pad must stay finite. ----
    constexpr int kBlocks = gemv_row_chunks(kSteps) / 64;
    static_assert((kVRows * kBlocks) % kGemvWaves == 0, "row blocks split evenly over the waves");
    const int src_l = kDown ? pair_l : pair_l / k_top;
#pragma unroll
    for (int m = 0; m < kVRows * kBlocks / kGemvWaves; ++m) {
      const int i = wave + kGemvWaves * m;  // uniform
      const int r = i / kBlocks;
      const int b = i - r * kBlocks;
      const int srow = __builtin_amdgcn_readlane(src_l, r);
      const uint16_t* row = act + (kDown ? (r & 1) * act_plane : 0) + (int64_t)srow * in_dim;
      const __amdgpu_buffer_rsrc_t rbuf = __builtin_amdgcn_make_buffer_rsrc(
          (void*)row, (short)0, r < nrows ? cpr * 16 : 0, kBufferWord3);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rbuf, (__attribute__((address_space(3))) void*)(xs + r * row_stride + b * 512), 16,
          (uint32_t)((b * 64 + lane) * 16), 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int r = tid >> 5;
      const int c = cpr + (tid & 31) + 32 * j;
      if (r < nrows && c < gemv_row_chunks(kSteps)) *reinterpret_cast<u32x4_t*>(xs + r * row_stride + c * 8) = u32x4_t{0u, 0u, 0u, 0u};
    }
    __builtin_amdgcn_sched_barrier(0);
    // ---- the ring prologue ----
#pragma unroll
    for (int t = 0; t < kR; ++t) ring[t] = chunk(tb, t, true);
    __builtin_amdgcn_sched_barrier(0);
    // every wave's rows have landed (the ring's loads after them stay in flight)
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(kR));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  } else {
    // ---- the fused layer's order: scale record, bias, ring prologue, then
    //      (after wait_inputs) the activation rows through registers ----
    load_rec(tile0, sc);
    bias_cur = load_bias(tile0);
    bias_next = bias_cur;
    __builtin_amdgcn_sched_barrier(0);  // the ring goes out before the rows' loads
#pragma unroll
    for (int t = 0; t < kR; ++t) ring[t] = chunk(tb, t, true);
    __builtin_amdgcn_sched_barrier(0);

    wait_inputs();

    int src[kVRows];
    {
      const int src_l = kDown ? pair_l : pair_l / k_top;
#pragma unroll
      for (int r = 0; r < kVRows; ++r) src[r] = __builtin_amdgcn_readlane(src_l, r);
    }
    u32x4_t xv[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int id = min(tid + i * kGemvThreads, nrows * cpr - 1);
      const int r = id / cpr;
      const int c = id - r * cpr;
      int srow = src[0];
#pragma unroll
      for (int q = 1; q < kVRows; ++q) srow = r == q ? src[q] : srow;
      const int64_t elem = (kDown ? (r & 1) * act_plane : 0) + (int64_t)srow * in_dim + c * 8;
      if constexpr (kDown) {
        // the hi/lo rows were stored by other workgroups of this launch
        const __amdgpu_buffer_rsrc_t abuf =
            __builtin_amdgcn_make_buffer_rsrc((void*)act, (short)0, 0x7fffffff, kBufferWord3);
        xv[i] = __builtin_amdgcn_raw_buffer_load_b128(abuf, (uint32_t)(elem * 2), 0, kAgentScope);
      } else {
        xv[i] = *reinterpret_cast<const u32x4_t*>(act + elem);
      }
    }
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int id = tid + i * kGemvThreads;
      const int r = id / cpr;
      const int c = id - r * cpr;
      // ids past the staged rows land in row 0's spare 16-byte slot, which nothing reads
      const int dst = id < nrows * cpr ? r * row_stride + c * 8 : row_stride - 8;
      *reinterpret_cast<u32x4_t*>(xs + dst) = xv[i];
    }
    {
      const int pad = kSteps * 128 - in_dim;  // zero: its A operand is zero, keep 0 * pad finite
      for (int i = tid; i < nrows * pad; i += kGemvThreads) {
        const int r = i / pad;
        xs[r * row_stride + in_dim + (i - r * pad)] = 0;
      }
    }
    __syncthreads();
  }

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
      // 2^(e-127) as float32 by v_ldexp_f32: e = 0 gives the subnormal
      // 2^-127, e = 255 gives inf, which the conversion reads as the MX NaN
      // scale.  A lane past the last group reads out-of-range codes (0) and
      // its scale byte is record padding, 0 in the packed layout: 0 * 2^-127.
      const int eb = (int)((sc[s >> 2] >> (8 * (s & 3))) & 0xffu);
      const float scale = __builtin_amdgcn_ldexpf(1.0f, eb - 127);
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
      // Lane (lq, lr) holds rows 4 lq .. 4 lq + 3 = (gate, up) of outputs
      // 2 lq and 2 lq + 1 (h = 0, 1) for token lr.  Tokens are < 8, so the
      // lanes lr >= 8 are free: they take output h = 1 of token lr - 8
      // (row_shr:8 inside each 16-lane row), and every active lane evaluates
      // one SwiGLU instead of two.
      static_assert(kUnitTokensGateUp <= 8, "gate_up tokens fit lanes 0-7 of a row");
      const int hs = lr >> 3;
      const float g1 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v[2]), 0x118, 0xf, 0xf, false));
      const float u1 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v[3]), 0x118, 0xf, 0xf, false));
      float gate = hs ? g1 : v[0], up = hs ? u1 : v[1];
      if (precision == KLC_PRECISION_BF16) {
        gate = round_bf16(gate);
        up = round_bf16(up);
      }
      gate += hs ? bias_row[2] : bias_row[0];
      up += hs ? bias_row[3] : bias_row[1];
      const float y = swiglu(gate, up, limit);
      // down input: hi/lo bfloat16 planes (lo = 0 when the reference rounds to bf16)
      const uint32_t hi = f32_to_bf16_rne(y);
      const uint32_t lo = precision == KLC_PRECISION_BF16 ? 0u : f32_to_bf16_rne(y - bf16_to_f32(hi));
      // lane lr < 8 collects h = 1 back from lane lr + 8 (row_shl:8)
      const uint32_t hi_1 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)hi, 0x108, 0xf, 0xf, false);
      const uint32_t lo_1 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)lo, 0x108, 0xf, 0xf, false);
      const float y_1 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(y), 0x108, 0xf, 0xf, false));
      if (lr < nt) {
        const int half = rows >> 1;
        // outputs (row0 / 2, row0 / 2 + 1) of the pair: one 4-byte word per
        // plane (row0 is a multiple of 4 and half is even)
        const int64_t idx = (int64_t)out_pair * half + (row0 >> 1);
        const uint32_t hi2 = hi | (hi_1 << 16), lo2 = lo | (lo_1 << 16);
        uint32_t* p = reinterpret_cast<uint32_t*>(out_split + idx);
        uint32_t* q = reinterpret_cast<uint32_t*>(out_split + out_plane + idx);
        if constexpr (kFused) {
          __hip_atomic_store(p, hi2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(q, lo2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
          if (out_raw) *reinterpret_cast<float2*>(out_raw + idx) = make_float2(y, y_1);
          *p = hi2;
          *q = lo2;
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
        if constexpr (kFused) {
          const __amdgpu_buffer_rsrc_t obuf =
              __builtin_amdgcn_make_buffer_rsrc((void*)out, (short)0, 0x7fffffff, kBufferWord3);
          const u32x4_t ov = {__float_as_uint(o[0]), __float_as_uint(o[1]), __float_as_uint(o[2]),
                              __float_as_uint(o[3])};
          __builtin_amdgcn_raw_buffer_store_b128(ov, obuf, (uint32_t)(((int64_t)pair * rows + row0) * 4), 0,
                                                 kAgentScope);
        } else {
          *reinterpret_cast<float4*>(out + (int64_t)pair * rows + row0) = make_float4(o[0], o[1], o[2], o[3]);
        }
      }
    }
  }
}

}  // namespace
}  // namespace klc
