// Prefill path: expert-grouped GEMM on MFMA (gfx950).
//
// For batches that give experts many tokens, each expert's weights are read
// once per 64-token unit and multiplied into all of the unit's tokens:
// a workgroup owns one GEMM unit (up to 64 tokens of one expert, from the
// dispatch) and 256 output rows (4 waves, each one 64-row packed tile, i.e.
// 4 row blocks of 16).  Per 128-deep k step every wave decodes its A chunks
// (MXFP4 -> bfloat16 with v_cvt_scalef32_pk_bf16_fp4, exact) and multiplies
// them with v_mfma_f32_16x16x32_bf16 into each 16-token column block of B.
//
// Both operand streams run kRing - 1 steps ahead of the MFMAs: A (per wave)
// in a register ring, B (shared by the 4 waves) in an LDS ring filled by
// global_load_lds_dwordx4, which writes lane l's 16 bytes at the
// instruction's LDS base + 16 l.  One instruction fills 4 token rows of 256
// bytes; the 16-byte piece q of row r sits in slot q ^ (r % 16), so the B
// reads of 16 consecutive rows at one piece hit 16 different slots (all 64
// banks).  A step waits once for its own loads (vector memory operations
// complete in order, so the later steps' loads stay in flight) and passes
// one barrier.  The products are exact and the sums run in float32, like
// the decode GEMVs, so both paths meet the same tolerance; gate_up reads the
// bfloat16 hidden state as is, down reads the float32 SwiGLU output as hi +
// lo bfloat16 planes (relative residual 2^-17).
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
// 8 activations of its token, piece 4 q + j of its row.
#include "klc_common.h"

namespace klc {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

// Waves (64-row tiles) per workgroup.  8 waves (512 rows) halve the B rows
// each wave stages per step but were slower (gate_up 467-478 -> 480-496 us,
// down 363-372 -> 381-398 us on the 2048-token layer): all 8 waves of a CU
// then meet at one barrier every step.
#ifndef KLC_GEMM_WAVES
#define KLC_GEMM_WAVES 4
#endif
#ifndef KLC_GEMM_WAVE_TILES
#define KLC_GEMM_WAVE_TILES 1
#endif
constexpr int kGemmWaves = KLC_GEMM_WAVES;
constexpr int kWaveTiles = KLC_GEMM_WAVE_TILES;     // 64-row packed tiles per wave
constexpr int kRb = 4 * kWaveTiles;                 // 16-row MFMA blocks per wave
constexpr int kGemmThreads = kGemmWaves * kWave;
constexpr int kGemmRows = kGemmWaves * kWaveTiles * kTileRows;  // output rows per workgroup
constexpr int kBRowsPerWave = kUnitTokensGemm / kGemmWaves;  // token rows each wave stages per step
constexpr int kBInstr = kBRowsPerWave / 4;          // LDS-DMA instructions per wave, plane and step (4 rows each)
static_assert(kBInstr >= 1 && kBRowsPerWave % 4 == 0, "token rows split evenly over the waves");
constexpr int kYStride = kGemmRows / 2 + 1;         // gate_up epilogue: floats per token row (odd: spreads the banks)
constexpr int kGemmCb = kUnitTokensGemm / 16;       // 4 column blocks of 16 tokens
template <int N>
struct ColumnBlocks {
  static constexpr int value = N;
};
constexpr int kXcds = 8;  // accelerator complex dies of an MI355X, each with its own L2
// Ring depths (steps in flight + 1).  gate_up: 3 keeps the kernel within
// 256 VGPRs without spilling (4 measured the same and spills 20 bytes).
#ifndef KLC_GEMM_RING_UP
#define KLC_GEMM_RING_UP 3
#endif
#ifndef KLC_GEMM_RING_DOWN
#define KLC_GEMM_RING_DOWN 2
#endif


__device__ __forceinline__ float swiglu(float gate, float up, float limit) {
  // streamed_moe_router.py:524-529; comparisons keep NaN like torch.clamp.
  // The sigmoid uses the hardware exp2 and reciprocal (a few ulp, far inside
  // the expert-output tolerance).
  gate = gate > limit ? limit : gate;
  up = up > limit ? limit : (up < -limit ? -limit : up);
  const float glu = gate * __builtin_amdgcn_rcpf(1.0f + __expf(-(gate * 1.702f)));
  return (up + 1.0f) * glu;
}

// One GEMM unit x one 256-row tile.  gate_up: act = bfloat16 hidden state
// [n_tok][in], one plane; writes the down input as hi/lo bfloat16 planes
// [2][pairs][in_down] (and float32 SwiGLU output to out_raw if set).  down:
// act = those planes (rows by pair); writes float32 expert outputs.

// Step barrier of the LDS ring.  Each wave first waits for its own step-s
// loads (vmcnt) and its LDS reads (lgkmcnt 0); the barrier then orders every
// wave's B rows before any wave's reads, and the acquire fence keeps the
// compiler from moving LDS reads above it.  (__syncthreads' release fence
// would wait for every outstanding LDS-DMA, i.e. for all later steps too.)
template <int kOutstanding>
__device__ __forceinline__ void ring_barrier() {
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(kOutstanding));
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// kPl: activation planes of B (gate_up 1; down 2 = hi + lo of the float32
// SwiGLU output, or 1 = its bfloat16 rounding, which is exactly the
// bfloat16-precision input, so the lo plane's zero products are skipped).
template <bool kDown, int kPl>
__host__ __device__ constexpr int gemm_ring() { return kDown && kPl == 2 ? KLC_GEMM_RING_DOWN : KLC_GEMM_RING_UP; }
template <bool kDown, int kPl>
__host__ __device__ constexpr int gemm_stage_bytes() { return kPl * kUnitTokensGemm * 256; }
// Each wave's tile of scale records copied into LDS (the packed layout,
// [S / 8][64 rows][4 quarters][8 bytes], at most 6 KiB for inputs <= 3072),
// where two workgroups of a CU still fit (not beside the two-plane down
// ring: that one keeps the records in registers).
constexpr int kScaleTileLds = kTileRows * 4 * 24;
constexpr int kScaleLdsBytes = kGemmWaves * kWaveTiles * kScaleTileLds;
template <bool kDown, int kPl>
__host__ __device__ constexpr bool gemm_scales_in_lds() { return !(kDown && kPl == 2); }
// LDS of one workgroup: the B ring, or the gate_up epilogue's output tile if
// larger, then the staged scales.
template <bool kDown, int kPl>
__host__ __device__ constexpr int gemm_lds_bytes() {
  const int ring = gemm_ring<kDown, kPl>() * gemm_stage_bytes<kDown, kPl>();
  const int tile = kDown ? 0 : kUnitTokensGemm * kYStride * 4;
  return (ring > tile ? ring : tile) + (gemm_scales_in_lds<kDown, kPl>() ? kScaleLdsBytes : 0);
}
static_assert(2 * gemm_lds_bytes<false, 1>() <= 160 * 1024 && 2 * gemm_lds_bytes<true, 1>() <= 160 * 1024 &&
                  2 * gemm_lds_bytes<true, 2>() <= 160 * 1024,
              "two workgroups per CU");

// One GEMM unit x one 256-row tile.  gate_up: act = bfloat16 hidden state
// [n_tok][in], one plane; writes the down input as hi/lo bfloat16 planes
// [2][pairs][in_down] (and float32 SwiGLU output to out_raw if set).  down:
// act = those planes (rows by pair); writes float32 expert outputs.
// kWide: activation planes past 2 GiB (rows addressed with 64-bit pointers
// instead of a buffer's 32-bit offsets).
template <bool kDown, int kPl, bool kWide>
__device__ __forceinline__ void moe_gemm_body(
    const uint8_t* const* __restrict__ wptr, const uint16_t* __restrict__ bias, const uint16_t* __restrict__ act,
    int64_t act_plane, float* __restrict__ out, uint16_t* __restrict__ out_split, int64_t out_plane,
    float* __restrict__ out_raw, const int32_t* __restrict__ offsets, const int32_t* __restrict__ pairs,
    const int32_t* __restrict__ units, const int32_t* __restrict__ n_units, int rows, int groups, int k_top,
    float limit, int precision, int row_wgs, int units_per_xcd) {
  static_assert(kPl == 1 || (kDown && kPl == 2), "gate_up reads one plane, down one or two");
  constexpr int kPlanes = kPl;
  constexpr int kRing = gemm_ring<kDown, kPl>();
  constexpr int kStage = gemm_stage_bytes<kDown, kPl>();  // one step: 64 token rows x 256 bytes per plane
  constexpr int kPlaneStage = kStage / kPlanes;
  constexpr int kLoadsPerStep = kRb + kBInstr * kPlanes;  // A: a chunk per row block; B: kBInstr per plane
  constexpr bool kScLds = gemm_scales_in_lds<kDown, kPl>();
  static_assert((kRing - 2) * kLoadsPerStep <= 63, "the ring's outstanding loads fit the vmcnt field");
  extern __shared__ __align__(16) uint8_t stage[];    // kRing x kStage

  // XCD-aware order: workgroups are handed to the 8 XCDs round-robin, so XCD
  // x = blockIdx.x % 8 runs units x, x + 8, ...; all row tiles of a unit run on
  // one XCD, which reads the unit's activation rows into its own L2 once.
  const int xcd = blockIdx.x % kXcds;
  const int j0 = blockIdx.x / kXcds;
  const int u = xcd + kXcds * (j0 / row_wgs);
  const int row_wg = j0 % row_wgs;
  if (j0 >= units_per_xcd * row_wgs || u >= *n_units) return;
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
  const int tile0 = (row_wg * kGemmWaves + wave) * kWaveTiles;  // the wave's first 64-row tile
  const bool wave_live = tile0 < tiles;
  const int in_dim = groups * 32;
  const int steps = (groups + 3) >> 2;

  // ---- B stream: wave w's LDS-DMA instruction i fills token rows 16 w + 4 i .. + 3;
  // lane l brings piece (l % 16) ^ (r % 16) of row r = 16 w + 4 i + l / 16.
  // Rows past the unit's tokens repeat its last token (their columns are
  // discarded); k past the input repeats its last piece (A is zero there). ----
  int64_t src_row[kBInstr];
  int piece[kBInstr];
#pragma unroll
  for (int i = 0; i < kBInstr; ++i) {
    const int r = kBRowsPerWave * wave + 4 * i + lq;
    const int p = pairs[pb + tc + min(r, nt - 1)];
    src_row[i] = (int64_t)(kDown ? p : p / k_top) * in_dim;
    piece[i] = lr ^ (r & 15);
  }
  // The lane's byte offset in its plane is a per-lane constant plus a uniform
  // step offset of 256 s bytes (no address arithmetic per step), with one
  // per-lane alternative for the last step, whose pieces past the input are
  // clamped (every address is inside the plane: planes < 2 GiB; larger ones
  // take the wide kernels).  (Two named resources: resource descriptors do not form arrays.)
  uint32_t boff[kBInstr], boff_last[kBInstr];
#pragma unroll
  for (int i = 0; i < kBInstr; ++i) {
    boff[i] = (uint32_t)((src_row[i] + piece[i] * 8) * 2);
    const int kl = min((steps - 1) * 128 + piece[i] * 8, in_dim - 8);
    boff_last[i] = (uint32_t)((src_row[i] + kl) * 2 - (int64_t)(steps - 1) * 256);
  }
  const __amdgpu_buffer_rsrc_t bbuf0 =
      __builtin_amdgcn_make_buffer_rsrc((void*)act, (short)0, 0x7fffffff, kBufferWord3);
  const __amdgpu_buffer_rsrc_t bbuf1 =
      __builtin_amdgcn_make_buffer_rsrc((void*)(act + (kPlanes > 1 ? act_plane : 0)), (short)0, 0x7fffffff, kBufferWord3);
  auto b_dma = [&](int s, int slot) {
    const int sc = min(s, steps - 1);
    const bool last = sc == steps - 1;
#pragma unroll
    for (int pl = 0; pl < kPlanes; ++pl) {
#pragma unroll
      for (int i = 0; i < kBInstr; ++i) {
        __attribute__((address_space(3))) void* dst =
            (__attribute__((address_space(3))) uint8_t*)stage + slot * kStage + pl * kPlaneStage + (kBRowsPerWave * wave + 4 * i) * 256;
        if constexpr (kWide) {
          const int kc = min(sc * 128 + piece[i] * 8, in_dim - 8);
          __builtin_amdgcn_global_load_lds(act + pl * act_plane + src_row[i] + kc, dst, 16, 0, 0);
        } else {
          __builtin_amdgcn_raw_ptr_buffer_load_lds(pl == 0 ? bbuf0 : bbuf1, dst, 16, last ? boff_last[i] : boff[i],
                                                   (uint32_t)sc * 256u, 0, 0);
        }
      }
    }
  };

  // ---- A stream: the wave's 64-row tile, 4 row blocks; steps past the end
  // load out of range (zeros, no traffic, no branch) ----
  // (a tile past the matrix reads tile 0's scales and no weights)
  const __amdgpu_buffer_rsrc_t wbuf = __builtin_amdgcn_make_buffer_rsrc(
      (void*)wptr[e], (short)0, (int)packed_matrix_bytes(rows, groups), kBufferWord3);
  int wtile[kWaveTiles];
  bool tile_live[kWaveTiles];
  uint32_t tile_off[kWaveTiles];
#pragma unroll
  for (int i = 0; i < kWaveTiles; ++i) {
    tile_live[i] = tile0 + i < tiles;
    wtile[i] = tile_live[i] ? tile0 + i : 0;
    tile_off[i] = (uint32_t)wtile[i] * (uint32_t)groups * 1024u;
  }
  // The epilogue's operands are loaded now, so that their latency passes
  // under the step loop: bias of the lane's rows (4 consecutive per row
  // block) and the pair ids of the token columns the lane writes.
  u32x2_t bias4[kRb];
#pragma unroll
  for (int rb = 0; rb < kRb; ++rb) {
    const int row0 = wtile[rb >> 2] * kTileRows + (rb & 3) * 16 + 4 * lq;
    bias4[rb] = *reinterpret_cast<const u32x2_t*>(bias + (int64_t)e * rows + row0);
  }
  int pcol[kGemmCb];
#pragma unroll
  for (int i = 0; i < kGemmCb; ++i) {
    // gate_up: the store loop's token c = tid / 16 + 16 i; down: column c = 16 i + lr
    const int c = kDown ? 16 * i + lr : (tid >> 4) + 16 * i;
    pcol[i] = pairs[pb + tc + min(c, nt - 1)];
  }

  const int rec = (int)packed_scale_record(groups);
  const uint32_t scale_base = (uint32_t)packed_block_bytes(rows, groups);
  // Two-plane down (scales in registers): the lane's scales for all steps
  // (one byte per step; inputs <= 3072 have <= 24 steps: three 8-byte words)
  // are loaded once: per-step 4-byte scale loads cost more issue time in the
  // texture unit than the weight chunks themselves.  (Words past a shorter
  // record repeat its last word.)
  // (three separately named arrays: the per-step choice among them is a
  // select, where one array indexed by a run-time word would go to scratch)
  u32x2_t srec0[kRb], srec1[kRb], srec2[kRb];
#pragma unroll
  for (int rb = 0; rb < kRb && !kScLds; ++rb) {
    const int row = wtile[rb >> 2] * kTileRows + (rb & 3) * 16 + lr;
    srec0[rb] = __builtin_amdgcn_raw_buffer_load_b64(wbuf, (uint32_t)packed_scale_word(groups, row, 0, lq), scale_base, 0);
    srec1[rb] = __builtin_amdgcn_raw_buffer_load_b64(
        wbuf, (uint32_t)packed_scale_word(groups, row, min(1, rec / 8 - 1), lq), scale_base, 0);
    srec2[rb] = __builtin_amdgcn_raw_buffer_load_b64(
        wbuf, (uint32_t)packed_scale_word(groups, row, min(2, rec / 8 - 1), lq), scale_base, 0);
  }
  // Scales in LDS: the wave copies its tile's records (rec / 4 KiB) with
  // buffer-to-LDS loads issued ahead of the ring's first steps (no register
  // round trip, so no wait); lane (lr, lq) of row block rb finds step s at
  // sc_lane[rb * 512 + (s / 8) * 2048 + s % 8].
  static_assert(kWaveTiles == 1, "one scale tile per wave");
  uint8_t* sc_lds = stage + (gemm_lds_bytes<kDown, kPl>() - kScaleLdsBytes) + wave * kScaleTileLds;
  const uint8_t* sc_lane = sc_lds + (lr * 4 + lq) * 8;
  if constexpr (kScLds) {
    // (inputs <= 3072 wide, checked by check_gemv_shapes: rec <= 24)
    const uint32_t tile_scales = scale_base + (uint32_t)wtile[0] * (uint32_t)(kTileRows * 4 * rec);
#pragma unroll
    for (int i = 0; i < kScaleTileLds / 1024; ++i)
      if (i < rec / 4)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wbuf, (__attribute__((address_space(3))) void*)(sc_lds + i * 1024), 16,
                                                 (uint32_t)(lane * 16 + i * 1024), tile_scales, 0, 0);
  }
  // The wave's 64-row tile as a buffer of its own (empty for a tile past the
  // matrix): the groups past the input and the steps past the last fall
  // outside it and load zeros (no traffic) by the range check alone, so a
  // step's loads cost one address add.
  const __amdgpu_buffer_rsrc_t abuf = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(wptr[e] + tile_off[0]), (short)0, tile_live[0] ? groups * 1024 : 0, kBufferWord3);
  const uint32_t aoff = (uint32_t)(lq * 1024 + lr * 16);
  auto a_load = [&](int s, u32x4_t (&a)[kRb]) {
    const uint32_t v = aoff + 4096u * (uint32_t)s;
#pragma unroll
    for (int rb = 0; rb < kRb; ++rb) a[rb] = __builtin_amdgcn_raw_buffer_load_b128(abuf, v, (uint32_t)(rb * 256), 0);
  };

  f32x4_t acc[kRb][kGemmCb];
#pragma unroll
  for (int rb = 0; rb < kRb; ++rb)
#pragma unroll
    for (int cb = 0; cb < kGemmCb; ++cb) acc[rb][cb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // B read offsets: lane (lr, lq) reads piece 4 lq + j of row 16 cb + lr
  // (kept as LDS pointers, one register each: every read of a step is then
  // one of them plus a constant offset, with no address add per step)
  typedef __attribute__((address_space(3))) const uint8_t* lds_cptr;
  lds_cptr b_ptr[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    b_ptr[j] = (lds_cptr)stage + lr * 256 + (((4 * lq + j) ^ lr) << 4);
    asm volatile("" : "+v"(b_ptr[j]));
  }

  // The lane's scale dword holding step s (4 steps per dword, at most 6 dwords).
  auto scale_words = [&](int s, uint32_t (&word)[kRb]) {
    const int d = min(s >> 2, 5);
#pragma unroll
    for (int rb = 0; rb < kRb; ++rb) {
      const u32x2_t pair = d >= 4 ? srec2[rb] : ((d & 2) ? srec1[rb] : srec0[rb]);
      word[rb] = (d & 1) ? pair.y : pair.x;
    }
  };

  // Step s for a unit of kNcb 16-token column blocks (a compile-time count,
  // so the MFMAs and their LDS reads are straight-line code the compiler can
  // pipeline; blocks past the unit's tokens are neither read nor multiplied).
  auto compute = [&](auto ncb_c, int s, int slot, const u32x4_t (&a_cur)[kRb], const uint32_t (&word)[kRb]) {
    constexpr int kNcb = decltype(ncb_c)::value;
    float scale[kRb];
    if constexpr (kScLds) {
      // E8M0 e -> 2^(e - 127) as float bits.  Past the last group of a
      // step the record's padding is 0 (2^-127, finite) and the codes load
      // as zeros.  Steps past the last one (the loop's padding) read the
      // last step's scales: their codes are zeros, so they add nothing (a
      // NaN scale there has already made the sum NaN).  No branch: the four
      // reads go out together.
      const int sc = min(s, steps - 1);
      const int soff = (sc >> 3) * 2048 + (sc & 7);
      uint32_t e8[kRb];
#pragma unroll
      for (int rb = 0; rb < kRb; ++rb) e8[rb] = sc_lane[rb * 512 + soff];
#pragma unroll
      for (int rb = 0; rb < kRb; ++rb) scale[rb] = __uint_as_float(max(e8[rb] << 23, 0x00400000u));
    } else {
      const bool live = 4 * s + lq < groups;
#pragma unroll
      for (int rb = 0; rb < kRb; ++rb) scale[rb] = cvt_scale_operand((word[rb] >> (8 * (s & 3))) & 0xffu, live);
    }
    // the B operands of a quarter are read one quarter ahead of their MFMAs
    bf16x8_t bq[2][kNcb][kPlanes];
    auto load_b = [&](int j, bf16x8_t (&dst)[kNcb][kPlanes]) {
#pragma unroll
      for (int cb = 0; cb < kNcb; ++cb)
#pragma unroll
        for (int pl = 0; pl < kPlanes; ++pl)
          dst[cb][pl] = *reinterpret_cast<__attribute__((address_space(3))) const bf16x8_t*>(
              b_ptr[j] + slot * kStage + pl * kPlaneStage + cb * 16 * 256);
    };
    load_b(0, bq[0]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (j < 3) load_b(j + 1, bq[(j + 1) & 1]);
      bf16x8_t a[kRb];
#pragma unroll
      for (int rb = 0; rb < kRb; ++rb) a[rb] = decode8(a_cur[rb][j], scale[rb]);
#pragma unroll
      for (int cb = 0; cb < kNcb; ++cb)
#pragma unroll
        for (int pl = 0; pl < kPlanes; ++pl)
#pragma unroll
          for (int rb = 0; rb < kRb; ++rb)
            acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[rb], bq[j & 1][cb][pl], acc[rb][cb], 0, 0, 0);
      if constexpr (kDown && kPlanes == 2) {
        // down (two planes): each quarter's B read, its kRb MFMAs and kRb VALU
        // instructions as one group, in order (330 against 345 us on the
        // 2048-token layer; the same grouping made gate_up spill and slower)
#pragma unroll
        for (int i = 0; i < kNcb * kPlanes; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // LDS read
          __builtin_amdgcn_sched_group_barrier(0x008, kRb, 0); // MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, kRb, 0); // VALU
        }
      }
    }
  };

  u32x4_t a_ring[kRing][kRb];
#pragma unroll
  for (int i = 0; i < kRing - 1; ++i) {
    a_load(i, a_ring[i]);
    b_dma(i, i);
  }

  // step s: wait for its own loads (the kRing - 2 later steps' stay in
  // flight), barrier (every wave's B rows of step s have landed and every
  // wave is done with step s - 1), issue step s + kRing - 1 into the slots
  // step s - 1 used, multiply.  Unrolled by kRing so slot indices are
  // constants, and run to a multiple of kRing steps with no branch around a
  // step (the steps past the end multiply zeros: A loads out of range and
  // its scales are 0), so no register of an in-flight load is copied.
  // The scale dwords are picked at a group's first step and again where a
  // step starts a new dword (s % 4 == 0); with kRing dividing 4 every group
  // starts at a multiple of kRing and needs only the first pick.
  const int steps_pad = (steps + kRing - 1) / kRing * kRing;
  auto run = [&](auto ncb_c) {
    for (int s0 = 0; s0 < steps_pad; s0 += kRing) {
      uint32_t word[kRb];
#pragma unroll
      for (int uu = 0; uu < kRing; ++uu) {
        const int s = s0 + uu;
        if (!kScLds && (uu == 0 || (4 % kRing != 0 && (s & 3) == 0))) scale_words(s, word);
        ring_barrier<(kRing - 2) * kLoadsPerStep>();
        a_load(s + kRing - 1, a_ring[(uu + kRing - 1) % kRing]);
        b_dma(s + kRing - 1, (uu + kRing - 1) % kRing);
        if (wave_live) compute(ncb_c, s, uu, a_ring[uu], word);
      }
    }
  };
  static_assert(kGemmCb == 4, "one loop per column-block count");
  switch (ncb) {  // uniform over the workgroup
    case 1: run(ColumnBlocks<1>{}); break;
    case 2: run(ColumnBlocks<2>{}); break;
    case 3: run(ColumnBlocks<3>{}); break;
    default: run(ColumnBlocks<4>{}); break;
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // no LDS-DMA may outlive the workgroup

  // ---- epilogue: lane holds rows rb * 16 + 4 lq + v of its tile, token column cb * 16 + lr ----
  if constexpr (!kDown) {
    // SwiGLU outputs of the workgroup (128 columns x up to 64 tokens) go
    // through LDS (the ring is idle now), so each token's 128 outputs leave
    // as 16-byte stores instead of 2-byte ones scattered over 16 rows
    static_assert(kUnitTokensGemm * kYStride * 4 <= gemm_lds_bytes<false, 1>(), "the output tile fits in the LDS");
    float* ytile = reinterpret_cast<float*>(stage);
    __syncthreads();  // every wave is done reading the ring
    if (wave_live) {
#pragma unroll
      for (int cb = 0; cb < kGemmCb; ++cb) {
        if (cb >= ncb) continue;
        const int c = cb * 16 + lr;
#pragma unroll
        for (int rb = 0; rb < kRb; ++rb) {
          if (!tile_live[rb >> 2]) continue;
          const f32x4_t v4 = acc[rb][cb];  // rows rb * 16 + 4 lq .. + 3 of the tile
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            float gate = v4[2 * h], up = v4[2 * h + 1];
            if (precision == KLC_PRECISION_BF16) {
              gate = round_bf16(gate);
              up = round_bf16(up);
            }
            const uint32_t b2 = h ? bias4[rb].y : bias4[rb].x;  // rows 4 lq + 2h, + 1
            gate += __uint_as_float(b2 << 16);
            up += __uint_as_float(b2 & 0xffff0000u);
            ytile[c * kYStride + wave * (kRb * 8) + rb * 8 + 2 * lq + h] = swiglu(gate, up, limit);
          }
        }
      }
    }
    __syncthreads();
    const int half = rows >> 1;
    const int col0 = row_wg * (kGemmRows / 2);
    const int ncols = min(kGemmRows / 2, half - col0);
    constexpr int kPieces = kGemmRows / 16;  // 8-column pieces of a token's outputs
    static_assert(kPieces == 16 && kUnitTokensGemm * kPieces == kGemmCb * kGemmThreads, "thread i covers token i / 16 + 16 it");
#pragma unroll
    for (int it = 0; it < kGemmCb; ++it) {  // (token, 8-column piece)
      const int i = tid + it * kGemmThreads;
      const int c = i / kPieces;
      const int ch = (i % kPieces) * 8;
      if (c >= nt || ch >= ncols) continue;
      const int p = pcol[it];
      float y[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) y[q] = ytile[c * kYStride + ch + q];
      uint32_t hi[4], lo[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t h2[2], l2[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          h2[t] = f32_to_bf16_rne(y[2 * q + t]);
          l2[t] = precision == KLC_PRECISION_BF16 ? 0u : f32_to_bf16_rne(y[2 * q + t] - bf16_to_f32(h2[t]));
        }
        hi[q] = h2[0] | (h2[1] << 16);
        lo[q] = l2[0] | (l2[1] << 16);
      }
      const int64_t idx = (int64_t)p * half + col0 + ch;  // half % 8 == 0: 16-byte aligned
      *reinterpret_cast<u32x4_t*>(out_split + idx) = u32x4_t{hi[0], hi[1], hi[2], hi[3]};
      *reinterpret_cast<u32x4_t*>(out_split + out_plane + idx) = u32x4_t{lo[0], lo[1], lo[2], lo[3]};
      if (out_raw) {
        reinterpret_cast<float4*>(out_raw + idx)[0] = make_float4(y[0], y[1], y[2], y[3]);
        reinterpret_cast<float4*>(out_raw + idx)[1] = make_float4(y[4], y[5], y[6], y[7]);
      }
    }
  } else {
    if (!wave_live) return;
#pragma unroll
    for (int cb = 0; cb < kGemmCb; ++cb) {
      if (cb >= ncb) continue;
      const int c = cb * 16 + lr;
      if (c >= nt) continue;
      const int p = pcol[cb];
#pragma unroll
      for (int rb = 0; rb < kRb; ++rb) {
        if (!tile_live[rb >> 2]) continue;
        const int row0 = tile0 * kTileRows + rb * 16 + 4 * lq;
        const f32x4_t v4 = acc[rb][cb];
        float o[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float t = precision == KLC_PRECISION_BF16 ? round_bf16(v4[v]) : v4[v];
          const uint32_t b2 = (v & 2) ? bias4[rb].y : bias4[rb].x;
          o[v] = t + __uint_as_float((v & 1) ? (b2 & 0xffff0000u) : (b2 << 16));
        }
        *reinterpret_cast<float4*>(out + (int64_t)p * rows + row0) = make_float4(o[0], o[1], o[2], o[3]);
      }
    }
  }
}

#ifndef KLC_GEMM_WAVES_PER_EU
#define KLC_GEMM_WAVES_PER_EU 2
#endif
// The kernels: planes below 2 GiB (every layer call) and past it.
template <bool kDown, int kPl>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(KLC_GEMM_WAVES_PER_EU))) void moe_gemm_kernel(
    const uint8_t* const* __restrict__ wptr, const uint16_t* __restrict__ bias, const uint16_t* __restrict__ act,
    int64_t act_plane, float* __restrict__ out, uint16_t* __restrict__ out_split, int64_t out_plane,
    float* __restrict__ out_raw, const int32_t* __restrict__ offsets, const int32_t* __restrict__ pairs,
    const int32_t* __restrict__ units, const int32_t* __restrict__ n_units, int rows, int groups, int k_top,
    float limit, int precision, int row_wgs, int units_per_xcd) {
  moe_gemm_body<kDown, kPl, false>(wptr, bias, act, act_plane, out, out_split, out_plane, out_raw, offsets, pairs,
                                   units, n_units, rows, groups, k_top, limit, precision, row_wgs, units_per_xcd);
}
template <bool kDown, int kPl>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(KLC_GEMM_WAVES_PER_EU))) void moe_gemm_wide_kernel(
    const uint8_t* const* __restrict__ wptr, const uint16_t* __restrict__ bias, const uint16_t* __restrict__ act,
    int64_t act_plane, float* __restrict__ out, uint16_t* __restrict__ out_split, int64_t out_plane,
    float* __restrict__ out_raw, const int32_t* __restrict__ offsets, const int32_t* __restrict__ pairs,
    const int32_t* __restrict__ units, const int32_t* __restrict__ n_units, int rows, int groups, int k_top,
    float limit, int precision, int row_wgs, int units_per_xcd) {
  moe_gemm_body<kDown, kPl, true>(wptr, bias, act, act_plane, out, out_split, out_plane, out_raw, offsets, pairs,
                                  units, n_units, rows, groups, k_top, limit, precision, row_wgs, units_per_xcd);
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
  const int groups = (int)(hidden / 32);
  // activation planes past 2 GiB take the 64-bit-pointer form
  auto kernel = n_tok * hidden * 2 > 0x7fffffff ? moe_gemm_wide_kernel<false, 1> : moe_gemm_kernel<false, 1>;
  kernel<<<grid, kGemmThreads, gemm_lds_bytes<false, 1>(), stream>>>(
      reinterpret_cast<const uint8_t* const*>(w), static_cast<const uint16_t*>(bias), static_cast<const uint16_t*>(x),
      0, nullptr, static_cast<uint16_t*>(gated_split), n_pairs * inter, gated_raw, offsets, pairs,
      units + units_offset_gemm(n_pairs, n_exp), units + 2, (int)rows, groups, (int)k, limit, precision,
      row_wgs, per_xcd);
  return check_launch("moe_gemm_kernel<gate_up>");
}

int launch_gemm_down(const void* const* w, const void* bias, const void* gated_split, int64_t n_pairs, int64_t n_exp,
                     const int32_t* offsets, const int32_t* pairs, const int32_t* units, int64_t hidden, int64_t inter,
                     int precision, float* eo, hipStream_t stream) {
  const int row_wgs = (int)((hidden + kGemmRows - 1) / kGemmRows);
  const int per_xcd = (int)((units_capacity(n_pairs, n_exp, kUnitTokensGemm) + kXcds - 1) / kXcds);
  const dim3 grid((unsigned)(kXcds * per_xcd * row_wgs));
  const int groups = (int)(inter / 32);
  // bfloat16 precision: the input is the hi plane alone (its lo plane is zero)
  // activation planes past 2 GiB take the 64-bit-pointer form
  const bool wide = n_pairs * inter * 2 > 0x7fffffff;
  auto kernel = precision == KLC_PRECISION_BF16 ? (wide ? moe_gemm_wide_kernel<true, 1> : moe_gemm_kernel<true, 1>)
                                                : (wide ? moe_gemm_wide_kernel<true, 2> : moe_gemm_kernel<true, 2>);
  const int lds = precision == KLC_PRECISION_BF16 ? gemm_lds_bytes<true, 1>() : gemm_lds_bytes<true, 2>();
  kernel<<<grid, kGemmThreads, lds, stream>>>(
      reinterpret_cast<const uint8_t* const*>(w), static_cast<const uint16_t*>(bias),
      static_cast<const uint16_t*>(gated_split), n_pairs * inter, eo, nullptr, 0, nullptr, offsets, pairs,
      units + units_offset_gemm(n_pairs, n_exp), units + 2, (int)hidden, groups, 1, 0.0f, precision,
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
