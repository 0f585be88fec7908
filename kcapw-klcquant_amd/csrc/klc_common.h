// Shared device helpers and host error plumbing for the KLC MoE library (gfx950).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "klc_moe.h"

namespace klc {

// ---- host side -------------------------------------------------------------

// Records a formatted message for klc_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...);
// Converts the last HIP launch error (if any) into a status.
int check_launch(const char* what);
// Packs n_mat checkpoint-layout matrices (blocks [rows][groups][16], scales
// [rows][groups], rows a multiple of 64) into the row-tile layout on `st`:
// the block region of matrix m at out_blocks + m * mat_stride, its scale
// region at out_scales + m * mat_stride.  Defined in klc_mxfp4.hip.
int launch_pack(const uint8_t* blocks, const uint8_t* scales, uint8_t* out_blocks, uint8_t* out_scales, int64_t n_mat,
                int rows, int groups, int64_t mat_stride, hipStream_t st);
// The same for one matrix of `rows` rows (a multiple of 64) whose blocks and
// scales are in pinned host memory (device-accessible addresses): the kernel
// reads them over PCIe, in source order.  Defined in klc_mxfp4.hip.
int launch_pack_from_host(const uint8_t* blocks, const uint8_t* scales, uint8_t* out_blocks, uint8_t* out_scales,
                          int rows, int groups, hipStream_t st);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

#define KLC_REQUIRE(cond, code, ...)                 \
  do {                                               \
    if (!(cond)) return ::klc::set_error((code), __VA_ARGS__); \
  } while (0)

constexpr int kWave = 64;

// The decode router's one-token form: one wave selects the token's experts
// (and, given a host record, writes its tag) with no workgroup barrier.
__host__ __device__ constexpr bool router_decode_one_wave(int64_t n_tok, int64_t n_exp) {
  return n_tok == 1 && n_exp <= 4 * kWave;
}

// Packed ("row-tile") MXFP4 layout used by the expert GEMV kernels.  One
// matrix of `rows` x `groups` MX blocks (rows a multiple of 64) is stored as
//   blocks: [rows / 64][groups][64 rows][16 bytes]
//   scales: [rows / 64][S / 8][64 rows][4 quarters][8 bytes],  S = round_up(ceil(groups / 4), 8)
// so one wave-wide 16-byte load fetches group g of 64 consecutive rows as
// 1 KiB of contiguous memory.  A lane that works on groups q, q + 4, ... of
// one row (step s = group / 4) finds the scale of step s in byte s % 8 of
// the 8-byte word (s / 8, row, q): a wave reading one such word for its 16
// rows x 4 quarters reads 512 contiguous bytes.
constexpr int kTileRows = 64;
__host__ __device__ inline int64_t packed_steps(int64_t groups) { return (groups + 3) / 4; }
__host__ __device__ inline int64_t packed_scale_record(int64_t groups) { return (packed_steps(groups) + 7) / 8 * 8; }
__host__ __device__ inline int64_t packed_block_bytes(int64_t rows, int64_t groups) { return (rows / kTileRows) * groups * 1024; }
__host__ __device__ inline int64_t packed_scale_bytes(int64_t rows, int64_t groups) {
  return (rows / kTileRows) * kTileRows * 4 * packed_scale_record(groups);
}
__host__ __device__ inline int64_t packed_matrix_bytes(int64_t rows, int64_t groups) {
  return packed_block_bytes(rows, groups) + packed_scale_bytes(rows, groups);
}
// Byte offset, from the start of the scales, of the 8-byte scale word
// (pair p of steps, row, quarter q).
__host__ __device__ __forceinline__ int64_t packed_scale_word(int64_t groups, int row, int p, int q) {
  const int64_t tile_bytes = (int64_t)kTileRows * 4 * packed_scale_record(groups);
  return (row / kTileRows) * tile_bytes + (((int64_t)p * kTileRows + row % kTileRows) * 4 + q) * 8;
}
// Byte offset of the scale of (row, group) inside a packed matrix.
__host__ __device__ __forceinline__ int64_t packed_scale_offset(int rows, int groups, int row, int group) {
  const int s = group >> 2;
  return packed_block_bytes(rows, groups) + packed_scale_word(groups, row, s >> 3, group & 3) + (s & 7);
}

// Work units of the expert kernels.  A unit is one pass of one active expert
// over up to kUnitTokens* of its tokens: the decode GEMVs stage 8 (gate_up)
// or 4 (down: hi and lo rows per token) activation rows per pass, the
// prefill grouped GEMM 64 tokens per tile.  An expert with more tokens gets
// several units, which run as separate workgroups.  The dispatch writes all
// three lists into one int32 array:
//   [0] gate_up unit count, [1] down unit count, [2] GEMM unit count, [3] 0,
//   then the gate_up list (capacity cap(8)), the down list (cap(4)) and the
//   GEMM list (cap(64)),
// a unit being expert | (pass << 10) (experts < 1024), experts ascending,
// passes ascending.
constexpr int kUnitTokensGateUp = 8;
constexpr int kUnitTokensDown = 4;
constexpr int kUnitTokensGemm = 64;
constexpr int kUnitHeader = 4;
__host__ __device__ __forceinline__ int32_t make_unit(int expert, int pass) { return expert | (pass << 10); }
__host__ __device__ __forceinline__ int unit_expert(int32_t u) { return u & 1023; }
__host__ __device__ __forceinline__ int unit_pass(int32_t u) { return (int)((uint32_t)u >> 10); }
// Upper bound on the units of n_pairs pairs over n_exp experts at `per`
// tokens per unit: sum_e ceil(c_e / per) <= (n_pairs + (per - 1) * active) / per.
__host__ __device__ inline int64_t units_capacity(int64_t n_pairs, int64_t n_exp, int per) {
  const int64_t active = n_pairs < n_exp ? n_pairs : n_exp;
  return (n_pairs + (per - 1) * active) / per;
}
__host__ __device__ inline int64_t units_offset_down(int64_t n_pairs, int64_t n_exp) {
  return kUnitHeader + units_capacity(n_pairs, n_exp, kUnitTokensGateUp);
}
__host__ __device__ inline int64_t units_offset_gemm(int64_t n_pairs, int64_t n_exp) {
  return units_offset_down(n_pairs, n_exp) + units_capacity(n_pairs, n_exp, kUnitTokensDown);
}
__host__ __device__ inline int64_t units_size(int64_t n_pairs, int64_t n_exp) {
  return units_offset_gemm(n_pairs, n_exp) + units_capacity(n_pairs, n_exp, kUnitTokensGemm);
}

// ---- device side -----------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// float32 -> bfloat16 bits, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16_rne(f)); }

// Exact float32 bit pattern of FP4_VALUES[code] * 2^(e - 127), as
// torch.ldexp produces it in float32: +-inf on overflow, NaN for a zero code
// with e = 255 (0 * inf), float32 subnormals for the smallest scales.
// E2M1 magnitude m = code & 7 is (1 + f/2) * 2^q with q = (m >> 1) - 1 and
// f = m & 1 for m >= 2; m = 1 is 0.5 (q = -1, f = 0).
__device__ __forceinline__ uint32_t mxfp4_f32_bits(uint32_t code, uint32_t e) {
  const uint32_t sign = (code & 8u) << 28;
  const uint32_t m = code & 7u;
  if (e == 255u) return m == 0u ? 0x7fc00000u : (sign | 0x7f800000u);
  if (m == 0u) return sign;
  const int q = (int)(m >> 1) - 1;
  const uint32_t f = (m > 1u) ? (m & 1u) : 0u;
  const int biased = q + (int)e;
  if (biased >= 255) return sign | 0x7f800000u;
  if (biased >= 1) return sign | ((uint32_t)biased << 23) | (f << 22);
  // biased in {-1, 0}: subnormal, value (2 + f) * 2^(biased - 128) = mant * 2^-149
  return sign | ((2u + f) << (biased + 21));
}

// 2^(e - 127) as float32 for an E8M0 byte (e = 255 -> NaN, the "no scale" code).
__device__ __forceinline__ float e8m0_to_f32(uint32_t e) {
  if (e == 0u) return __uint_as_float(0x00400000u);
  if (e == 255u) return __uint_as_float(0x7fc00000u);
  return __uint_as_float(e << 23);
}

// Two E2M1 codes of byte `sel` of `word` as float32 (low nibble first),
// unscaled.  Uses gfx950's v_cvt_scalef32_pk_f32_fp4 with scale 1.0.
template <int kSel>
__device__ __forceinline__ float2 fp4x2_to_f32(uint32_t word) {
  typedef float f2v __attribute__((ext_vector_type(2)));
  f2v v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, 1.0f, kSel);
  return make_float2(v.x, v.y);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// Raw buffer descriptor word 3 for gfx9-family buffer loads (32-bit data, no swizzle).
constexpr int kBufferWord3 = 0x00020000;
// A per-lane buffer offset (VGPR voffset) past every buffer: such raw-buffer
// loads are out of range, return 0 and touch no memory, without a branch.
// Only voffset is ever set to it; the uniform soffset always stays a valid
// in-buffer offset, so the sum cannot wrap (buffers are far below 1 GiB).
constexpr uint32_t kOutOfRange = 0x40000000u;
// Cache policy of a raw buffer load that streams data read once: the
// non-temporal hint (gfx950 cache-policy bit 1).  Streaming reads of expert
// weights reach about 7.1 TB/s with it against about 6.2 TB/s without.
constexpr int kStreamPolicy = 2;
// Cache policy of raw buffer stores and loads that hand data to workgroups
// on other XCDs within one launch (gfx950 cache-policy bit sc1, agent
// scope): stores write through the XCD's L2, loads miss in the caches that
// are not coherent across XCDs.
constexpr int kAgentScope = 16;

// s_waitcnt immediate that waits until at most n vector memory operations
// and no LDS operation are outstanding (gfx9 encoding; export counter free).
constexpr int vmcnt_imm(int n) { return (n & 0xf) | ((n >> 4) << 14) | 0x70; }

// Eight E2M1 codes (one dword, input order) times the scale -> 8 bf16 (MFMA A operand).
__device__ __forceinline__ bf16x8_t decode8(uint32_t word, float scale) {
  const bf16x2_t p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 0);
  const bf16x2_t p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 1);
  const bf16x2_t p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 2);
  const bf16x2_t p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 3);
  return __builtin_shufflevector(__builtin_shufflevector(p0, p1, 0, 1, 2, 3),
                                 __builtin_shufflevector(p2, p3, 0, 1, 2, 3), 0, 1, 2, 3, 4, 5, 6, 7);
}

// E8M0 byte as the float32 scale operand of the scaled E2M1 conversions:
// 2^(e-127) (e = 0: the float32 subnormal 2^-127), or 0 for a lane that has
// no group (E2M1 values times 0 are +-0).
__device__ __forceinline__ float cvt_scale_operand(uint32_t e, bool live) {
  const uint32_t bits = e == 0u ? 0x00400000u : (e << 23);
  return __uint_as_float(live ? bits : 0u);
}

}  // namespace klc
