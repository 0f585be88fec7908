// MXFP4 -> dense dequant and checkpoint -> row-tile repack (gfx950).
//
// Dequant is HBM bound (1 byte of codes + 1/32 byte of scale in, 2 bytes out
// per value for bfloat16), so the kernel is built around coalesced traffic:
// a workgroup owns a strip of 64 output columns (64 checkpoint rows, i.e. a
// contiguous 64 x groups x 16-byte region) and walks the input dimension in
// chunks of 16 groups.  Packed bytes are staged in LDS, then every thread
// decodes a 4 (input rows) x 8 (output columns) block and writes four 16-byte
// rows, so each wave-wide store covers full 128-byte lines of the transposed
// [in, out] output.  The stores carry the non-temporal hint (the output is
// written once and not read back by this kernel): 555 -> 536-548 us for 128
// 2880 x 2880 matrices to bfloat16.  Values come from gfx950's scaled E2M1 conversions
// (v_cvt_scalef32_pk_{bf16,f16,f32}_fp4), exact for every scale byte below
// 255; the MX NaN scale 255 takes an integer path (mxfp4_f32_bits) that
// reproduces the reference's +-inf / NaN.
#include <algorithm>
#include <type_traits>

#include "klc_common.h"

namespace klc {
namespace {

constexpr int kDqThreads = 256;
constexpr int kDqCols = 64;      // output columns (= checkpoint rows) per workgroup
constexpr int kDqGroups = 16;    // MX groups (32 inputs each) per iteration
constexpr int kLdsStride = kDqGroups * 4 + 1;  // dwords per staged row: data + 1 pad (bank spread)
constexpr int kSclStride = kDqGroups + 1;      // dwords per staged scale row

// Converts one exact float32 bit pattern to the output dtype's bits.
template <int kDtype>
__device__ __forceinline__ uint32_t to_out_bits(uint32_t f32bits) {
  if constexpr (kDtype == KLC_DTYPE_BF16) {
    return f32bits >> 16;  // every finite MXFP4 value is exact in bfloat16
  } else if constexpr (kDtype == KLC_DTYPE_F16) {
    return (uint32_t)__half_as_ushort(__float2half_rn(__uint_as_float(f32bits)));
  } else {
    return f32bits;
  }
}

// Workgroup barrier that orders LDS accesses only: __syncthreads' release
// fence would also wait for every outstanding global store.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Byte `h` of `v16` (two E2M1 codes, low nibble first) times `scale`, as two
// 16-bit values packed low-first (bfloat16 or float16 per kDtype).
template <int kDtype>
__device__ __forceinline__ uint32_t cvt_pair(uint32_t v16, float scale, int h) {
  if constexpr (kDtype == KLC_DTYPE_F16) {
    const f16x2_t v = h ? __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v16, scale, 1)
                        : __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v16, scale, 0);
    return __builtin_bit_cast(uint32_t, v);
  } else {
    const bf16x2_t v = h ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v16, scale, 1)
                         : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v16, scale, 0);
    return __builtin_bit_cast(uint32_t, v);
  }
}

__device__ __forceinline__ f32x2_t cvt_pair_f32(uint32_t v16, float scale, int h) {
  return h ? __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(v16, scale, 1)
           : __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(v16, scale, 0);
}

template <int kDtype, bool kPacked>
__global__ __launch_bounds__(kDqThreads) void dequant_kernel(const uint8_t* __restrict__ blocks,
                                                             const uint8_t* __restrict__ scales,
                                                             void* __restrict__ out, int rows, int groups,
                                                             int64_t packed_stride) {
  __shared__ uint32_t s_blk[kDqCols * kLdsStride];
  __shared__ uint32_t s_scl[kDqCols * kSclStride];

  const int strips = (rows + kDqCols - 1) / kDqCols;
  const int m = blockIdx.x / strips;
  const int col0 = (blockIdx.x - m * strips) * kDqCols;
  const int tid = threadIdx.x;
  const int in_dim = groups * 32;

  // load mapping: 16-byte chunks (row, 4 * i + gi), i = 0..3, per thread
  const int l_row = tid >> 2;
  const int l_gi = tid & 3;
  // compute mapping: 4 input rows x 8 output columns per thread and sub-chunk
  const int c_oc = tid & 7;
  const int c_iq = tid >> 3;          // 0..31 quads of input rows in a 4-group sub-chunk
  const int c_gi = c_iq >> 3;         // group within the sub-chunk
  const int c_q4 = c_iq & 7;          // quad within the group
  const int col = col0 + c_oc * 8;

  const uint8_t* mat = blocks;
  if constexpr (kPacked) mat = blocks + (int64_t)m * packed_stride;

  // ---- one iteration = 16 groups: loads into registers, staged in LDS,
  // decoded 4 groups at a time and stored as 16-byte rows of [in, out] ----
  const int r_ld = col0 + l_row;
  uint4 v[4];
  uint32_t e[4];
  // kClamp: every load reads a valid chunk (groups past the end re-read the
  // last one; their values are never stored), so no branch guards a load
  auto load_chunks = [&](int g0, auto clamp) {
    constexpr bool kClamp = decltype(clamp)::value;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int g = g0 + 4 * i + l_gi;
      if constexpr (kClamp) g = min(g, groups - 1);
      v[i] = make_uint4(0u, 0u, 0u, 0u);
      e[i] = 127u;
      if (kClamp || (r_ld < rows && g < groups)) {
        if constexpr (kPacked) {
          const uint8_t* src = mat + ((int64_t)(r_ld / kTileRows) * groups + g) * 1024 + (r_ld % kTileRows) * 16;
          v[i] = *reinterpret_cast<const uint4*>(src);
          e[i] = mat[packed_scale_offset(rows, groups, r_ld, g)];
        } else {
          const int64_t chunk = ((int64_t)m * rows + r_ld) * groups + g;
          v[i] = *reinterpret_cast<const uint4*>(blocks + chunk * 16);
          e[i] = scales[chunk];
        }
      }
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t* dst = s_blk + l_row * kLdsStride + (4 * i + l_gi) * 4;
      dst[0] = v[i].x;
      dst[1] = v[i].y;
      dst[2] = v[i].z;
      dst[3] = v[i].w;
      s_scl[l_row * kSclStride + 4 * i + l_gi] = e[i];
    }
  };
  // 4 groups (sub-chunk sc) of the staged iteration: 4 input rows x 8 output
  // columns per thread.  kFull: the strip's 64 columns and the 4 groups all
  // exist and rows % 8 == 0, so every store is one unconditional 16-byte row.
  auto compute = [&](int g0, int sc, auto full) {
    constexpr bool kFull = decltype(full)::value;
    const int gl = 4 * sc + c_gi;  // group within the iteration
    uint32_t bits[4][8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int lr = c_oc * 8 + j;
      const uint32_t word = s_blk[lr * kLdsStride + gl * 4 + (c_q4 >> 1)];
      const uint32_t v16 = (word >> ((c_q4 & 1) * 16)) & 0xffffu;
      const uint32_t ee = s_scl[lr * kSclStride + gl];
      // hardware E2M1 x 2^(e-127) conversion, exact for e < 255 (e = 0: the
      // float32 subnormal 2^-127 as scale).  E8M0 255 (the MX NaN scale):
      // the reference's fp32 ldexp gives +-inf, and NaN for the zero codes;
      // that value is selected, not branched to, so the loop body has no
      // branch (a branch made the compiler wait for every store at the
      // next iteration's loads).
      const bool nan_scale = ee == 255u;
      const float scale = __uint_as_float(ee == 0u ? 0x00400000u : (ee << 23));
#pragma unroll
      for (int h = 0; h < 2; ++h) {  // rows 2h and 2h + 1
        if constexpr (kDtype == KLC_DTYPE_F32) {
          const f32x2_t cv = cvt_pair_f32(v16, scale, h);
          bits[2 * h][j] = __float_as_uint(cv.x);
          bits[2 * h + 1][j] = __float_as_uint(cv.y);
        } else {
          const uint32_t pair = cvt_pair<kDtype>(v16, scale, h);
          bits[2 * h][j] = pair & 0xffffu;
          bits[2 * h + 1][j] = pair >> 16;
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t nan_bits = to_out_bits<kDtype>(mxfp4_f32_bits((v16 >> (4 * r)) & 0xfu, 255u));
        bits[r][j] = nan_scale ? nan_bits : bits[r][j];
      }
    }
    const int i0 = (g0 + gl) * 32 + c_q4 * 4;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t row_off = ((int64_t)m * in_dim + i0 + r) * rows;
      if constexpr (kDtype == KLC_DTYPE_F32) {
        float* o = static_cast<float*>(out) + row_off + col;
        if (kFull || (col + 8 <= rows && (rows & 3) == 0)) {
          __builtin_nontemporal_store(u32x4_t{bits[r][0], bits[r][1], bits[r][2], bits[r][3]},
                                      reinterpret_cast<u32x4_t*>(o));
          __builtin_nontemporal_store(u32x4_t{bits[r][4], bits[r][5], bits[r][6], bits[r][7]},
                                      reinterpret_cast<u32x4_t*>(o) + 1);
        } else {
          for (int j = 0; j < 8; ++j)
            if (col + j < rows) o[j] = __uint_as_float(bits[r][j]);
        }
      } else {
        uint16_t* o = static_cast<uint16_t*>(out) + row_off + col;
        if (kFull || (col + 8 <= rows && (rows & 7) == 0)) {
          __builtin_nontemporal_store(u32x4_t{bits[r][0] | (bits[r][1] << 16), bits[r][2] | (bits[r][3] << 16),
                                              bits[r][4] | (bits[r][5] << 16), bits[r][6] | (bits[r][7] << 16)},
                                      reinterpret_cast<u32x4_t*>(o));
        } else {
          for (int j = 0; j < 8; ++j)
            if (col + j < rows) o[j] = (uint16_t)bits[r][j];
        }
      }
    }
  };

  int g0 = 0;
  if (col0 + kDqCols <= rows && (rows & 7) == 0 && groups >= kDqGroups) {
    // Full iterations of a full strip, in straight-line code: the next
    // iteration's loads are issued before this iteration's stores.  Loads and
    // stores share one completion counter and retire in order, so waiting
    // for those loads leaves the stores in flight; the LDS-only barriers do
    // not wait for them either.
    // The first iteration is peeled, so the loop is entered, like its back
    // edge, with one iteration's loads and then its stores outstanding (a
    // loop entered with only loads outstanding gets one wait for all).
    const int full = groups / kDqGroups * kDqGroups;
    auto iteration = [&](int g) {
      stage();
      lds_barrier();
      load_chunks(g + kDqGroups < groups ? g + kDqGroups : g, std::true_type{});
#pragma unroll
      for (int sc = 0; sc < kDqGroups / 4; ++sc) compute(g, sc, std::true_type{});
    };
    load_chunks(0, std::true_type{});
    iteration(0);
    for (g0 = kDqGroups; g0 < full; g0 += kDqGroups) {
      lds_barrier();  // every thread is done reading the staged chunks
      iteration(g0);
    }
    if (g0 < groups) {  // the tail iteration's chunks are already loaded
      lds_barrier();
      stage();
      lds_barrier();
#pragma unroll 1
      for (int sc = 0; sc < kDqGroups / 4; ++sc) {
        if (g0 + 4 * sc + c_gi >= groups) break;  // uniform per 8-lane group; no barrier inside
        compute(g0, sc, std::false_type{});
      }
    }
    return;
  }
  // Partial strips: one iteration at a time.
  for (; g0 < groups; g0 += kDqGroups) {
    load_chunks(g0, std::false_type{});
    stage();
    __syncthreads();
#pragma unroll 1
    for (int sc = 0; sc < kDqGroups / 4; ++sc) {
      if (g0 + 4 * sc + c_gi >= groups) break;  // uniform per 8-lane group; no barrier inside
      compute(g0, sc, std::false_type{});
    }
    __syncthreads();
  }
}

// Checkpoint layout -> bfloat16 [in, out] in long output runs: workgroup
// (matrix, column block, group quad) stages 4 groups' code chunks (a 64-byte
// run of each checkpoint row) and scale bytes of up to kDqrCols checkpoint
// rows (= output columns) in LDS, word-major (word w of row r at
// sw[w * kDqrCols + r]), and writes output rows 128 q .. 128 q + 127 at its
// columns: runs of 2 * ncols bytes.  The two quads that share a 128-byte
// line of each row run side by side on one XCD (workgroups go to the XCDs
// round-robin), so that line is fetched once.  A task is 8 output rows (a
// band: one word of one group's chunks) x 8 output columns; the threads take
// consecutive tasks, so a task's 8 16-byte stores are, across the workgroup,
// runs of consecutive 16-byte pieces of output rows.  The scaled conversion
// (exact for every scale byte below 255) gives pairs of input elements of one
// row; v_perm_b32 pairs them up as pairs of columns.  Scale byte 255 (the MX
// NaN scale) is rare: those tasks are written again with the exact integer
// path (mxfp4_f32_bits) after the main loop, by the thread that wrote them
// (program order), so the main loop has no branch for it.
//
// Measured (128 x 2880 x 2880 to bfloat16): 768 columns and 512 threads
// (52 KB of LDS, 3 workgroups per CU) 511-518 us against 535-551 us for the
// 64-column strips above; 1536 columns (one workgroup per CU) 551-558 us; one
// group per workgroup (16-byte reads at the row stride) 1,010 us; several
// items per workgroup with the next one's loads in flight, or buffer stores,
// were slower.
constexpr int kDqrThreads = 512;
constexpr int kDqrGroups = 4;                                    // groups per workgroup
constexpr int kDqrCols = 768;                                    // checkpoint rows per column block
constexpr int kDqrRounds = kDqrCols * kDqrGroups / kDqrThreads;  // 16-byte loads per thread
static_assert(kDqrCols * kDqrGroups % kDqrThreads == 0, "whole load rounds");

__host__ __device__ constexpr int dqr_col_blocks(int rows) { return (rows + kDqrCols - 1) / kDqrCols; }
// Column block cb of nb over rows (a multiple of 64): nearly equal widths, multiples of 64 columns
__host__ __device__ inline int dqr_col0(int rows, int nb, int cb) { return (int)((int64_t)rows / 64 * cb / nb) * 64; }

__global__ __launch_bounds__(kDqrThreads) void dequant_rows_bf16_kernel(const uint8_t* __restrict__ blocks,
                                                                        const uint8_t* __restrict__ scales,
                                                                        uint16_t* __restrict__ out, int n_mat,
                                                                        int rows, int groups) {
  extern __shared__ __align__(16) uint32_t lds_words[];  // [16][kDqrCols] code words, then scale bytes
  // workgroup -> (pair of quads P, half h): P's two workgroups are 8 apart in a window of 16
  const int nb = dqr_col_blocks(rows);
  const int quads = (groups + kDqrGroups - 1) / kDqrGroups;
  const int pairs = (quads + 1) / 2;
  const int b = blockIdx.x;
  const int pair = (b >> 4) * 8 + (b & 7);
  const int quad = 2 * (pair % pairs) + ((b >> 3) & 1);
  const int mcb = pair / pairs;  // (matrix, column block)
  if (quad >= quads || mcb >= n_mat * nb) return;
  const int m = mcb / nb;
  const int cb = mcb - m * nb;
  const int col0 = dqr_col0(rows, nb, cb);
  const int ncols = dqr_col0(rows, nb, cb + 1) - col0;
  const int g0 = quad * kDqrGroups;
  const int ng = min(kDqrGroups, groups - g0);
  uint32_t* sw = lds_words;
  uint8_t* ss = reinterpret_cast<uint8_t*>(lds_words + 4 * kDqrGroups * kDqrCols);
  const int tid = threadIdx.x;
  const int64_t first = (int64_t)m * rows * groups + (int64_t)col0 * groups + g0;  // chunk (col0, g0)
  const int span = (ncols - 1) * groups + ng;                                     // chunks to the last one
  const __amdgpu_buffer_rsrc_t cbuf =
      __builtin_amdgcn_make_buffer_rsrc((void*)(blocks + first * 16), (short)0, span * 16, kBufferWord3);
  const __amdgpu_buffer_rsrc_t sbuf =
      __builtin_amdgcn_make_buffer_rsrc((void*)(scales + first), (short)0, span, kBufferWord3);
  // load i: row r = (tid + i * threads) / 4, chunk c = tid % 4; rows and groups past the end read out of
  // range (zeros, no traffic).  Every load first, then the LDS writes.
  const int c = tid & 3;
  u32x4_t v[kDqrRounds];
  uint32_t e[kDqrRounds];
#pragma unroll
  for (int i = 0; i < kDqrRounds; ++i) {
    const int r = (tid >> 2) + i * (kDqrThreads / 4);
    const bool live = r < ncols && c < ng;
    const uint32_t chunk = (uint32_t)r * (uint32_t)groups + (uint32_t)c;
    v[i] = __builtin_amdgcn_raw_buffer_load_b128(cbuf, live ? chunk * 16u : kOutOfRange, 0, 0);
    e[i] = __builtin_amdgcn_raw_buffer_load_b8(sbuf, live ? chunk : kOutOfRange, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < kDqrRounds; ++i) {
    const int r = (tid >> 2) + i * (kDqrThreads / 4);
    if (r < ncols) {
#pragma unroll
      for (int w = 0; w < 4; ++w) sw[(4 * c + w) * kDqrCols + r] = v[i][w];
      ss[c * kDqrCols + r] = (uint8_t)e[i];
    }
  }
  __syncthreads();

  const int cpr = ncols >> 3;  // 16-byte pieces (8 columns) per output run
  const int ntask = 4 * ng * cpr;
  uint16_t* obase = out + ((int64_t)m * groups + g0) * 32 * rows + col0;
  bool nan_scale = false;
  for (int t = tid; t < ntask; t += kDqrThreads) {
    const int band = t / cpr;  // group band / 4, word band % 4
    const int oc = t - band * cpr;
    const uint32_t* wrow = sw + band * kDqrCols + oc * 8;
    const u32x4_t wa = *reinterpret_cast<const u32x4_t*>(wrow);
    const u32x4_t wb = *reinterpret_cast<const u32x4_t*>(wrow + 4);
    const uint2 sc8 = *reinterpret_cast<const uint2*>(ss + (band >> 2) * kDqrCols + oc * 8);
    const uint32_t word[8] = {wa[0], wa[1], wa[2], wa[3], wb[0], wb[1], wb[2], wb[3]};
    // pr[j][q]: elements 2q, 2q + 1 of the band for column j (checkpoint row col0 + 8 oc + j)
    uint32_t pr[8][4];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t eb = ((j < 4 ? sc8.x : sc8.y) >> (8 * (j & 3))) & 0xffu;
      nan_scale |= eb == 255u;
      const float scale = __uint_as_float(eb == 0u ? 0x00400000u : (eb << 23));
      pr[j][0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word[j], scale, 0));
      pr[j][1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word[j], scale, 1));
      pr[j][2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word[j], scale, 2));
      pr[j][3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word[j], scale, 3));
    }
    uint16_t* o = obase + (int64_t)(8 * band) * rows + oc * 8;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        // output row 8 band + 2 q + h: half h of every column's pair q, columns paired low-first
        const uint32_t sel = h ? 0x07060302u : 0x05040100u;
        const u32x4_t row = {__builtin_amdgcn_perm(pr[1][q], pr[0][q], sel), __builtin_amdgcn_perm(pr[3][q], pr[2][q], sel),
                             __builtin_amdgcn_perm(pr[5][q], pr[4][q], sel), __builtin_amdgcn_perm(pr[7][q], pr[6][q], sel)};
        __builtin_nontemporal_store(row, reinterpret_cast<u32x4_t*>(o + (int64_t)(2 * q + h) * rows));
      }
    }
  }
  if (!__syncthreads_or(nan_scale)) return;
  // tasks with a scale byte 255, again with the integer path, by the same threads (same addresses,
  // program order: these stores land after the first ones)
  for (int t = tid; t < ntask; t += kDqrThreads) {
    const int band = t / cpr;
    const int oc = t - band * cpr;
    const uint8_t* sc = ss + (band >> 2) * kDqrCols + oc * 8;
    bool any = false;
    for (int j = 0; j < 8; ++j) any |= sc[j] == 255u;
    if (!any) continue;
    uint16_t* o = obase + (int64_t)(8 * band) * rows + oc * 8;
    for (int i = 0; i < 8; ++i) {
      for (int j = 0; j < 8; ++j) {
        const uint32_t code = (sw[band * kDqrCols + oc * 8 + j] >> (4 * i)) & 0xfu;
        o[(int64_t)i * rows + j] = (uint16_t)(mxfp4_f32_bits(code, sc[j]) >> 16);
      }
    }
  }
}

// Checkpoint layout -> row-tile layout: one thread per (matrix, tile, group,
// row in tile) 16-byte chunk, writes coalesced; runs once per load.  The
// block and scale regions of matrix m start at out_blocks / out_scales +
// m * mat_stride, so a run of whole tiles can be packed into the middle of a
// larger matrix.
__global__ __launch_bounds__(256) void pack_blocks_kernel(const uint8_t* __restrict__ blocks,
                                                          uint8_t* __restrict__ out_blocks, int64_t n_mat, int rows,
                                                          int groups, int64_t mat_stride) {
  const int tiles = rows / kTileRows;
  const int64_t total = n_mat * tiles * groups * kTileRows;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int rr = (int)(idx % kTileRows);
    int64_t rest = idx / kTileRows;
    const int g = (int)(rest % groups);
    rest /= groups;
    const int tile = (int)(rest % tiles);
    const int64_t m = rest / tiles;
    const int r = tile * kTileRows + rr;
    const uint4 v = *reinterpret_cast<const uint4*>(blocks + ((m * rows + r) * groups + g) * 16);
    *reinterpret_cast<uint4*>(out_blocks + m * mat_stride + ((int64_t)tile * groups + g) * 1024 + rr * 16) = v;
  }
}

// Scale records: one thread per (matrix, row, quarter, step) byte, padding zero.
__global__ __launch_bounds__(256) void pack_scales_kernel(const uint8_t* __restrict__ scales,
                                                          uint8_t* __restrict__ out_scales, int64_t n_mat, int rows,
                                                          int groups, int64_t mat_stride) {
  // one thread per packed scale byte, in packed order: (matrix, tile, pair,
  // row in tile, quarter, byte); padding bytes (steps past the last group) are 0
  const int rec = (int)packed_scale_record(groups);
  const int64_t total = n_mat * rows * 4 * rec;
  const int64_t per_mat = (int64_t)rows * 4 * rec;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = idx / per_mat;
    int64_t rest = idx - m * per_mat;
    const int b = (int)(rest & 7);
    rest >>= 3;
    const int q = (int)(rest & 3);
    rest >>= 2;
    const int rr = (int)(rest % kTileRows);
    rest /= kTileRows;
    const int p = (int)(rest % (rec / 8));
    const int tile = (int)(rest / (rec / 8));
    const int r = tile * kTileRows + rr;
    const int g = 4 * (8 * p + b) + q;
    const uint8_t e = g < groups ? scales[(m * rows + r) * groups + g] : (uint8_t)0;
    out_scales[m * mat_stride + packed_scale_word(groups, r, p, q) + b] = e;
  }
}

// Packs one run of whole tiles read straight from pinned host memory (the
// GPU reads it over PCIe, so every read is 16 bytes per lane in source order:
// a wavefront reads 1 KiB of contiguous host memory).  Three grid-stride
// passes: block chunks (four loads in flight per thread before the four
// scattered 16-byte stores), scale bytes read 16 at a time and scattered
// (a row's 32 consecutive groups land in 32 contiguous bytes), and the zero
// bytes that pad each row's scale record.  rows * groups < 2^30.
__global__ __launch_bounds__(256) void pack_host_kernel(const uint8_t* __restrict__ blocks,
                                                        const uint8_t* __restrict__ scales,
                                                        uint8_t* __restrict__ out_blocks,
                                                        uint8_t* __restrict__ out_scales, int rows, int groups) {
  const int n = rows * groups;  // block chunks = scale bytes
  const int stride = (int)(gridDim.x * blockDim.x);
  const int tid = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  const uint4* src = reinterpret_cast<const uint4*>(blocks);
  uint4* dst = reinterpret_cast<uint4*>(out_blocks);
  for (int base = tid; base < n; base += 4 * stride) {
    uint4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (base + k * stride < n) v[k] = src[base + k * stride];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int i = base + k * stride;
      if (i < n) {
        const int r = i / groups, g = i - r * groups;
        dst[((r / kTileRows) * groups + g) * kTileRows + (r % kTileRows)] = v[k];
      }
    }
  }
  const uint4* ssrc = reinterpret_cast<const uint4*>(scales);
  for (int j = tid; j < n / 16; j += stride) {
    const uint4 v = ssrc[j];
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    int r = (16 * j) / groups, g = 16 * j - r * groups;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int step = g >> 2;
      out_scales[packed_scale_word(groups, r, step >> 3, g & 3) + (step & 7)] = (uint8_t)(w[k >> 2] >> (8 * (k & 3)));
      if (++g == groups) {
        g = 0;
        ++r;
      }
    }
  }
  const int pad = 4 * (int)packed_scale_record(groups) - groups;
  for (int k = tid; k < rows * pad; k += stride) {
    const int r = k / pad, g = groups + (k - r * pad);
    const int step = g >> 2;
    out_scales[packed_scale_word(groups, r, step >> 3, g & 3) + (step & 7)] = 0;
  }
}

}  // namespace

int launch_pack_from_host(const uint8_t* blocks, const uint8_t* scales, uint8_t* out_blocks, uint8_t* out_scales,
                          int rows, int groups, hipStream_t st) {
  if (rows == 0) return KLC_OK;
  KLC_REQUIRE(rows % kTileRows == 0 && (int64_t)rows * groups < (int64_t)1 << 30 &&
                  (int64_t)rows * 4 * packed_scale_record(groups) < (int64_t)1 << 31,
              KLC_ERR_UNSUPPORTED, "pack_host_kernel: %d rows x %d groups in one run", rows, groups);
  // PCIe reads: a few hundred wavefronts with four 1 KiB reads each keep
  // enough bytes in flight; more workgroups only add contention (a plain
  // host-to-device copy kernel measured 51.7 GB/s at 64 workgroups, 40 at 512)
  const int64_t want = ((int64_t)rows * groups + 1023) / 1024;
  pack_host_kernel<<<(unsigned)std::min<int64_t>(128, std::max<int64_t>(1, want)), 256, 0, st>>>(
      blocks, scales, out_blocks, out_scales, rows, groups);
  return check_launch("pack_host_kernel");
}

int launch_pack(const uint8_t* blocks, const uint8_t* scales, uint8_t* out_blocks, uint8_t* out_scales, int64_t n_mat,
                int rows, int groups, int64_t mat_stride, hipStream_t st) {
  if (n_mat == 0 || rows == 0) return KLC_OK;
  const int64_t chunks = n_mat * rows * groups;
  const unsigned grid_b = (unsigned)((chunks + 255) / 256 < 65536 ? (chunks + 255) / 256 : 65536);
  pack_blocks_kernel<<<grid_b, 256, 0, st>>>(blocks, out_blocks, n_mat, rows, groups, mat_stride);
  const int rc = check_launch("pack_blocks_kernel");
  if (rc) return rc;
  const int64_t bytes = n_mat * rows * 4 * packed_scale_record(groups);
  const unsigned grid_s = (unsigned)((bytes + 255) / 256 < 65536 ? (bytes + 255) / 256 : 65536);
  pack_scales_kernel<<<grid_s, 256, 0, st>>>(scales, out_scales, n_mat, rows, groups, mat_stride);
  return check_launch("pack_scales_kernel");
}

namespace {

template <bool kPacked>
int launch_dequant(const void* blocks, const void* scales, void* out, int64_t n_mat, int64_t rows, int64_t groups,
                   int dtype, int64_t packed_stride, hipStream_t stream) {
  if constexpr (!kPacked) {
    // checkpoint layout to bfloat16, rows a multiple of 64: long output runs per workgroup (a
    // matrix's codes below kOutOfRange bytes, so the out-of-range loads stay out of range)
    if (dtype == KLC_DTYPE_BF16 && rows % 64 == 0 && rows * groups * 16 < (int64_t)kOutOfRange) {
      const int64_t pairs = n_mat * dqr_col_blocks((int)rows) * (((groups + kDqrGroups - 1) / kDqrGroups + 1) / 2);
      const int64_t grid = (pairs + 7) / 8 * 16;
      if (grid <= 0x7fffffff) {
        const size_t lds = (size_t)kDqrCols * kDqrGroups * 17;
        dequant_rows_bf16_kernel<<<(unsigned)grid, kDqrThreads, lds, stream>>>(
            static_cast<const uint8_t*>(blocks), static_cast<const uint8_t*>(scales), static_cast<uint16_t*>(out),
            (int)n_mat, (int)rows, (int)groups);
        return check_launch("dequant_rows_bf16_kernel");
      }
    }
  }
  const int64_t strips = (rows + kDqCols - 1) / kDqCols;
  const int64_t grid = n_mat * strips;
  KLC_REQUIRE(grid <= 0x7fffffff, KLC_ERR_UNSUPPORTED, "dequant: too many matrices (%lld)", (long long)n_mat);
  const auto* b = static_cast<const uint8_t*>(blocks);
  const auto* s = static_cast<const uint8_t*>(scales);
  switch (dtype) {
    case KLC_DTYPE_BF16:
      dequant_kernel<KLC_DTYPE_BF16, kPacked><<<(unsigned)grid, kDqThreads, 0, stream>>>(b, s, out, (int)rows, (int)groups, packed_stride);
      break;
    case KLC_DTYPE_F16:
      dequant_kernel<KLC_DTYPE_F16, kPacked><<<(unsigned)grid, kDqThreads, 0, stream>>>(b, s, out, (int)rows, (int)groups, packed_stride);
      break;
    case KLC_DTYPE_F32:
      dequant_kernel<KLC_DTYPE_F32, kPacked><<<(unsigned)grid, kDqThreads, 0, stream>>>(b, s, out, (int)rows, (int)groups, packed_stride);
      break;
    default:
      return set_error(KLC_ERR_ARGUMENT, "dequant: unknown dtype %d", dtype);
  }
  return check_launch("dequant_kernel");
}

}  // namespace
}  // namespace klc

using namespace klc;

extern "C" int klc_mxfp4_dequant(const void* blocks, const void* scales, void* out, int64_t n_mat, int64_t out_dim,
                                 int64_t groups, int out_dtype, void* stream) {
  KLC_REQUIRE(blocks && scales && out, KLC_ERR_ARGUMENT, "klc_mxfp4_dequant: null pointer");
  KLC_REQUIRE(n_mat >= 0 && out_dim > 0 && groups > 0, KLC_ERR_ARGUMENT,
              "klc_mxfp4_dequant: bad sizes n_mat=%lld out_dim=%lld groups=%lld", (long long)n_mat,
              (long long)out_dim, (long long)groups);
  KLC_REQUIRE(out_dim < (1 << 30) && groups < (1 << 24), KLC_ERR_UNSUPPORTED, "klc_mxfp4_dequant: matrix too large");
  if (n_mat == 0) return KLC_OK;
  return launch_dequant<false>(blocks, scales, out, n_mat, out_dim, groups, out_dtype, 0, as_stream(stream));
}

extern "C" int64_t klc_mxfp4_packed_bytes(int64_t out_dim, int64_t groups) {
  if (out_dim <= 0 || groups <= 0)
    return set_error(KLC_ERR_ARGUMENT, "klc_mxfp4_packed_bytes: bad sizes out_dim=%lld groups=%lld",
                     (long long)out_dim, (long long)groups);
  if (out_dim % kTileRows)
    return set_error(KLC_ERR_SHAPE, "klc_mxfp4_packed_bytes: out_dim=%lld is not a multiple of %d",
                     (long long)out_dim, kTileRows);
  return packed_matrix_bytes(out_dim, groups);
}

extern "C" int klc_mxfp4_pack(const void* blocks, const void* scales, void* packed, int64_t n_mat, int64_t out_dim,
                              int64_t groups, void* stream) {
  KLC_REQUIRE(blocks && scales && packed, KLC_ERR_ARGUMENT, "klc_mxfp4_pack: null pointer");
  const int64_t stride = klc_mxfp4_packed_bytes(out_dim, groups);
  if (stride < 0) return (int)stride;
  KLC_REQUIRE(n_mat >= 0, KLC_ERR_ARGUMENT, "klc_mxfp4_pack: n_mat=%lld", (long long)n_mat);
  KLC_REQUIRE(out_dim < (1 << 30) && groups < (1 << 24), KLC_ERR_UNSUPPORTED, "klc_mxfp4_pack: matrix too large");
  uint8_t* out = static_cast<uint8_t*>(packed);
  return launch_pack(static_cast<const uint8_t*>(blocks), static_cast<const uint8_t*>(scales), out,
                     out + packed_block_bytes(out_dim, groups), n_mat, (int)out_dim, (int)groups, stride,
                     as_stream(stream));
}

extern "C" int klc_mxfp4_dequant_packed(const void* packed, void* out, int64_t n_mat, int64_t out_dim,
                                        int64_t groups, int out_dtype, void* stream) {
  KLC_REQUIRE(packed && out, KLC_ERR_ARGUMENT, "klc_mxfp4_dequant_packed: null pointer");
  const int64_t stride = klc_mxfp4_packed_bytes(out_dim, groups);
  if (stride < 0) return (int)stride;
  KLC_REQUIRE(n_mat >= 0, KLC_ERR_ARGUMENT, "klc_mxfp4_dequant_packed: n_mat=%lld", (long long)n_mat);
  KLC_REQUIRE(out_dim < (1 << 30) && groups < (1 << 24), KLC_ERR_UNSUPPORTED,
              "klc_mxfp4_dequant_packed: matrix too large");
  if (n_mat == 0) return KLC_OK;
  return launch_dequant<true>(packed, packed, out, n_mat, out_dim, groups, out_dtype, stride, as_stream(stream));
}
