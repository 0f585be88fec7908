// Measurement library for the tests (not part of libklcmoe.so): the CDNA4
// scaled MFMA v_mfma_scale_f32_16x16x128_f8f6f4 with MXFP4 weights (A) and
// FP8 E4M3 activations (B), each 32-element block with its own E8M0 scale.
// It runs the operation the grouped GEMM would run if it took the weights in
// their own format, so a test can measure its sums against exact ones.
//
// Operand layout (dense 16x16x128, FP4 A and FP8 B, established on the GPU with
// one-hot operands): lane l holds row (A) or column (B) l % 16.  A: the 16
// bytes in the first four VGPRs hold k = 32 (l / 16) .. 32 (l / 16) + 31, low
// nibble first.  B: bytes 0..15 hold k = 16 (l / 16) .. 16 (l / 16) + 15 and
// bytes 16..31 hold k = 64 + 16 (l / 16) .. 64 + 16 (l / 16) + 15.  Scales: byte
// 0 of lane l's scale operand is the E8M0 scale of row / column l % 16 for
// k-block l / 16 (k = 32 (l / 16) .. 32 (l / 16) + 31), for A and B alike.  The
// result lane l holds column l % 16, rows 4 (l / 16) .. 4 (l / 16) + 3.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef int32_t i32x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

namespace {

// out[n][m] = sum over steps s < n_steps and planes p < n_planes of
// A_s (rows, MXFP4) times B_s,p (tokens, FP8 E4M3), accumulated by the MFMA
// itself (C operand) step by step, plane by plane.  Workgroup (x, y) computes
// rows 16 x .. 16 x + 15 of tokens 16 y .. 16 y + 15.
//   a_codes  [row tile][s][16 rows][64 bytes]      a_scales [row tile][s][16 rows][4]
//   b_codes  [token tile][s][p][16 tokens][128]    b_scales [token tile][s][p][16 tokens][4]
//   out      [tokens][n_rows] float32
__global__ __launch_bounds__(64) void fp4_fp8_gemm_kernel(const uint8_t* __restrict__ a_codes,
                                                          const uint8_t* __restrict__ a_scales,
                                                          const uint8_t* __restrict__ b_codes,
                                                          const uint8_t* __restrict__ b_scales, int n_steps,
                                                          int n_planes, int n_rows, float* __restrict__ out) {
  const int rt = blockIdx.x, ct = blockIdx.y;
  const int lane = threadIdx.x;
  const int r = lane & 15, kb = lane >> 4;
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int s = 0; s < n_steps; ++s) {
    const int64_t ts = (int64_t)rt * n_steps + s;
    const uint32_t* ap = reinterpret_cast<const uint32_t*>(a_codes + (ts * 16 + r) * 64 + kb * 16);
    const i32x8_t a = {(int32_t)ap[0], (int32_t)ap[1], (int32_t)ap[2], (int32_t)ap[3], 0, 0, 0, 0};
    const int sa = a_scales[(ts * 16 + r) * 4 + kb];
    for (int p = 0; p < n_planes; ++p) {
      const int64_t tsp = ((int64_t)ct * n_steps + s) * n_planes + p;
      const uint32_t* bp = reinterpret_cast<const uint32_t*>(b_codes + (tsp * 16 + r) * 128 + kb * 32);
      i32x8_t b;
      for (int i = 0; i < 8; ++i) b[i] = (int32_t)bp[i];
      const int sb = b_scales[(tsp * 16 + r) * 4 + kb];
      // A format 4 (FP4 E2M1), B format 0 (FP8 E4M3); scale bytes 0
      acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc, 4, 0, 0, sa, 0, sb);
    }
  }
  for (int v = 0; v < 4; ++v) out[(int64_t)(ct * 16 + r) * n_rows + rt * 16 + 4 * kb + v] = acc[v];
}

}  // namespace

extern "C" int fp4_fp8_gemm(const void* a_codes, const void* a_scales, const void* b_codes, const void* b_scales,
                            int row_tiles, int token_tiles, int n_steps, int n_planes, float* out, void* stream) {
  if (row_tiles <= 0 || token_tiles <= 0 || n_steps <= 0 || n_planes <= 0 || token_tiles > 65535) return -1;
  fp4_fp8_gemm_kernel<<<dim3(row_tiles, token_tiles), 64, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      static_cast<const uint8_t*>(a_codes), static_cast<const uint8_t*>(a_scales),
      static_cast<const uint8_t*>(b_codes), static_cast<const uint8_t*>(b_scales), n_steps, n_planes, row_tiles * 16,
      out);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}
