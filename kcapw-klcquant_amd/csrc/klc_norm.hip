// RMSNorm of the hidden state before each MoE layer of a stacked decode
// (gfx950).  One workgroup per token row: 16-byte loads, float64 sum of
// squares, then the reference's rounding points (streamed_attention.py:27-28):
// mean of squares in float32, + eps in float32, rsqrt rounded to bfloat16,
// then two bfloat16 multiplies each rounded to bfloat16.
#include "klc_common.h"

namespace klc {
namespace {

constexpr int kNormThreads = 256;
constexpr int kNormChunks = 4;  // 16-byte chunks per thread: hidden <= 256 * 4 * 8 = 8192

__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(const uint16_t* __restrict__ x,
                                                                const uint16_t* __restrict__ w,
                                                                uint16_t* __restrict__ out, int hidden, float eps) {
  __shared__ double partial[kNormThreads / kWave];
  const int64_t row = (int64_t)blockIdx.x * hidden;
  const int nchunk = hidden >> 3;
  uint4 xv[kNormChunks];
  double ss = 0.0;
#pragma unroll
  for (int i = 0; i < kNormChunks; ++i) {
    const int c = (int)threadIdx.x + i * kNormThreads;
    const uint4 v = *reinterpret_cast<const uint4*>(x + row + (int64_t)min(c, nchunk - 1) * 8);
    xv[i] = c < nchunk ? v : make_uint4(0u, 0u, 0u, 0u);
  }
#pragma unroll
  for (int i = 0; i < kNormChunks; ++i) {
    const uint32_t wd[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const double lo = (double)__uint_as_float(wd[q] << 16);
      const double hi = (double)__uint_as_float(wd[q] & 0xffff0000u);
      ss += lo * lo + hi * hi;  // each square is exact in float64
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = ss;
  __syncthreads();
  double tot = 0.0;
#pragma unroll
  for (int i = 0; i < kNormThreads / kWave; ++i) tot += partial[i];
  const float ms = (float)(tot / (double)hidden);
  const float s = ms + eps;
  const float r = round_bf16((float)(1.0 / sqrt((double)s)));
#pragma unroll
  for (int i = 0; i < kNormChunks; ++i) {
    const int c = (int)threadIdx.x + i * kNormThreads;
    if (c < nchunk) {
      const uint4 wv = *reinterpret_cast<const uint4*>(w + c * 8);
      const uint32_t xd[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
      const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
      uint32_t od[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float a0 = round_bf16(__uint_as_float(xd[q] << 16) * r) * __uint_as_float(wd[q] << 16);
        const float a1 = round_bf16(__uint_as_float(xd[q] & 0xffff0000u) * r) * __uint_as_float(wd[q] & 0xffff0000u);
        od[q] = f32_to_bf16_rne(a0) | (f32_to_bf16_rne(a1) << 16);
      }
      *reinterpret_cast<uint4*>(out + row + (int64_t)c * 8) = make_uint4(od[0], od[1], od[2], od[3]);
    }
  }
}

}  // namespace
}  // namespace klc

using namespace klc;

extern "C" int klc_rms_norm(const void* x, const void* weight, void* out, int64_t n_tokens, int64_t hidden, float eps,
                            void* stream) {
  KLC_REQUIRE(x && weight && out, KLC_ERR_ARGUMENT, "klc_rms_norm: null pointer");
  KLC_REQUIRE(n_tokens > 0 && hidden > 0, KLC_ERR_ARGUMENT, "klc_rms_norm: bad sizes n_tokens=%lld hidden=%lld",
              (long long)n_tokens, (long long)hidden);
  KLC_REQUIRE(hidden % 8 == 0, KLC_ERR_SHAPE, "klc_rms_norm: hidden=%lld must be a multiple of 8", (long long)hidden);
  KLC_REQUIRE(hidden <= kNormThreads * kNormChunks * 8 && n_tokens < ((int64_t)1 << 31), KLC_ERR_UNSUPPORTED,
              "klc_rms_norm: hidden=%lld > %d", (long long)hidden, kNormThreads * kNormChunks * 8);
  rms_norm_kernel<<<(unsigned)n_tokens, kNormThreads, 0, as_stream(stream)>>>(
      static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(out),
      (int)hidden, eps);
  return check_launch("rms_norm_kernel");
}
