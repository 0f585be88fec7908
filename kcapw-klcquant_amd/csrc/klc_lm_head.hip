// lm_head logits GEMV and the greedy next token (gfx950).
//
// logits[v] = f32(sum_h f64(w[v][h]) * f64(x[h])) for a resident bfloat16
// weight [V][H] and a float32 hidden state [H]: a bfloat16 x float32 product
// has at most 32 significant bits, so it is exact in float64, and the float64
// sum rounded once is the correctly rounded float32 dot product.  The pass
// is HBM bound (2 bytes per weight, 1.16 GB for gpt-oss's 201,088 x 2880
// head), so the float64 arithmetic rides under the stream.
//
// Each wavefront owns whole rows: lane l reads the 16-byte chunks l, l+64,
// ... of a row (a wave-wide load covers 1 KiB of contiguous weight) with
// non-temporal buffer loads, keeps its slice of x in registers as float64
// for every row, and two rows are in flight per iteration.  Measured on the
// gpt-oss head: plain global loads 5.7 TB/s whatever the grid, rows in
// flight or accumulator count; non-temporal buffer loads 6.7 TB/s.  A xor-shuffle sums a row across the wave.  The same
// pass keeps the best (nan_to_num(logit), first index) per workgroup; one
// small kernel reduces those to the token.
//
// Replaces StreamedTransformerExecutor.logits (streamed_transformer_executor.py:177-209),
// which multiplies 4096-row chunks in float32 and copies each to the host,
// and the nan_to_num + argmax of its callers (generation_runtime.py:118-122,
// inference_server.py:383-386).
#include <math.h>

#include "klc_common.h"

namespace klc {
namespace {

constexpr int kLmThreads = 256;
constexpr int kLmWaves = kLmThreads / kWave;
constexpr int kLmRows = 2;           // rows in flight per wave and iteration
constexpr int kLmMaxWorkgroups = 512;  // two per CU, each wave streams its rows

// torch.nan_to_num(v, nan=-1e9, posinf=1e9, neginf=-1e9)
__device__ __forceinline__ float nan_to_num(float v) {
  if (v != v) return -1e9f;
  if (isinf(v)) return v > 0.f ? 1e9f : -1e9f;
  return v;
}

// (value, index) order of argmax: larger value first, then the lower index
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

template <int J>
__global__ __launch_bounds__(kLmThreads) void lm_head_kernel(const uint16_t* __restrict__ w, const float* __restrict__ x,
                                                             float* __restrict__ logits, int vocab, int hidden,
                                                             float* __restrict__ part_val,
                                                             int32_t* __restrict__ part_idx) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int chunks = hidden / 8;  // 16-byte chunks of 8 bfloat16 per row
  double h[J][8];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int c = lane + kWave * j;
    if (c < chunks) {
      const float4 a = reinterpret_cast<const float4*>(x)[2 * c];
      const float4 b = reinterpret_cast<const float4*>(x)[2 * c + 1];
      h[j][0] = a.x, h[j][1] = a.y, h[j][2] = a.z, h[j][3] = a.w;
      h[j][4] = b.x, h[j][5] = b.y, h[j][6] = b.z, h[j][7] = b.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) h[j][i] = 0.0;
    }
  }
  float best_v = -INFINITY;
  int best_i = 0x7fffffff;
  const int waves = gridDim.x * kLmWaves;
  for (int r0 = (blockIdx.x * kLmWaves + wave) * kLmRows; r0 < vocab; r0 += waves * kLmRows) {
    uint4 v[kLmRows][J];
#pragma unroll
    for (int rr = 0; rr < kLmRows; ++rr) {
      // one buffer resource per row: lanes past the row's last chunk read 0
      const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(w + (int64_t)min(r0 + rr, vocab - 1) * hidden), (short)0, hidden * 2, kBufferWord3);
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const auto q = __builtin_amdgcn_raw_buffer_load_b128(rb, (unsigned)(lane + kWave * j) * 16u, 0, kStreamPolicy);
        v[rr][j] = make_uint4(q[0], q[1], q[2], q[3]);
      }
    }
#pragma unroll
    for (int rr = 0; rr < kLmRows; ++rr) {
      // four independent float64 chains per lane, summed at the end
      double acc[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const uint32_t q[4] = {v[rr][j].x, v[rr][j].y, v[rr][j].z, v[rr][j].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          acc[(2 * k) & 3] = fma((double)__uint_as_float(q[k] << 16), h[j][2 * k], acc[(2 * k) & 3]);
          acc[(2 * k + 1) & 3] = fma((double)__uint_as_float(q[k] & 0xffff0000u), h[j][2 * k + 1], acc[(2 * k + 1) & 3]);
        }
      }
      double sum = (acc[0] + acc[1]) + (acc[2] + acc[3]);
#pragma unroll
      for (int off = kWave / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
      const int r = r0 + rr;
      if (r < vocab) {  // every lane holds the row's sum
        const float lf = (float)sum;
        if (lane == 0) logits[r] = lf;
        const float m = nan_to_num(lf);
        if (better(m, r, best_v, best_i)) best_v = m, best_i = r;
      }
    }
  }
  __shared__ float sv[kLmWaves];
  __shared__ int si[kLmWaves];
  if (lane == 0) sv[wave] = best_v, si[wave] = best_i;
  __syncthreads();
  if (threadIdx.x == 0) {
    float bv = sv[0];
    int bi = si[0];
    for (int k = 1; k < kLmWaves; ++k)
      if (better(sv[k], si[k], bv, bi)) bv = sv[k], bi = si[k];
    part_val[blockIdx.x] = bv;
    part_idx[blockIdx.x] = bi;
  }
}

// One workgroup: the best of n partial (value, index) pairs.
__global__ __launch_bounds__(kLmThreads) void argmax_reduce_kernel(const float* __restrict__ part_val,
                                                                   const int32_t* __restrict__ part_idx, int n,
                                                                   int32_t* __restrict__ token,
                                                                   float* __restrict__ token_logit) {
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int k = threadIdx.x; k < n; k += kLmThreads)
    if (better(part_val[k], part_idx[k], bv, bi)) bv = part_val[k], bi = part_idx[k];
  __shared__ float sv[kLmThreads];
  __shared__ int si[kLmThreads];
  sv[threadIdx.x] = bv;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int s = kLmThreads / 2; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s && better(sv[threadIdx.x + s], si[threadIdx.x + s], sv[threadIdx.x], si[threadIdx.x])) {
      sv[threadIdx.x] = sv[threadIdx.x + s];
      si[threadIdx.x] = si[threadIdx.x + s];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    token[0] = si[0];
    if (token_logit != nullptr) token_logit[0] = sv[0];
  }
}

int lm_workgroups(int64_t vocab) {
  const int64_t want = (vocab + kLmWaves * kLmRows - 1) / (kLmWaves * kLmRows);
  return (int)(want < kLmMaxWorkgroups ? want : kLmMaxWorkgroups);
}

}  // namespace
}  // namespace klc

using namespace klc;

extern "C" int64_t klc_lm_head_workspace_bytes(int64_t vocab) {
  if (vocab <= 0) return set_error(KLC_ERR_ARGUMENT, "klc_lm_head_workspace_bytes: vocab=%lld", (long long)vocab);
  return (int64_t)lm_workgroups(vocab) * 8;
}

extern "C" int klc_lm_head_logits(const void* w, const float* x, float* logits, int64_t vocab, int64_t hidden,
                                  void* workspace, int64_t workspace_bytes, int32_t* token, float* token_logit,
                                  void* stream) {
  KLC_REQUIRE(w && x && logits && workspace && token, KLC_ERR_ARGUMENT, "klc_lm_head_logits: null pointer");
  KLC_REQUIRE(vocab > 0 && vocab < (1ll << 31) - 2 * kLmRows * kLmMaxWorkgroups * kLmWaves, KLC_ERR_ARGUMENT,
              "klc_lm_head_logits: vocab=%lld", (long long)vocab);
  KLC_REQUIRE(hidden > 0 && hidden % 8 == 0 && hidden <= 8 * 8 * kWave, KLC_ERR_UNSUPPORTED,
              "klc_lm_head_logits: hidden=%lld (a multiple of 8, at most %d)", (long long)hidden, 8 * 8 * kWave);
  KLC_REQUIRE(((uintptr_t)w | (uintptr_t)x | (uintptr_t)workspace) % 16 == 0, KLC_ERR_ARGUMENT,
              "klc_lm_head_logits: w, x and workspace must be 16-byte aligned");
  const int wgs = lm_workgroups(vocab);
  KLC_REQUIRE(workspace_bytes >= (int64_t)wgs * 8, KLC_ERR_ARGUMENT,
              "klc_lm_head_logits: workspace of %lld bytes, need %lld", (long long)workspace_bytes,
              (long long)wgs * 8);
  float* part_val = static_cast<float*>(workspace);
  int32_t* part_idx = reinterpret_cast<int32_t*>(part_val + wgs);
  hipStream_t st = as_stream(stream);
  const uint16_t* wb = static_cast<const uint16_t*>(w);
  const int J = (int)((hidden / 8 + kWave - 1) / kWave);
#define KLC_LM_CASE(n)                                                                                         \
  case n:                                                                                                      \
    lm_head_kernel<n><<<wgs, kLmThreads, 0, st>>>(wb, x, logits, (int)vocab, (int)hidden, part_val, part_idx); \
    break;
  switch (J) {
    KLC_LM_CASE(1)
    KLC_LM_CASE(2)
    KLC_LM_CASE(3)
    KLC_LM_CASE(4)
    KLC_LM_CASE(5)
    KLC_LM_CASE(6)
    KLC_LM_CASE(7)
    KLC_LM_CASE(8)
  }
#undef KLC_LM_CASE
  int rc = check_launch("lm_head_kernel");
  if (rc) return rc;
  argmax_reduce_kernel<<<1, kLmThreads, 0, st>>>(part_val, part_idx, wgs, token, token_logit);
  return check_launch("argmax_reduce_kernel");
}
