// Decode attention on a device-resident KV ring (gfx950): RoPE + append, and
// grouped-query attention with sink logits over a window of the ring.
//
// Replaces, for one decode token, apply_rope + KVCacheManager.append/get +
// the score / softmax / context steps of StreamedAttention.forward
// (streamed_attention.py:80-98, 120-141; kv_cache_manager.py:39-56).  The
// reference stacks the whole cache into fresh tensors every step and runs
// torch einsum/softmax; here the keys never move.
//
// Numerics follow the reference's cast points: RoPE rounds every bfloat16 op
// (a*cos, b*sin, difference/sum) and the rotated key and the value are
// stored in the cache's type (float16 by default, or bfloat16); scores are
// float32 q.k / sqrt(D) (the dot product accumulated in float64 and rounded
// once); the softmax over [scores, sink] is float32 with the maximum
// subtracted; probabilities are rounded to the cache's type before the value
// sum, which accumulates in float32 per split and float64 across splits, is
// rounded to the cache's type and then to bfloat16 (o_proj's input type).
//
// Kernels per step: scores (workgroup = one KV head x 64 keys, its whole
// query group), probabilities x values (workgroup = one query head x 256
// keys, each taking its head's max and sum over all the scores first), and
// the sum of the splits; a window of at most 256 keys (one split) runs as
// one launch, scores to context, one workgroup per query head.
#include <math.h>

#include "klc_common.h"

namespace klc {
namespace {

constexpr int kAttnThreads = 256;
constexpr int kScoreKeys = 64;   // keys per scores workgroup
constexpr int kPvKeys = 256;     // keys per value-sum workgroup
constexpr int kMaxHeadDim = 128;
constexpr int kMaxGroup = 16;    // query heads per KV head

__device__ __forceinline__ float bf(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ uint16_t to_bf(float f) { return (uint16_t)f32_to_bf16_rne(f); }
__device__ __forceinline__ float rbf(float f) { return bf(to_bf(f)); }
// the cache's element type: float16 (the reference's default "fp16") or bfloat16
__device__ __forceinline__ float kv_f(uint16_t b, bool f16) { return f16 ? __half2float(__ushort_as_half(b)) : bf(b); }
__device__ __forceinline__ uint16_t to_kv(float f, bool f16) {
  return f16 ? __half_as_ushort(__float2half_rn(f)) : to_bf(f);
}
__device__ __forceinline__ float rkv(float f, bool f16) { return kv_f(to_kv(f, f16), f16); }

// q [NH][D], k/v [NKV][D] -> q_out [NH][D]; k, v into ring slot `slot`.
__global__ __launch_bounds__(kAttnThreads) void rope_append_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ cosv, const uint16_t* __restrict__ sinv, uint16_t* __restrict__ q_out,
    uint16_t* __restrict__ k_out, uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache, int64_t slot, int nh, int nkv, int d, bool f16) {
  const int half = d / 2;
  const int pairs = (nh + nkv) * half;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < pairs + nkv * d; i += gridDim.x * blockDim.x) {
    if (i < pairs) {
      const int row = i / half, j = i - row * half;
      const bool is_q = row < nh;
      const uint16_t* src = is_q ? q + (int64_t)row * d : k + (int64_t)(row - nh) * d;
      uint16_t* dst = is_q ? q_out + (int64_t)row * d : k_cache + (slot * nkv + (row - nh)) * d;
      const float a = bf(src[j]), b = bf(src[j + half]), c = bf(cosv[j]), s = bf(sinv[j]);
      const float lo = rbf(rbf(a * c) - rbf(b * s)), hi = rbf(rbf(b * c) + rbf(a * s));  // bfloat16 rotation
      dst[j] = is_q ? to_bf(lo) : to_kv(lo, f16);  // the key is stored in the cache's type
      dst[j + half] = is_q ? to_bf(hi) : to_kv(hi, f16);
      if (!is_q && k_out != nullptr) {  // the rotated key before storage, for diagnostics
        k_out[(int64_t)(row - nh) * d + j] = to_bf(lo);
        k_out[(int64_t)(row - nh) * d + j + half] = to_bf(hi);
      }
    } else {
      const int e = i - pairs;
      v_cache[slot * nkv * d + e] = f16 ? to_kv(bf(v[e]), true) : v[e];
    }
  }
}

// scores[h][i] for the keys i in [64 * blockIdx.y, +64) of KV head blockIdx.x
__global__ __launch_bounds__(kAttnThreads) void attn_scores_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_cache, float* __restrict__ scores, int64_t cap,
    int64_t first, int count, int nh, int nkv, int d, float sqrt_d, bool f16) {
  __shared__ float qs[kMaxGroup][kMaxHeadDim];
  const int g = nh / nkv, kvh = blockIdx.x;
  const int key = blockIdx.y * kScoreKeys + (threadIdx.x % kScoreKeys);
  const int part = threadIdx.x / kScoreKeys;  // 4 parts share the group's heads
  const bool live = key < count;
  // the key row goes into registers before the query staging, so its loads
  // overlap the staging and its barrier
  uint4 kr[kMaxHeadDim / 8] = {};
  const uint16_t* krow = k_cache + (((first + (live ? key : 0)) % cap) * nkv + kvh) * d;
#pragma unroll
  for (int c = 0; c < kMaxHeadDim / 8; ++c)
    if (live && c * 8 < d) kr[c] = *reinterpret_cast<const uint4*>(krow + c * 8);
  for (int i = threadIdx.x; i < g * d; i += blockDim.x) qs[i / d][i % d] = bf(q[(int64_t)(kvh * g + i / d) * d + i % d]);
  __syncthreads();
  if (!live) return;
  for (int hh = part; hh < g; hh += kAttnThreads / kScoreKeys) {
    double acc = 0.0;
#pragma unroll
    for (int c = 0; c < kMaxHeadDim / 8; ++c) {
      if (c * 8 >= d) break;
      // opaque per head: the conversions stay in the loop instead of being
      // hoisted as 128 float64 values
      uint32_t wd[4] = {kr[c].x, kr[c].y, kr[c].z, kr[c].w};
      asm volatile("" : "+v"(wd[0]), "+v"(wd[1]), "+v"(wd[2]), "+v"(wd[3]));
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        acc = fma((double)kv_f((uint16_t)(wd[t] & 0xffffu), f16), (double)qs[hh][8 * c + 2 * t], acc);
        acc = fma((double)kv_f((uint16_t)(wd[t] >> 16), f16), (double)qs[hh][8 * c + 2 * t + 1], acc);
      }
    }
    scores[(int64_t)(kvh * g + hh) * count + key] = (float)acc / sqrt_d;
  }
}

// Query head h's m = max(scores, sink) and l = sum exp(x - m) over [scores,
// sink], l summed in float64 and rounded once; each reduction is a wave
// shuffle tree plus one exchange of the 4 waves' values.  Every thread of
// the workgroup calls it and gets both.
__device__ __forceinline__ void head_stats(const float* __restrict__ s, int count, const uint16_t* __restrict__ sinks,
                                           int h, float& m_out, float& l_out) {
  __shared__ float wm[kAttnThreads / kWave];
  __shared__ double wl[kAttnThreads / kWave];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  // both passes issue 8 loads before using them (a thread's scores are
  // otherwise a chain of dependent L2 round trips); the sum keeps the
  // thread's order i, i + 256, ...
  constexpr int kAhead = 8;
  float m = sinks != nullptr ? bf(sinks[h]) : -INFINITY;
  int i = threadIdx.x;
  for (; i + (kAhead - 1) * kAttnThreads < count; i += kAhead * kAttnThreads) {
    float x[kAhead];
#pragma unroll
    for (int j = 0; j < kAhead; ++j) x[j] = s[i + j * kAttnThreads];
#pragma unroll
    for (int j = 0; j < kAhead; ++j) m = fmaxf(m, x[j]);
  }
  for (; i < count; i += kAttnThreads) m = fmaxf(m, s[i]);
  for (int off = kWave / 2; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if (lane == 0) wm[wave] = m;
  __syncthreads();
  m = wm[0];
  for (int w = 1; w < kAttnThreads / kWave; ++w) m = fmaxf(m, wm[w]);
  double l = 0.0;
  i = threadIdx.x;
  for (; i + (kAhead - 1) * kAttnThreads < count; i += kAhead * kAttnThreads) {
    float x[kAhead];
#pragma unroll
    for (int j = 0; j < kAhead; ++j) x[j] = s[i + j * kAttnThreads];
#pragma unroll
    for (int j = 0; j < kAhead; ++j) l += (double)expf(x[j] - m);
  }
  for (; i < count; i += kAttnThreads) l += (double)expf(s[i] - m);
  if (threadIdx.x == 0 && sinks != nullptr) l += (double)expf(bf(sinks[h]) - m);
  for (int off = kWave / 2; off > 0; off >>= 1) l += __shfl_xor(l, off);
  if (lane == 0) wl[wave] = l;
  __syncthreads();
  double t = 0.0;
  for (int w = 0; w < kAttnThreads / kWave; ++w) t += wl[w];
  m_out = m;
  l_out = (float)t;
}

// The body of a value workgroup: partial[h][split][d] = sum over the
// split's keys of p * v, p rounded to the cache type, for query head
// h = blockIdx.x whose `count` scores s_head holds (global memory or LDS).
// The workgroup first takes its head's max and sum over all the scores
// (16 KB of L2 reads at 4,096 keys: cheaper than a launch of its own).
// kWhole (count <= 256, one split): it also writes the context, so the step
// needs no combine launch.
template <bool kWhole>
__device__ __forceinline__ void pv_body(const float* __restrict__ s_head, const uint16_t* __restrict__ sinks,
                                        const uint16_t* __restrict__ v_cache, float* __restrict__ partial,
                                        uint16_t* __restrict__ context, int64_t cap, int64_t first, int count, int nh,
                                        int nkv, int d, bool f16) {
  __shared__ float p[kPvKeys];
  __shared__ float acc_s[kAttnThreads / 32][kMaxHeadDim];
  const int h = blockIdx.x, split = blockIdx.y, g = nh / nkv, kvh = h / g;
  const int k0 = split * kPvKeys, nk = min(kPvKeys, count - k0);
  float m, l;
  head_stats(s_head, count, sinks, h, m, l);
  for (int i = threadIdx.x; i < nk; i += kAttnThreads) p[i] = rkv(expf(s_head[k0 + i] - m) / l, f16);
  __syncthreads();
  // thread (slice, four dims): slices of keys; each thread issues the 8-byte
  // loads of four keys before their multiply-adds, so L2 round trips overlap
  const int quads = d / 4, slices = kAttnThreads / quads;
  const int dq = threadIdx.x % quads, sl = threadIdx.x / quads;
  float a[4] = {0.f, 0.f, 0.f, 0.f};
  auto vrow = [&](int i) {
    return *reinterpret_cast<const uint2*>(v_cache + (((first + k0 + i) % cap) * nkv + kvh) * d + 4 * dq);
  };
  auto add = [&](float pi, uint2 w) {
    a[0] = fmaf(pi, kv_f((uint16_t)(w.x & 0xffffu), f16), a[0]);
    a[1] = fmaf(pi, kv_f((uint16_t)(w.x >> 16), f16), a[1]);
    a[2] = fmaf(pi, kv_f((uint16_t)(w.y & 0xffffu), f16), a[2]);
    a[3] = fmaf(pi, kv_f((uint16_t)(w.y >> 16), f16), a[3]);
  };
  if (sl < slices) {
    int i = sl;
    for (; i + 3 * slices < nk; i += 4 * slices) {
      const uint2 w0 = vrow(i), w1 = vrow(i + slices), w2 = vrow(i + 2 * slices), w3 = vrow(i + 3 * slices);
      add(p[i], w0);
      add(p[i + slices], w1);
      add(p[i + 2 * slices], w2);
      add(p[i + 3 * slices], w3);
    }
    for (; i < nk; i += slices) add(p[i], vrow(i));
  }
  // sum the slices, kAttnThreads / 32 of them at a time through LDS
  for (int base = 0; base < slices; base += kAttnThreads / 32) {
    if (sl >= base && sl < base + kAttnThreads / 32) {
#pragma unroll
      for (int e = 0; e < 4; ++e) acc_s[sl - base][4 * dq + e] = a[e];
    }
    __syncthreads();
    if ((int)threadIdx.x < d) {
      float t = 0.f;
      for (int s2 = 0; s2 < min(kAttnThreads / 32, slices - base); ++s2) t += acc_s[s2][threadIdx.x];
      float* out = partial + ((int64_t)h * gridDim.y + split) * d + threadIdx.x;
      *out = base == 0 ? t : *out + t;
    }
    __syncthreads();
  }
  if constexpr (kWhole) {
    if ((int)threadIdx.x < d) {
      const float t = partial[((int64_t)h * gridDim.y + split) * d + threadIdx.x];
      context[(int64_t)h * d + threadIdx.x] = to_bf(rkv(t, f16));
    }
  }
}

__global__ __launch_bounds__(kAttnThreads) void attn_pv_kernel(const float* __restrict__ scores,
                                                               const uint16_t* __restrict__ sinks,
                                                               const uint16_t* __restrict__ v_cache,
                                                               float* __restrict__ partial,
                                                               uint16_t* __restrict__ context, int64_t cap,
                                                               int64_t first, int count, int nh, int nkv, int d,
                                                               bool f16) {
  pv_body<false>(scores + (int64_t)blockIdx.x * count, sinks, v_cache, partial, context, cap, first, count, nh, nkv,
                 d, f16);
}

// A window of at most 256 keys in one launch: workgroup = query head
// blockIdx.x.  Its scores (the same float64 dot products as
// attn_scores_kernel, one key per thread) go to LDS, then the value body
// takes the max, the sum and the context.
__global__ __launch_bounds__(kAttnThreads) void attn_window_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_cache, const uint16_t* __restrict__ sinks,
    const uint16_t* __restrict__ v_cache, float* __restrict__ partial, uint16_t* __restrict__ context, int64_t cap,
    int64_t first, int count, int nh, int nkv, int d, float sqrt_d, bool f16) {
  __shared__ float qs[kMaxHeadDim];
  __shared__ float sc[kPvKeys];
  const int h = blockIdx.x, kvh = h / (nh / nkv);
  const int key = threadIdx.x;
  const bool live = key < count;
  uint4 kr[kMaxHeadDim / 8] = {};
  const uint16_t* krow = k_cache + (((first + (live ? key : 0)) % cap) * nkv + kvh) * d;
#pragma unroll
  for (int c = 0; c < kMaxHeadDim / 8; ++c)
    if (live && c * 8 < d) kr[c] = *reinterpret_cast<const uint4*>(krow + c * 8);
  for (int i = threadIdx.x; i < d; i += blockDim.x) qs[i] = bf(q[(int64_t)h * d + i]);
  __syncthreads();
  if (live) {
    double acc = 0.0;
#pragma unroll
    for (int c = 0; c < kMaxHeadDim / 8; ++c) {
      if (c * 8 >= d) break;
      const uint32_t wd[4] = {kr[c].x, kr[c].y, kr[c].z, kr[c].w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        acc = fma((double)kv_f((uint16_t)(wd[t] & 0xffffu), f16), (double)qs[8 * c + 2 * t], acc);
        acc = fma((double)kv_f((uint16_t)(wd[t] >> 16), f16), (double)qs[8 * c + 2 * t + 1], acc);
      }
    }
    sc[key] = (float)acc / sqrt_d;
  }
  __syncthreads();
  pv_body<true>(sc, sinks, v_cache, partial, context, cap, first, count, nh, nkv, d, f16);
}

// context[h][d] = bf16(sum over splits of partial[h][split][d])
__global__ __launch_bounds__(kAttnThreads) void attn_combine_kernel(const float* __restrict__ partial, int splits,
                                                                    int nh, int d, uint16_t* __restrict__ context,
                                                                    bool f16) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nh * d) return;
  const int h = i / d, e = i - h * d;
  const float* src = partial + (int64_t)h * splits * d + e;
  // 8 loads in flight, summed in split order
  double t = 0.0;
  int s = 0;
  for (; s + 7 < splits; s += 8) {
    float x[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = src[(int64_t)(s + j) * d];
#pragma unroll
    for (int j = 0; j < 8; ++j) t += x[j];
  }
  for (; s < splits; ++s) t += src[(int64_t)s * d];
  context[i] = to_bf(rkv((float)t, f16));  // the cache type's einsum result, then bfloat16
}

int64_t attn_splits(int64_t count) { return (count + kPvKeys - 1) / kPvKeys; }

}  // namespace
}  // namespace klc

using namespace klc;

extern "C" int klc_rope_append(const void* q, const void* k, const void* v, const void* cos_half,
                               const void* sin_half, void* q_out, void* k_out, void* k_cache, void* v_cache,
                               int64_t slot,
                               int64_t cap, int64_t n_heads, int64_t n_kv, int64_t head_dim, int kv_dtype,
                               void* stream) {
  KLC_REQUIRE(q && k && v && cos_half && sin_half && q_out && k_cache && v_cache, KLC_ERR_ARGUMENT,
              "klc_rope_append: null pointer");
  KLC_REQUIRE(n_heads > 0 && n_kv > 0 && head_dim > 0 && head_dim % 2 == 0 && head_dim <= kMaxHeadDim &&
                  n_heads % n_kv == 0 && n_heads <= 4096,
              KLC_ERR_SHAPE, "klc_rope_append: heads %lld / %lld, head_dim %lld", (long long)n_heads,
              (long long)n_kv, (long long)head_dim);
  KLC_REQUIRE(slot >= 0 && slot < cap, KLC_ERR_ARGUMENT, "klc_rope_append: slot %lld of %lld", (long long)slot,
              (long long)cap);
  KLC_REQUIRE(kv_dtype == KLC_DTYPE_BF16 || kv_dtype == KLC_DTYPE_F16, KLC_ERR_UNSUPPORTED,
              "klc_rope_append: kv_dtype %d (bfloat16 or float16)", kv_dtype);
  const int64_t items = (n_heads + n_kv) * (head_dim / 2) + n_kv * head_dim;  // one thread each
  rope_append_kernel<<<(unsigned)((items + kAttnThreads - 1) / kAttnThreads), kAttnThreads, 0, as_stream(stream)>>>(
      static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
      static_cast<const uint16_t*>(cos_half), static_cast<const uint16_t*>(sin_half), static_cast<uint16_t*>(q_out),
      static_cast<uint16_t*>(k_out), static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), slot, (int)n_heads, (int)n_kv,
      (int)head_dim, kv_dtype == KLC_DTYPE_F16);
  return check_launch("rope_append_kernel");
}

extern "C" int64_t klc_attn_workspace_bytes(int64_t n_heads, int64_t head_dim, int64_t count) {
  if (n_heads <= 0 || head_dim <= 0 || count <= 0)
    return set_error(KLC_ERR_ARGUMENT, "klc_attn_workspace_bytes: bad sizes");
  return 4 * (n_heads * count + n_heads * attn_splits(count) * head_dim);
}

extern "C" int klc_attn_decode(const void* q, const void* k_cache, const void* v_cache, const void* sinks,
                               int64_t cap, int64_t first, int64_t count, int64_t n_heads, int64_t n_kv,
                               int64_t head_dim, int kv_dtype, void* workspace, int64_t workspace_bytes,
                               void* context, void* stream) {
  KLC_REQUIRE(q && k_cache && v_cache && workspace && context, KLC_ERR_ARGUMENT, "klc_attn_decode: null pointer");
  KLC_REQUIRE(n_heads > 0 && n_kv > 0 && n_heads % n_kv == 0 && n_heads / n_kv <= kMaxGroup && head_dim >= 8 &&
                  head_dim % 8 == 0 && head_dim <= kMaxHeadDim,
              KLC_ERR_SHAPE, "klc_attn_decode: heads %lld / %lld (group <= %d), head_dim %lld (8..%d, multiple of 8)",
              (long long)n_heads, (long long)n_kv, kMaxGroup, (long long)head_dim, kMaxHeadDim);
  KLC_REQUIRE(cap > 0 && count > 0 && count <= cap && first >= 0 && first < cap && count <= (1 << 22) &&
                  n_heads * count < ((int64_t)1 << 31),
              KLC_ERR_ARGUMENT, "klc_attn_decode: %lld keys from slot %lld of a %lld-slot ring", (long long)count,
              (long long)first, (long long)cap);
  KLC_REQUIRE(((uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)workspace) % 16 == 0, KLC_ERR_ARGUMENT,
              "klc_attn_decode: caches and workspace must be 16-byte aligned");
  KLC_REQUIRE(kv_dtype == KLC_DTYPE_BF16 || kv_dtype == KLC_DTYPE_F16, KLC_ERR_UNSUPPORTED,
              "klc_attn_decode: kv_dtype %d (bfloat16 or float16)", kv_dtype);
  const bool f16 = kv_dtype == KLC_DTYPE_F16;
  const int64_t need = klc_attn_workspace_bytes(n_heads, head_dim, count);
  KLC_REQUIRE(workspace_bytes >= need, KLC_ERR_ARGUMENT, "klc_attn_decode: workspace of %lld bytes, need %lld",
              (long long)workspace_bytes, (long long)need);
  float* scores = static_cast<float*>(workspace);
  float* partial = scores + n_heads * count;
  const int splits = (int)attn_splits(count);
  hipStream_t st = as_stream(stream);
  const uint16_t* qb = static_cast<const uint16_t*>(q);
  const uint16_t* kb = static_cast<const uint16_t*>(k_cache);
  const uint16_t* vb = static_cast<const uint16_t*>(v_cache);
  const uint16_t* sk = static_cast<const uint16_t*>(sinks);
  uint16_t* ctx = static_cast<uint16_t*>(context);
  const float sqrt_d = sqrtf((float)head_dim);
  if (splits == 1) {  // a window of at most 256 keys: one launch, one workgroup per query head
    static_assert(kPvKeys == kAttnThreads, "one key per thread");
    attn_window_kernel<<<(unsigned)n_heads, kAttnThreads, 0, st>>>(
        qb, kb, sk, vb, partial, ctx, cap, first, (int)count, (int)n_heads, (int)n_kv, (int)head_dim, sqrt_d, f16);
    return check_launch("attn_window_kernel");
  }
  attn_scores_kernel<<<dim3((unsigned)n_kv, (unsigned)((count + kScoreKeys - 1) / kScoreKeys)), kAttnThreads, 0, st>>>(
      qb, kb, scores, cap, first, (int)count, (int)n_heads, (int)n_kv, (int)head_dim, sqrt_d, f16);
  int rc = check_launch("attn_scores_kernel");
  if (rc) return rc;
  attn_pv_kernel<<<dim3((unsigned)n_heads, (unsigned)splits), kAttnThreads, 0, st>>>(
      scores, sk, vb, partial, ctx, cap, first, (int)count, (int)n_heads, (int)n_kv, (int)head_dim, f16);
  if ((rc = check_launch("attn_pv_kernel"))) return rc;
  attn_combine_kernel<<<(unsigned)((n_heads * head_dim + kAttnThreads - 1) / kAttnThreads), kAttnThreads, 0, st>>>(
      partial, splits, (int)n_heads, (int)head_dim, static_cast<uint16_t*>(context), f16);
  return check_launch("attn_combine_kernel");
}
