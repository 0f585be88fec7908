// Router logits, top-k + softmax, and expert-sorted dispatch (gfx950).
//
// Logits: one wave per (expert, block of 8 tokens).  Lanes stride the hidden
// dimension with 16-byte loads; each bfloat16 product is exact in float32 and
// is accumulated in float64, so the only roundings are the reference's own:
// float32 of the dot product, float32 bias add, bfloat16 result
// (streamed_moe_router.py:269).
//
// Top-k: one wave per token.  Each logit becomes a 64-bit key (ordered value
// bits, then inverted expert index), so a wave-wide max picks the largest
// value and, among equal values, the lowest expert index; k rounds of that
// give the descending top-k.  The softmax over the k values is evaluated in
// float64 and rounded to float32, then to bfloat16.
//
// Dispatch: one workgroup performs a stable counting sort of the (token, slot)
// pairs by expert: per-64-pair-chunk histograms from wave ballots, an
// exclusive scan over chunks and experts, then an in-order scatter.
#include "klc_common.h"

namespace klc {
namespace {

constexpr int kRouterTok = 8;     // tokens per workgroup
constexpr int kRouterChunks = 8;  // 16-byte weight chunks per lane: hidden <= 64 * 8 * 8 = 4096

// One wave per (expert, block of up to 8 tokens).  The workgroup stages the
// block's hidden rows in LDS; every lane first issues all of its weight-row
// loads, then accumulates float64 sums of exact float32 products per token.
__device__ void router_logits_tile(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                   const uint16_t* __restrict__ b, uint16_t* logits, float* __restrict__ x_f32,
                                   int n_tok, int hidden, int n_exp, uint16_t* xs /* LDS [kRouterTok][hidden] */) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int t0 = blockIdx.y * kRouterTok;
  const int nt = min(kRouterTok, n_tok - t0);
  const int e = blockIdx.x * 4 + wave;
  const int nchunk = hidden >> 3;  // hidden % 8 == 0 (checked on the host)

  // every load is unconditional (indices clamped into range, surplus values
  // discarded) so all of a lane's loads are in flight together
  uint4 wv[kRouterChunks];
  {
    const uint16_t* wr = w + (int64_t)min(e, n_exp - 1) * hidden;
#pragma unroll
    for (int i = 0; i < kRouterChunks; ++i) {
      const int c = lane + i * kWave;
      const uint4 v = *reinterpret_cast<const uint4*>(wr + min(c, nchunk - 1) * 8);
      wv[i] = c < nchunk ? v : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  const int64_t base = (int64_t)t0 * hidden;
  const int n_stage = nt * nchunk;
  constexpr int kStage = kRouterTok * kWave * kRouterChunks / 256;  // chunks per thread (blockDim.x == 256)
  uint4 xv[kStage];
#pragma unroll
  for (int j = 0; j < kStage; ++j) {
    const int i = min((int)threadIdx.x + j * 256, n_stage - 1);
    xv[j] = *reinterpret_cast<const uint4*>(x + base + (int64_t)i * 8);
  }
#pragma unroll
  for (int j = 0; j < kStage; ++j) {
    const int i = (int)threadIdx.x + j * 256;
    if (i < n_stage) {
      const uint4 v = xv[j];
      *reinterpret_cast<uint4*>(xs + i * 8) = v;
      if (x_f32 != nullptr && blockIdx.x == 0) {
        const uint32_t words[4] = {v.x, v.y, v.z, v.w};
        float4* dst = reinterpret_cast<float4*>(x_f32 + base + (int64_t)i * 8);
        dst[0] = make_float4(__uint_as_float(words[0] << 16), __uint_as_float(words[0] & 0xffff0000u),
                             __uint_as_float(words[1] << 16), __uint_as_float(words[1] & 0xffff0000u));
        dst[1] = make_float4(__uint_as_float(words[2] << 16), __uint_as_float(words[2] & 0xffff0000u),
                             __uint_as_float(words[3] << 16), __uint_as_float(words[3] & 0xffff0000u));
      }
    }
  }
  __syncthreads();
  if (e >= n_exp) return;  // the caller synchronises the block only after this function

  double acc[kRouterTok];
#pragma unroll
  for (int j = 0; j < kRouterTok; ++j) {
    acc[j] = 0.0;
    if (j < nt) {
      double s = 0.0;
#pragma unroll
      for (int i = 0; i < kRouterChunks; ++i) {
        const int c = lane + i * kWave;
        if (c < nchunk) {
          const uint4 xv = *reinterpret_cast<const uint4*>(xs + j * hidden + c * 8);
          const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
          const uint32_t ww[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            s += (double)(__uint_as_float(xw[q] << 16) * __uint_as_float(ww[q] << 16));
            s += (double)(__uint_as_float(xw[q] & 0xffff0000u) * __uint_as_float(ww[q] & 0xffff0000u));
          }
        }
      }
      acc[j] = s;
    }
  }
#pragma unroll
  for (int j = 0; j < kRouterTok; ++j) {
    if (j < nt) {
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) acc[j] += __shfl_xor(acc[j], off);
    }
  }
  if (lane < nt) {
    double mine = 0.0;
#pragma unroll
    for (int j = 0; j < kRouterTok; ++j)
      if (j == lane) mine = acc[j];
    logits[(int64_t)(t0 + lane) * n_exp + e] = (uint16_t)f32_to_bf16_rne((float)mine + bf16_to_f32(b[e]));
  }
}

// Logits on the float64 matrix cores: one workgroup per tile of 16 experts x
// 16 tokens, its 4 waves splitting the hidden dimension into quarters.  Per
// 32-deep chunk lane l loads 8 consecutive weights of expert row l % 16 and
// 8 hidden values of token l % 16 (k = 32 c + 8 (l / 16) + i), converts them
// to float64 (bfloat16 products are exact in float64) and issues 8
// v_mfma_f64_16x16x4_f64 (A lane l = row l % 16, k = l / 16; B lane l =
// column l % 16, same k; D lane l register i = row l / 16 + 4 i, column
// l % 16), alternating two accumulators.  The quarters are summed through LDS
// in wave order, then rounded like F.linear in bfloat16: bf16(f32(sum) + b).
typedef double f64x4_t __attribute__((ext_vector_type(4)));
constexpr int kRouterMfmaRows = 16;

__device__ void router_logits_mfma_tile(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                        const uint16_t* __restrict__ b, uint16_t* logits, float* __restrict__ x_f32,
                                        int n_tok, int hidden, int n_exp, int e0, int t0,
                                        double* red /* LDS [3][64][4] */) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int nchunk = (hidden + 31) >> 5;
  const int per = (nchunk + 3) >> 2;
  const int c0 = wave * per;
  const int c1 = min(c0 + per, nchunk);
  const uint16_t* wrow = w + (int64_t)min(e0 + r, n_exp - 1) * hidden;
  const int tok = t0 + r;
  const uint16_t* xrow = x + (int64_t)min(tok, n_tok - 1) * hidden;
  f64x4_t acc0 = {0.0, 0.0, 0.0, 0.0}, acc1 = {0.0, 0.0, 0.0, 0.0};
  for (int c = c0; c < c1; ++c) {
    const int k = c * 32 + g * 8;
    const bool ok = k < hidden;  // hidden % 8 == 0: a lane's 8 values are all in or all out
    const int kc = ok ? k : 0;
    uint4 wv = *reinterpret_cast<const uint4*>(wrow + kc);
    uint4 xv = *reinterpret_cast<const uint4*>(xrow + kc);
    if (!ok) {
      wv = make_uint4(0u, 0u, 0u, 0u);
      xv = make_uint4(0u, 0u, 0u, 0u);
    }
    if (x_f32 != nullptr && e0 == 0 && ok && tok < n_tok) {
      float4* dst = reinterpret_cast<float4*>(x_f32 + (int64_t)tok * hidden + k);
      dst[0] = make_float4(__uint_as_float(xv.x << 16), __uint_as_float(xv.x & 0xffff0000u),
                           __uint_as_float(xv.y << 16), __uint_as_float(xv.y & 0xffff0000u));
      dst[1] = make_float4(__uint_as_float(xv.z << 16), __uint_as_float(xv.z & 0xffff0000u),
                           __uint_as_float(xv.w << 16), __uint_as_float(xv.w & 0xffff0000u));
    }
    const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc0 = __builtin_amdgcn_mfma_f64_16x16x4f64((double)__uint_as_float(ww[q] << 16),
                                                   (double)__uint_as_float(xw[q] << 16), acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f64_16x16x4f64((double)__uint_as_float(ww[q] & 0xffff0000u),
                                                   (double)__uint_as_float(xw[q] & 0xffff0000u), acc1, 0, 0, 0);
    }
  }
  f64x4_t acc = acc0 + acc1;
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) red[((wave - 1) * 64 + lane) * 4 + i] = acc[i];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int q = 0; q < 3; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] += red[(q * 64 + lane) * 4 + i];
    if (tok < n_tok) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = e0 + g + 4 * i;
        if (e < n_exp)
          logits[(int64_t)tok * n_exp + e] = (uint16_t)f32_to_bf16_rne((float)acc[i] + bf16_to_f32(b[e]));
      }
    }
  }
}

__global__ __launch_bounds__(256) void router_logits_mfma_kernel(const uint16_t* __restrict__ x,
                                                                 const uint16_t* __restrict__ w,
                                                                 const uint16_t* __restrict__ b,
                                                                 uint16_t* __restrict__ logits,
                                                                 float* __restrict__ x_f32, int n_tok, int hidden,
                                                                 int n_exp) {
  __shared__ double red[3 * 64 * 4];
  router_logits_mfma_tile(x, w, b, logits, x_f32, n_tok, hidden, n_exp, blockIdx.x * kRouterMfmaRows,
                          blockIdx.y * kRouterMfmaRows, red);
}

// Orderable key: larger key = larger logit; NaN is the largest value; -0 == +0;
// among equal values the lower expert index has the larger key.
__device__ __forceinline__ uint64_t logit_key(uint32_t bf16bits, int idx) {
  uint32_t u = bf16bits << 16;
  uint32_t k32;
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    k32 = 0xffffffffu;
  } else {
    if ((u & 0x7fffffffu) == 0u) u = 0u;
    k32 = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  }
  return ((uint64_t)k32 << 32) | (uint64_t)(0xffffffffu - (uint32_t)idx);
}

constexpr int kTopkMaxPerLane = 16;  // n_experts <= 1024

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint64_t o = __shfl_xor(v, off);
    v = o > v ? o : v;
  }
  return v;
}

// Top-k + softmax of one token's logits row by one wave.
__device__ void topk_softmax_row(const uint16_t* row, int n_exp, int k, int64_t t, int32_t* __restrict__ ids,
                                 float* __restrict__ values, uint16_t* __restrict__ weights) {
  const int lane = threadIdx.x & 63;
  uint64_t keys[kTopkMaxPerLane];
#pragma unroll
  for (int s = 0; s < kTopkMaxPerLane; ++s) {
    const int idx = lane + s * kWave;
    keys[s] = idx < n_exp ? logit_key(row[idx], idx) : 0ull;
  }
  // lane r keeps the r-th selection
  int my_id = 0;
  float my_val = 0.0f;
  for (int r = 0; r < k; ++r) {
    uint64_t best = 0ull;
#pragma unroll
    for (int s = 0; s < kTopkMaxPerLane; ++s) best = keys[s] > best ? keys[s] : best;
    best = wave_max_u64(best);
#pragma unroll
    for (int s = 0; s < kTopkMaxPerLane; ++s)
      if (keys[s] == best) keys[s] = 0ull;
    if (lane == r) {
      my_id = (int)(0xffffffffu - (uint32_t)(best & 0xffffffffull));
      my_val = bf16_to_f32(row[my_id]);
    }
  }
  // softmax over the k values: max is the first selection (NaN propagates),
  // exponentials summed in selection order, all in float64
  const double mx = (double)__shfl(my_val, 0);
  double sum = 0.0;
  for (int r = 0; r < k; ++r) sum += exp((double)__shfl(my_val, r) - mx);
  if (lane < k) {
    const int64_t o = t * k + lane;
    ids[o] = my_id;
    if (values) values[o] = my_val;
    weights[o] = (uint16_t)f32_to_bf16_rne((float)(exp((double)my_val - mx) / sum));
  }
}

__global__ __launch_bounds__(256) void topk_softmax_kernel(const uint16_t* __restrict__ logits,
                                                           int32_t* __restrict__ ids, float* __restrict__ values,
                                                           uint16_t* __restrict__ weights, int n_tok, int n_exp,
                                                           int k) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= n_tok) return;
  topk_softmax_row(logits + (int64_t)t * n_exp, n_exp, k, t, ids, values, weights);
}

// Softmax of caller-chosen scores (one thread per token): the routing-locality
// path picks the experts on the host and hands over their fp32 scores.  The
// maximum propagates NaN; exponentials are summed in slot order in float64.
__global__ __launch_bounds__(256) void softmax_weights_kernel(const float* __restrict__ values,
                                                              uint16_t* __restrict__ weights, int n_tok, int k) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_tok) return;
  const float* v = values + (int64_t)t * k;
  double mx = (double)v[0];
  for (int r = 1; r < k; ++r) {
    const double x = (double)v[r];
    mx = (x != x || x > mx) ? x : mx;
  }
  double sum = 0.0;
  for (int r = 0; r < k; ++r) sum += exp((double)v[r] - mx);
  for (int r = 0; r < k; ++r)
    weights[(int64_t)t * k + r] = (uint16_t)f32_to_bf16_rne((float)(exp((double)v[r] - mx) / sum));
}

constexpr int kDispatchThreads = 256;
constexpr int kDispatchMaxExperts = 256;

// Exclusive prefix sum of LDS array `v[n]` (n <= 256) by the calling wave;
// total written to *total.  4 entries per lane.
__device__ void wave_exclusive_scan_256(int32_t* v, int n, int32_t* total, int lane) {
  int32_t local[4];
  int32_t s = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = lane * 4 + i;
    local[i] = idx < n ? v[idx] : 0;
    s += local[i];
  }
  int32_t incl = s;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int32_t o = __shfl_up(incl, off);
    if (lane >= off) incl += o;
  }
  int32_t run = incl - s;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = lane * 4 + i;
    if (idx < n) v[idx] = run;
    run += local[i];
  }
  if (lane == kWave - 1) *total = incl;
}

// Pairs are taken in chunks of 64 (one wave-wide pass); wave w owns the
// contiguous chunks [w * cpw, (w + 1) * cpw), cpw = ceil(chunks / 4), and
// ranks its pairs among the wave's earlier pairs of the same expert.  A wave
// takes 4 chunks at a time so that their ballots overlap.
constexpr int kDispatchChunk = kWave;
constexpr int kDispatchGroup = 4;
constexpr int kDispatchWaves = kDispatchThreads / kWave;

__host__ __device__ constexpr int dispatch_chunks(int n_pairs) { return (n_pairs + kDispatchChunk - 1) / kDispatchChunk; }

// LDS bytes block_dispatch needs for n_pairs pairs: the pairs' experts and
// ranks (uint16 each), per-wave counts and five per-expert arrays.
__host__ __device__ constexpr size_t dispatch_lds_bytes(int n_pairs, int /*n_exp*/) {
  return 2 * (((size_t)n_pairs * sizeof(uint16_t) + 15) / 16 * 16) +
         (kDispatchWaves + 5) * kDispatchMaxExperts * sizeof(int32_t) + 8 * sizeof(int32_t);
}

// Largest n_pairs whose staging fits in 160 KiB of LDS.
constexpr int kDispatchMaxPairs = 38648;
static_assert(dispatch_lds_bytes(kDispatchMaxPairs, kDispatchMaxExperts) <= 160 * 1024, "dispatch LDS");
static_assert(dispatch_lds_bytes(kDispatchMaxPairs + 8, kDispatchMaxExperts) > 160 * 1024, "dispatch LDS");

// For each of N keys (key < 512) held by this lane: the lanes of the wave
// holding the same key, from one ballot per key bit.
template <int N>
__device__ __forceinline__ void wave_peers(const uint32_t (&key)[N], uint64_t (&peers)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) peers[i] = ~0ull;
#pragma unroll
  for (int b = 0; b < 9; ++b) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const bool bit = (key[i] >> b) & 1u;
      const uint64_t m = __ballot(bit);
      peers[i] &= bit ? m : ~m;
    }
  }
}

// Stable counting sort of the pairs by expert, by one 256-thread block, and
// the work-unit lists (klc_common.h).  A pair's position is its expert's
// offset + the pairs of that expert in earlier waves' chunks + its rank in
// its wave's chunks (ballots within a chunk, a per-wave running count across
// chunks), so no step is serial over pairs.  lds holds
// dispatch_lds_bytes(n_pairs, n_exp) bytes.
__device__ void block_dispatch(const int32_t* ids, int n_pairs, int n_exp, int32_t* __restrict__ offsets,
                               int32_t* __restrict__ sorted, int32_t* __restrict__ active,
                               int32_t* __restrict__ n_active, int32_t* __restrict__ units, char* lds) {
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int nchunk = dispatch_chunks(n_pairs);
  const int cpw = (nchunk + kDispatchWaves - 1) / kDispatchWaves;
  const size_t pair_bytes = ((size_t)n_pairs * sizeof(uint16_t) + 15) / 16 * 16;
  uint16_t* sid = reinterpret_cast<uint16_t*>(lds);  // expert of each pair, 0xffff = skip
  uint16_t* rank = reinterpret_cast<uint16_t*>(lds + pair_bytes);
  int32_t* cnt = reinterpret_cast<int32_t*>(lds + 2 * pair_bytes);  // [wave][expert]
  int32_t* total = cnt + kDispatchWaves * kDispatchMaxExperts;
  int32_t* flags = total + kDispatchMaxExperts;
  int32_t* ugu = flags + kDispatchMaxExperts;  // units per expert, then their prefix (gate_up)
  int32_t* udn = ugu + kDispatchMaxExperts;    // same for down
  int32_t* ugm = udn + kDispatchMaxExperts;    // same for the GEMM
  int32_t* sums = ugm + kDispatchMaxExperts;
  const uint64_t below = (1ull << lane) - 1ull;

  for (int i = tid; i < kDispatchWaves * kDispatchMaxExperts; i += kDispatchThreads) cnt[i] = 0;
  for (int p0 = 0; p0 < n_pairs; p0 += 8 * kDispatchThreads) {
    int32_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = ids[min(p0 + j * kDispatchThreads + tid, n_pairs - 1)];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int p = p0 + j * kDispatchThreads + tid;
      if (p < n_pairs) sid[p] = (v[j] >= 0 && v[j] < n_exp) ? (uint16_t)v[j] : (uint16_t)0xffffu;
    }
  }
  __syncthreads();
  // 1. ranks: within a chunk from the ballots, plus the wave's running count
  //    of the expert (read by all its lanes, then advanced by the lowest one;
  //    a wave's LDS accesses complete in program order)
  {
    int32_t* wcnt = cnt + wave * kDispatchMaxExperts;
    const int cend = min((wave + 1) * cpw, nchunk);
    for (int c0 = wave * cpw; c0 < cend; c0 += kDispatchGroup) {
      uint32_t key[kDispatchGroup];
      uint64_t peers[kDispatchGroup];
#pragma unroll
      for (int i = 0; i < kDispatchGroup; ++i) {
        const int p = (c0 + i) * kDispatchChunk + lane;
        const uint32_t e = (c0 + i < cend && p < n_pairs) ? (uint32_t)sid[p] : 0xffffu;
        key[i] = e < (uint32_t)n_exp ? e : 511u;
      }
      wave_peers(key, peers);
#pragma unroll
      for (int i = 0; i < kDispatchGroup; ++i) {
        if (key[i] != 511u) {
          const int32_t before = wcnt[key[i]];
          rank[(c0 + i) * kDispatchChunk + lane] = (uint16_t)(before + __popcll(peers[i] & below));
          if ((peers[i] & below) == 0ull) wcnt[key[i]] = before + __popcll(peers[i]);
        }
        __builtin_amdgcn_wave_barrier();
      }
    }
  }
  __syncthreads();
  // 2. per expert: the waves' counts become their exclusive prefix; totals
  //    and unit counts
  for (int e = tid; e < n_exp; e += kDispatchThreads) {
    int32_t run = 0;
#pragma unroll
    for (int w = 0; w < kDispatchWaves; ++w) {
      const int32_t v = cnt[w * kDispatchMaxExperts + e];
      cnt[w * kDispatchMaxExperts + e] = run;
      run += v;
    }
    total[e] = run;
    flags[e] = run > 0 ? 1 : 0;
    ugu[e] = (run + kUnitTokensGateUp - 1) / kUnitTokensGateUp;
    udn[e] = (run + kUnitTokensDown - 1) / kUnitTokensDown;
    ugm[e] = (run + kUnitTokensGemm - 1) / kUnitTokensGemm;
  }
  __syncthreads();
  // total[] becomes the expert offsets, flags[] the active-list positions,
  // ugu[]/udn[]/ugm[] the first unit of each expert: one wave per array
  if (wave == 0) {
    wave_exclusive_scan_256(total, n_exp, &sums[0], lane);
    wave_exclusive_scan_256(ugm, n_exp, &sums[4], lane);
  } else if (wave == 1) {
    wave_exclusive_scan_256(flags, n_exp, &sums[1], lane);
  } else if (wave == 2) {
    wave_exclusive_scan_256(ugu, n_exp, &sums[2], lane);
  } else {
    wave_exclusive_scan_256(udn, n_exp, &sums[3], lane);
  }
  __syncthreads();
  // 3. scatter
  for (int p = tid; p < n_pairs; p += kDispatchThreads) {
    const uint32_t e = sid[p];
    if (e < (uint32_t)n_exp) {
      const int w = (p / kDispatchChunk) / cpw;
      sorted[total[e] + cnt[w * kDispatchMaxExperts + e] + rank[p]] = p;
    }
  }
  // 4. unit lists, all three as one index space, 4 units per thread at a
  //    time: a unit's expert is the last one whose first unit is <= the
  //    unit (experts without units share the next one's first unit), found
  //    by 8 bisection steps run in lockstep
  {
    const int n_gu = sums[2], n_dn = sums[3], n_all = sums[2] + sums[3] + sums[4];
    int32_t* const gu_list = units + kUnitHeader;
    int32_t* const dn_list = units + units_offset_down(n_pairs, n_exp);
    int32_t* const gm_list = units + units_offset_gemm(n_pairs, n_exp);
    for (int u0 = tid; u0 < n_all; u0 += 4 * kDispatchThreads) {
      int lo[4], uu[4], base[4];
      int32_t* dst[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int u = u0 + i * kDispatchThreads;
        const int l = u < n_gu ? 0 : (u < n_gu + n_dn ? 1 : 2);
        uu[i] = u - (l == 0 ? 0 : (l == 1 ? n_gu : n_gu + n_dn));
        base[i] = l * kDispatchMaxExperts;  // ugu, udn, ugm are consecutive
        dst[i] = l == 0 ? gu_list : (l == 1 ? dn_list : gm_list);
        lo[i] = 0;
      }
#pragma unroll
      for (int step = kDispatchMaxExperts / 2; step >= 1; step >>= 1) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int cand = lo[i] + step;
          const int32_t f = ugu[base[i] + min(cand, n_exp - 1)];
          if (cand < n_exp && f <= uu[i]) lo[i] = cand;
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int u = u0 + i * kDispatchThreads;
        if (u < n_all) dst[i][uu[i]] = make_unit(lo[i], uu[i] - ugu[base[i] + lo[i]]);
      }
    }
    if (tid == 0) {
      units[0] = sums[2];
      units[1] = sums[3];
      units[2] = sums[4];
      units[3] = 0;
    }
  }
  for (int e = tid; e < n_exp; e += kDispatchThreads) {
    offsets[e] = total[e];
    const int next = e + 1 < n_exp ? total[e + 1] : sums[0];
    if (next > total[e]) active[flags[e]] = e;
    if (e >= sums[1]) active[e] = -1;
  }
  if (tid == 0) {
    offsets[n_exp] = sums[0];
    *n_active = sums[1];
  }
}

__global__ __launch_bounds__(kDispatchThreads) void dispatch_kernel(const int32_t* __restrict__ ids, int n_pairs,
                                                                    int n_exp, int32_t* __restrict__ offsets,
                                                                    int32_t* __restrict__ sorted,
                                                                    int32_t* __restrict__ active,
                                                                    int32_t* __restrict__ n_active,
                                                                    int32_t* __restrict__ units) {
  extern __shared__ char dlds[];
  block_dispatch(ids, n_pairs, n_exp, offsets, sorted, active, n_active, units, dlds);
}

// Router for decode batches in one launch: every workgroup computes its
// (4 experts x 8 tokens) logits tile; the last workgroup to finish (counted
// in *done, which it resets to 0) then selects the top-k of every token and
// builds the expert-sorted dispatch.  Release/acquire fences at agent scope
// make the other workgroups' logits visible across XCDs.
__global__ __launch_bounds__(256) void router_fused_kernel(const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ w,
                                                           const uint16_t* __restrict__ b, uint16_t* logits,
                                                           int n_tok, int hidden, int n_exp, int k, int32_t* ids,
                                                           float* __restrict__ values, uint16_t* __restrict__ weights,
                                                           int32_t* __restrict__ offsets, int32_t* __restrict__ sorted,
                                                           int32_t* __restrict__ active,
                                                           int32_t* __restrict__ n_active, int32_t* __restrict__ units,
                                                           uint32_t* done) {
  extern __shared__ char flds[];
  router_logits_tile(x, w, b, logits, nullptr, n_tok, hidden, n_exp, reinterpret_cast<uint16_t*>(flds));
  __shared__ uint32_t last;
  __syncthreads();
  if (threadIdx.x == 0) {
    __threadfence();
    const uint32_t n_blocks = gridDim.x * gridDim.y;
    const uint32_t prev = atomicAdd(done, 1u);
    last = prev == n_blocks - 1 ? 1u : 0u;
    if (last) {
      *done = 0u;  // ready for the next launch
      __threadfence();
    }
  }
  __syncthreads();
  if (!last) return;
  for (int t = threadIdx.x >> 6; t < n_tok; t += 4) {
    const uint16_t* row = logits + (int64_t)t * n_exp;
    topk_softmax_row(row, n_exp, k, t, ids, values, weights);
  }
  __threadfence_block();
  __syncthreads();
  block_dispatch(ids, n_tok * k, n_exp, offsets, sorted, active, n_active, units, flds);
}

}  // namespace

int launch_router_logits(const void* x, const void* w, const void* b, void* logits, float* x_f32, int64_t n_tok,
                         int64_t hidden, int64_t n_exp, hipStream_t stream) {
  const dim3 grid((unsigned)((n_exp + kRouterMfmaRows - 1) / kRouterMfmaRows),
                  (unsigned)((n_tok + kRouterMfmaRows - 1) / kRouterMfmaRows));
  router_logits_mfma_kernel<<<grid, 256, 0, stream>>>(
      static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), static_cast<const uint16_t*>(b),
      static_cast<uint16_t*>(logits), x_f32, (int)n_tok, (int)hidden, (int)n_exp);
  return check_launch("router_logits_mfma_kernel");
}

int launch_topk(const void* logits, int32_t* ids, float* values, void* weights, int64_t n_tok, int64_t n_exp,
                int64_t k, hipStream_t stream) {
  topk_softmax_kernel<<<(unsigned)((n_tok + 3) / 4), 256, 0, stream>>>(
      static_cast<const uint16_t*>(logits), ids, values, static_cast<uint16_t*>(weights), (int)n_tok, (int)n_exp,
      (int)k);
  return check_launch("topk_softmax_kernel");
}

int launch_dispatch(const int32_t* ids, int64_t n_pairs, int64_t n_exp, int32_t* offsets, int32_t* sorted,
                    int32_t* active, int32_t* n_active, int32_t* units, hipStream_t stream) {
  dispatch_kernel<<<1, kDispatchThreads, dispatch_lds_bytes((int)n_pairs, (int)n_exp), stream>>>(
      ids, (int)n_pairs, (int)n_exp, offsets, sorted, active, n_active, units);
  return check_launch("dispatch_kernel");
}

int launch_router_fused(const void* x, const void* w, const void* b, void* logits, int64_t n_tok, int64_t hidden,
                        int64_t n_exp, int64_t k, int32_t* ids, float* values, void* weights, int32_t* offsets,
                        int32_t* sorted, int32_t* active, int32_t* n_active, int32_t* units, uint32_t* done,
                        hipStream_t stream) {
  const dim3 grid((unsigned)((n_exp + 3) / 4), (unsigned)((n_tok + kRouterTok - 1) / kRouterTok));
  const size_t lds_logits = (size_t)kRouterTok * hidden * sizeof(uint16_t);
  const size_t lds_dispatch = dispatch_lds_bytes((int)(n_tok * k), (int)n_exp);
  router_fused_kernel<<<grid, 256, lds_logits > lds_dispatch ? lds_logits : lds_dispatch, stream>>>(
      static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), static_cast<const uint16_t*>(b),
      static_cast<uint16_t*>(logits), (int)n_tok, (int)hidden, (int)n_exp, (int)k, ids, values,
      static_cast<uint16_t*>(weights), offsets, sorted, active, n_active, units, done);
  return check_launch("router_fused_kernel");
}

int check_router_args(int64_t n_tok, int64_t hidden, int64_t n_exp) {
  KLC_REQUIRE(n_tok > 0 && hidden > 0 && n_exp > 0, KLC_ERR_ARGUMENT,
              "router: bad sizes n_tokens=%lld hidden=%lld n_experts=%lld", (long long)n_tok, (long long)hidden,
              (long long)n_exp);
  KLC_REQUIRE(hidden % 8 == 0, KLC_ERR_SHAPE, "router: hidden=%lld must be a multiple of 8", (long long)hidden);
  KLC_REQUIRE(n_tok <= (int64_t)65535 * kRouterTok && hidden <= 64 * 8 * kRouterChunks && n_exp <= 1024,
              KLC_ERR_UNSUPPORTED,
              "router: unsupported sizes n_tokens=%lld hidden=%lld n_experts=%lld (hidden <= %d, n_experts <= 1024)",
              (long long)n_tok, (long long)hidden, (long long)n_exp, 64 * 8 * kRouterChunks);
  return KLC_OK;
}

int check_topk_args(int64_t n_tok, int64_t n_exp, int64_t k) {
  KLC_REQUIRE(n_tok > 0 && n_exp > 0 && k > 0, KLC_ERR_ARGUMENT, "topk: bad sizes n_tokens=%lld n_experts=%lld k=%lld",
              (long long)n_tok, (long long)n_exp, (long long)k);
  KLC_REQUIRE(k <= n_exp, KLC_ERR_SHAPE, "topk: k=%lld exceeds n_experts=%lld", (long long)k, (long long)n_exp);
  KLC_REQUIRE(k <= 32 && n_exp <= 1024 && n_tok < ((int64_t)1 << 31) / 4, KLC_ERR_UNSUPPORTED,
              "topk: unsupported k=%lld n_experts=%lld (k <= 32, n_experts <= 1024)", (long long)k,
              (long long)n_exp);
  return KLC_OK;
}

int check_dispatch_args(int64_t n_pairs, int64_t n_exp) {
  KLC_REQUIRE(n_pairs > 0 && n_exp > 0, KLC_ERR_ARGUMENT, "dispatch: bad sizes n_pairs=%lld n_experts=%lld",
              (long long)n_pairs, (long long)n_exp);
  KLC_REQUIRE(n_exp <= kDispatchMaxExperts, KLC_ERR_UNSUPPORTED, "dispatch: n_experts=%lld > %d", (long long)n_exp,
              kDispatchMaxExperts);
  KLC_REQUIRE(n_pairs <= kDispatchMaxPairs, KLC_ERR_UNSUPPORTED,
              "dispatch: n_pairs=%lld > %d (the pairs' experts and ranks are staged in 160 KiB of LDS)",
              (long long)n_pairs, kDispatchMaxPairs);
  return KLC_OK;
}

}  // namespace klc

using namespace klc;

extern "C" int klc_moe_router_logits(const void* x, const void* w, const void* b, void* logits, float* x_f32,
                                     int64_t n_tokens, int64_t hidden, int64_t n_experts, void* stream) {
  KLC_REQUIRE(x && w && b && logits, KLC_ERR_ARGUMENT, "klc_moe_router_logits: null pointer");
  const int rc = check_router_args(n_tokens, hidden, n_experts);
  if (rc) return rc;
  return launch_router_logits(x, w, b, logits, x_f32, n_tokens, hidden, n_experts, as_stream(stream));
}

extern "C" int klc_moe_topk_softmax(const void* logits, int32_t* ids, float* values, void* weights, int64_t n_tokens,
                                    int64_t n_experts, int64_t k, void* stream) {
  KLC_REQUIRE(logits && ids && weights, KLC_ERR_ARGUMENT, "klc_moe_topk_softmax: null pointer");
  const int rc = check_topk_args(n_tokens, n_experts, k);
  if (rc) return rc;
  return launch_topk(logits, ids, values, weights, n_tokens, n_experts, k, as_stream(stream));
}

extern "C" int klc_moe_softmax_weights(const float* values, void* weights, int64_t n_tokens, int64_t k,
                                       void* stream) {
  KLC_REQUIRE(values && weights, KLC_ERR_ARGUMENT, "klc_moe_softmax_weights: null pointer");
  KLC_REQUIRE(n_tokens > 0 && k > 0 && n_tokens < ((int64_t)1 << 31) && k <= 1024, KLC_ERR_ARGUMENT,
              "klc_moe_softmax_weights: bad sizes n_tokens=%lld k=%lld", (long long)n_tokens, (long long)k);
  softmax_weights_kernel<<<(unsigned)((n_tokens + 255) / 256), 256, 0, as_stream(stream)>>>(
      values, static_cast<uint16_t*>(weights), (int)n_tokens, (int)k);
  return check_launch("softmax_weights_kernel");
}

extern "C" int klc_moe_dispatch(const int32_t* ids, int64_t n_pairs, int64_t n_experts, int32_t* offsets,
                                int32_t* sorted_pairs, int32_t* active, int32_t* n_active, int32_t* units,
                                void* stream) {
  KLC_REQUIRE(ids && offsets && sorted_pairs && active && n_active && units, KLC_ERR_ARGUMENT,
              "klc_moe_dispatch: null pointer");
  const int rc = check_dispatch_args(n_pairs, n_experts);
  if (rc) return rc;
  return launch_dispatch(ids, n_pairs, n_experts, offsets, sorted_pairs, active, n_active, units,
                         as_stream(stream));
}

extern "C" int64_t klc_moe_units_size(int64_t n_pairs, int64_t n_experts) {
  const int rc = check_dispatch_args(n_pairs, n_experts);
  if (rc) return rc;
  return units_size(n_pairs, n_experts);
}
