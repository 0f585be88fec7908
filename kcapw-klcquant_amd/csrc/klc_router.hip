// Router logits, top-k + softmax, and expert-sorted dispatch (gfx950).
//
// Logits: float64 MFMA tiles of 16 experts x 16 tokens.  Each bfloat16
// product is exact in float64 and the sums are float64, so the only roundings
// are the reference's own: float32 of the dot product, float32 bias add,
// bfloat16 result (streamed_moe_router.py:269).
//
// Top-k: one wave per token.  Each logit becomes a 64-bit key (ordered value
// bits, then inverted expert index), so a wave-wide max picks the largest
// value and, among equal values, the lowest expert index; k rounds of that
// give the descending top-k.  The softmax over the k values is evaluated in
// float64 and rounded to float32, then to bfloat16.
//
// Dispatch: one workgroup performs a stable counting sort of the (token, slot)
// pairs by expert: ranks from wave ballots and per-wave running counts, a
// per-expert prefix over the waves, then a scatter.
//
// Decode batches run all three in one launch (router_decode_kernel): the
// logits tiles are split along the hidden dimension over many workgroups and
// the last workgroup to finish each step (counted in self-resetting
// counters) goes on to the next one.
#include "klc_router_dev.h"

namespace klc {
namespace {

__global__ __launch_bounds__(256) void router_logits_mfma_kernel(const uint16_t* __restrict__ x,
                                                                 const uint16_t* __restrict__ w,
                                                                 const uint16_t* __restrict__ b,
                                                                 uint16_t* __restrict__ logits,
                                                                 float* __restrict__ x_f32, int n_tok, int hidden,
                                                                 int n_exp) {
  __shared__ double red[3 * 64 * 4];
  const int e0 = blockIdx.x * kRouterTile;
  const int t0 = blockIdx.y * kRouterTile;
  // the tile's biases first (branch-free: out-of-range experts read 0), so
  // they arrive with the weights instead of after the dot product
  const __amdgpu_buffer_rsrc_t bbuf = bias_rsrc(b, n_exp);
  float bias4[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) bias4[i] = load_bias_f32(bbuf, e0 + ((threadIdx.x & 63) >> 4) + 4 * i);
  const f64x4_t acc = router_block_dot(x, w, n_tok, hidden, n_exp, e0, t0, 0, (hidden + 31) >> 5,
                                       blockIdx.x == 0 ? x_f32 : nullptr, red);
  if (threadIdx.x < kWave) router_tile_store(acc, bias4, logits, n_tok, n_exp, e0, t0);
}

__global__ __launch_bounds__(256) void topk_softmax_kernel(const uint16_t* __restrict__ logits,
                                                           int32_t* __restrict__ ids, float* __restrict__ values,
                                                           uint16_t* __restrict__ weights, int n_tok, int n_exp,
                                                           int k, int32_t* host_ids, uint16_t* host_weights) {
  extern __shared__ __align__(16) char lds[];  // topk_tie_scratch_bytes(n_exp) per wave
  __shared__ int tie_list[17];
  const int wave = threadIdx.x >> 6;
  const int64_t t_base = (int64_t)blockIdx.x * 16;  // 16 tokens per workgroup
  uint32_t* tie_scratch = reinterpret_cast<uint32_t*>(lds + wave * topk_tie_scratch_bytes(n_exp));
  const SelectionOut sel{ids, values, weights, nullptr, host_ids, host_weights};
  topk_softmax_block([&](int t) { return logits + (t_base + t) * n_exp; }, (int)min<int64_t>(16, n_tok - t_base),
                     n_exp, k, t_base, sel, tie_scratch, tie_list);
}

// Softmax of caller-chosen scores (one thread per token), as torch's CPU
// softmax computes it (klc_torch_order.h): the routing-locality path picks
// the experts on the host and hands over their float32 scores in slot order.
__global__ __launch_bounds__(256) void softmax_weights_kernel(const float* __restrict__ values,
                                                              uint16_t* __restrict__ weights, int n_tok, int k) {
#pragma clang fp contract(off)
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_tok) return;
  const float* v = values + (int64_t)t * k;
  float mx = v[0];
  for (int r = 1; r < k; ++r) mx = torch_vec_max(mx, v[r]);
  float sum = sleef_expf_u10(v[0] - mx);
  for (int r = 1; r < k; ++r) sum = sum + sleef_expf_u10(v[r] - mx);
  const float inv = 1.0f / sum;
  for (int r = 0; r < k; ++r)
    weights[(int64_t)t * k + r] = (uint16_t)f32_to_bf16_rne(sleef_expf_u10(v[r] - mx) * inv);
}

__global__ __launch_bounds__(kDispatchThreads) void dispatch_kernel(const int32_t* __restrict__ ids, int n_pairs,
                                                                    int n_exp, int32_t* __restrict__ offsets,
                                                                    int32_t* __restrict__ sorted,
                                                                    int32_t* __restrict__ active,
                                                                    int32_t* __restrict__ n_active,
                                                                    int32_t* __restrict__ units) {
  extern __shared__ __align__(16) char dlds[];
  block_dispatch([&](int p) { return ids[p]; }, n_pairs, n_exp, offsets, sorted, active, n_active, units, dlds);
}

// The same dispatch (block_dispatch's outputs) over one workgroup per
// expert, for large batches.  Every workgroup reads all pair ids (from L2
// after the first) and counts every expert's pairs in LDS, so it knows all
// offsets, active-list positions and unit prefixes without a hand-off
// between workgroups; it then writes its own expert's pairs in pair order,
// offset, active-list entries and units.  Wave w takes the pairs
// [w Q, (w + 1) Q), Q = ceil(n_pairs / 4), 64 consecutive pairs per
// coalesced load and 8 loads in flight: a first pass counts (LDS atomics
// for the histogram, a ballot for the own expert), a second pass places the
// own expert's pairs at its offset + the earlier waves' count + the wave's
// running count + the rank within the 64.
constexpr int kDispatchMultiBatch = 8;
__global__ __launch_bounds__(kDispatchThreads) void dispatch_multi_kernel(const int32_t* __restrict__ ids, int n_pairs,
                                                                          int n_exp, int32_t* __restrict__ offsets,
                                                                          int32_t* __restrict__ sorted,
                                                                          int32_t* __restrict__ active,
                                                                          int32_t* __restrict__ n_active,
                                                                          int32_t* __restrict__ units) {
  __shared__ int32_t hist[kDispatchMaxExperts];  // counts, then offsets
  __shared__ int32_t flags[kDispatchMaxExperts];  // active, then active-list positions
  __shared__ int32_t ucnt[3][kDispatchMaxExperts];  // units per expert, then first unit (gate_up, down, GEMM)
  __shared__ int32_t sums[8];
  __shared__ int32_t wave_own[kDispatchWaves];
  const int own = blockIdx.x;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const uint64_t below = (1ull << lane) - 1ull;
  for (int e = tid; e < kDispatchMaxExperts; e += kDispatchThreads) hist[e] = 0;
  lds_barrier();
  const int q = (n_pairs + kDispatchWaves - 1) / kDispatchWaves;
  const int w0 = min(wave * q, n_pairs), w1 = min(w0 + q, n_pairs);
  // pass 1: histogram and the wave's count of the own expert
  int own_count = 0;
  for (int b = w0; b < w1; b += kDispatchMultiBatch * kWave) {
    int32_t v[kDispatchMultiBatch];
#pragma unroll
    for (int i = 0; i < kDispatchMultiBatch; ++i) {
      const int p = b + i * kWave + lane;
      v[i] = p < w1 ? ids[p] : -1;
    }
#pragma unroll
    for (int i = 0; i < kDispatchMultiBatch; ++i) {
      const bool valid = v[i] >= 0 && v[i] < n_exp;
      if (valid) atomicAdd(&hist[v[i]], 1);
      own_count += __popcll(__ballot(v[i] == own));
    }
  }
  if (lane == 0) wave_own[wave] = own_count;
  lds_barrier();
  const int32_t own_total = hist[own];  // read before the scan below turns counts into offsets
  for (int e = tid; e < n_exp; e += kDispatchThreads) {
    const int32_t c = hist[e];
    flags[e] = c > 0 ? 1 : 0;
    ucnt[0][e] = (c + kUnitTokensGateUp - 1) / kUnitTokensGateUp;
    ucnt[1][e] = (c + kUnitTokensDown - 1) / kUnitTokensDown;
    ucnt[2][e] = (c + kUnitTokensGemm - 1) / kUnitTokensGemm;
  }
  lds_barrier();
  if (wave == 0) {
    wave_exclusive_scan_256(hist, n_exp, &sums[0], lane);
    wave_exclusive_scan_256(ucnt[2], n_exp, &sums[4], lane);
  } else if (wave == 1) {
    wave_exclusive_scan_256(flags, n_exp, &sums[1], lane);
  } else if (wave == 2) {
    wave_exclusive_scan_256(ucnt[0], n_exp, &sums[2], lane);
  } else {
    wave_exclusive_scan_256(ucnt[1], n_exp, &sums[3], lane);
  }
  lds_barrier();
  // pass 2: the own expert's pairs
  if (own_total > 0) {
    int run = hist[own];
    for (int w = 0; w < wave; ++w) run += wave_own[w];
    for (int b = w0; b < w1; b += kDispatchMultiBatch * kWave) {
      int32_t v[kDispatchMultiBatch];
#pragma unroll
      for (int i = 0; i < kDispatchMultiBatch; ++i) {
        const int p = b + i * kWave + lane;
        v[i] = p < w1 ? ids[p] : -1;
      }
#pragma unroll
      for (int i = 0; i < kDispatchMultiBatch; ++i) {
        const uint64_t m = __ballot(v[i] == own);
        if (v[i] == own) sorted[run + __popcll(m & below)] = b + i * kWave + lane;
        run += __popcll(m);
      }
    }
  }
  // the own expert's offset, active-list entries and units
  int32_t* const gu_list = units + kUnitHeader;
  int32_t* const dn_list = units + units_offset_down(n_pairs, n_exp);
  int32_t* const gm_list = units + units_offset_gemm(n_pairs, n_exp);
  for (int j = tid; j * kUnitTokensGateUp < own_total; j += kDispatchThreads) gu_list[ucnt[0][own] + j] = make_unit(own, j);
  for (int j = tid; j * kUnitTokensDown < own_total; j += kDispatchThreads) dn_list[ucnt[1][own] + j] = make_unit(own, j);
  for (int j = tid; j * kUnitTokensGemm < own_total; j += kDispatchThreads) gm_list[ucnt[2][own] + j] = make_unit(own, j);
  if (tid == 0) {
    offsets[own] = hist[own];
    if (own_total > 0) active[flags[own]] = own;
    if (own >= sums[1]) active[own] = -1;
    if (own == 0) {
      offsets[n_exp] = sums[0];
      *n_active = sums[1];
      units[0] = sums[2];
      units[1] = sums[3];
      units[2] = sums[4];
      units[3] = 0;
    }
  }
}

// Router of a decode batch in one launch.  Workgroup (et, tt, ks) computes
// the partial logits of the tile (experts 16 et.., tokens 16 tt..) over the
// ks-th of gridDim.z slices of the hidden dimension and stores them.  The
// last of a token tile's workgroups to arrive (counted in a self-resetting
// counter) sums every expert tile's slices in slice order (a fixed order, so
// the result does not depend on which workgroup is last), rounds the logits,
// and selects the top-k + softmax of the tile's tokens from an LDS copy.
// With one token tile it then builds the expert-sorted dispatch itself;
// otherwise the last token tile to finish does.  With units == nullptr the
// launch routes only (ids, values, weights, logits) and builds no dispatch.
// counters: [n_tt] token-tile counters and 1 final counter, zero before the
// first launch and left zero by every launch.  partials: [n_tt][n_et]
// [gridDim.z][256] float64.  host_ids / host_weights (optional): copies of
// the selection in a host record (SelectionOut); with one token, host_tag
// (optional) then receives tag_value once they are in host memory.
// kCls: router_expert_class(n_exp, k), or 0 for any expert count.  kOne:
// router_decode_one_wave(n_tok, n_exp) -- the one-token kernel holds only
// the one-wave selection and the multi-token kernel only the workgroup
// selection and dispatches (a shorter kernel starts its workgroups sooner:
// 3,551 against 12,055 instructions for 128 experts, k = 4).
template <int kCls, bool kOne>
__global__ __launch_bounds__(256) void router_decode_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, const uint16_t* __restrict__ b, uint16_t* logits,
    int n_tok, int hidden, int n_exp, int k, int32_t* ids, float* values, uint16_t* weights,
    int32_t* __restrict__ offsets, int32_t* __restrict__ sorted, int32_t* __restrict__ active,
    int32_t* __restrict__ n_active, int32_t* __restrict__ units, uint32_t* counters, double* partials,
    int32_t* host_ids, uint16_t* host_weights, uint32_t* host_tag, uint32_t tag_value) {
  // wave sums (float64); then the token tile's logits; then the dispatch's
  // staging.  16-byte aligned: the static flag below comes first in LDS.
  extern __shared__ __align__(16) char lds[];
  __shared__ uint32_t flag;
  __shared__ int32_t tile_ids[kRouterTile * kRouterMaxK];  // one token tile's ids, for its own dispatch
  __shared__ int tie_list[17];  // the tile's rows with ties, and their count
  const int et = blockIdx.x, tt = blockIdx.y, ks = blockIdx.z;
  const int n_et = gridDim.x, n_tt = gridDim.y, n_ks = gridDim.z;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int t0 = tt * kRouterTile;
  const int nchunk = (hidden + 31) >> 5;
  const int per_slice = (nchunk + n_ks - 1) / n_ks;
  const int cb = min(ks * per_slice, nchunk);
  const int ce = min(cb + per_slice, nchunk);
  const f64x4_t part =
      router_block_dot(x, w, n_tok, hidden, n_exp, et * kRouterTile, t0, cb, ce, nullptr, reinterpret_cast<double*>(lds));
  // [n_et][n_ks][64 lanes][4] float64; lane l holds token t0 + l % 16, so
  // only lanes of the tile's real tokens store and read their partials
  double* tile_parts = partials + (int64_t)tt * n_et * n_ks * 256;
  const __amdgpu_buffer_rsrc_t pbuf = __builtin_amdgcn_make_buffer_rsrc(
      tile_parts, (short)0, (int)(n_et * n_ks * 256 * sizeof(double)), kBufferWord3);
  const bool real_tok = t0 + (lane & 15) < n_tok;
  if (threadIdx.x < kWave && real_tok) {
    const uint32_t off = (uint32_t)(((et * n_ks + ks) * 256 + lane * 4) * sizeof(double));
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, make_double2(part[0], part[1])), pbuf, off, 0,
                                           kAgentScope);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, make_double2(part[2], part[3])), pbuf, off,
                                           16, kAgentScope);
  }
  if (!arrive_last(counters + tt, (uint32_t)(n_et * n_ks), &flag)) return;
  uint16_t* rows = reinterpret_cast<uint16_t*>(lds);  // [16][n_exp]
  // sums: wave w takes expert tiles w, w + 4, w + 8, ..., two per pass with
  // both tiles' loads in flight before the first is summed
  const __amdgpu_buffer_rsrc_t bbuf = bias_rsrc(b, n_exp);
  for (int e_t = wave; e_t < n_et; e_t += 8) {
    if (!real_tok) continue;
    const bool second = e_t + 4 < n_et;
    // the bias loads go first: they are independent of the partials, and
    // branch-free (a branch around each would wait for it before the next)
    float bias4[2][4];
    u32x4_t v[2][2 * kRouterMaxSlices];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int et_h = h == 1 && second ? e_t + 4 : e_t;  // a missing second tile reloads the first
#pragma unroll
      for (int i = 0; i < 4; ++i) bias4[h][i] = load_bias_f32(bbuf, et_h * kRouterTile + (lane >> 4) + 4 * i);
#pragma unroll
      for (int q = 0; q < kRouterMaxSlices; ++q) {
        const int qq = min(q, n_ks - 1);
        const uint32_t off = (uint32_t)(((et_h * n_ks + qq) * 256 + lane * 4) * sizeof(double));
        v[h][2 * q] = __builtin_amdgcn_raw_buffer_load_b128(pbuf, off, 0, kAgentScope);
        v[h][2 * q + 1] = __builtin_amdgcn_raw_buffer_load_b128(pbuf, off, 16, kAgentScope);
      }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (h == 1 && !second) break;
      f64x4_t acc = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
      for (int q = 0; q < kRouterMaxSlices; ++q) {
        if (q < n_ks) {
          const double2 lo = __builtin_bit_cast(double2, v[h][2 * q]);
          const double2 hi = __builtin_bit_cast(double2, v[h][2 * q + 1]);
          acc[0] += lo.x;
          acc[1] += lo.y;
          acc[2] += hi.x;
          acc[3] += hi.y;
        }
      }
      router_tile_store(acc, bias4[h], logits, n_tok, n_exp, (e_t + 4 * h) * kRouterTile, t0, rows);
    }
  }
  lds_barrier();  // the rows are in LDS; the logits' global stores need not have completed
  if constexpr (kOne) {
    // One token: its k experts are distinct, so the dispatch reduces to
    // ranking them; one wave does the top-k and the whole dispatch with no
    // workgroup barrier (the block form below pays one per step).
    if (wave != 0) return;
    uint32_t* tie_scratch = reinterpret_cast<uint32_t*>(lds + decode_rows_bytes(n_exp));
    topk_softmax_row<kCls>(rows, n_exp, k, 0, SelectionOut{ids, values, weights, tile_ids, host_ids, host_weights},
                           tie_scratch);
    // the selection's host stores are fenced (SelectionOut::put, lanes < k of this wave): the tag follows
    if (host_tag != nullptr && lane == 0)
      __hip_atomic_store(host_tag, tag_value, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    wave_lds_sync();
    if (units != nullptr) single_token_dispatch(tile_ids, n_exp, k, offsets, sorted, active, n_active, units);
    return;
  } else {
    // each wave's tie scratch follows the 16 logits rows
    uint32_t* tie_scratch = reinterpret_cast<uint32_t*>(lds + decode_rows_bytes(n_exp) +
                                                        wave * topk_tie_scratch_bytes(n_exp));
    const SelectionOut sel{ids, values, weights, n_tt == 1 ? tile_ids : nullptr, host_ids, host_weights};
    topk_softmax_block<kCls>([&](int t) { return rows + t * n_exp; }, min(kRouterTile, n_tok - t0), n_exp, k, t0,
                             sel, tie_scratch, tie_list);
    if (units == nullptr) return;  // routing only: no dispatch
    if (n_tt > 1) {
      if (!arrive_last(counters + n_tt, (uint32_t)n_tt, &flag)) return;
      block_dispatch([&](int p) { return __hip_atomic_load(ids + p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); },
                     n_tok * k, n_exp, offsets, sorted, active, n_active, units, lds);
    } else if (n_tok * k <= kWave && n_exp <= kDispatchMaxExperts) {
      // one token tile of at most 64 pairs: one wave dispatches from the ids in LDS
      lds_barrier();  // every wave is done with the logits rows, whose LDS the dispatch reuses
      if (wave != 0) return;
      wave_dispatch(tile_ids, n_tok * k, n_exp, offsets, sorted, active, n_active, units,
                    reinterpret_cast<int32_t*>(lds));
    } else {
      // one token tile: its ids are still in LDS
      lds_barrier();
      block_dispatch([&](int p) { return tile_ids[p]; }, n_tok * k, n_exp, offsets, sorted, active, n_active, units,
                     lds);
    }
  }
}

}  // namespace

int launch_router_logits(const void* x, const void* w, const void* b, void* logits, float* x_f32, int64_t n_tok,
                         int64_t hidden, int64_t n_exp, hipStream_t stream) {
  const dim3 grid((unsigned)((n_exp + kRouterTile - 1) / kRouterTile), (unsigned)((n_tok + kRouterTile - 1) / kRouterTile));
  router_logits_mfma_kernel<<<grid, 256, 0, stream>>>(
      static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), static_cast<const uint16_t*>(b),
      static_cast<uint16_t*>(logits), x_f32, (int)n_tok, (int)hidden, (int)n_exp);
  return check_launch("router_logits_mfma_kernel");
}

int launch_topk(const void* logits, int32_t* ids, float* values, void* weights, int64_t n_tok, int64_t n_exp,
                int64_t k, hipStream_t stream, int32_t* host_ids, void* host_weights) {
  topk_softmax_kernel<<<(unsigned)((n_tok + 15) / 16), 256, 4 * topk_tie_scratch_bytes((int)n_exp), stream>>>(
      static_cast<const uint16_t*>(logits), ids, values, static_cast<uint16_t*>(weights), (int)n_tok, (int)n_exp,
      (int)k, host_ids, static_cast<uint16_t*>(host_weights));
  return check_launch("topk_softmax_kernel");
}

// Pairs at and above which the dispatch runs over one workgroup per expert
// (below, block_dispatch's LDS staging holds them: 1024 < kDispatchLdsMaxPairs).
constexpr int kDispatchMultiPairs = 1024;
static_assert(kDispatchMultiPairs <= kDispatchLdsMaxPairs, "the one-workgroup dispatch stages its pairs in LDS");

int launch_dispatch(const int32_t* ids, int64_t n_pairs, int64_t n_exp, int32_t* offsets, int32_t* sorted,
                    int32_t* active, int32_t* n_active, int32_t* units, hipStream_t stream) {
  if (n_pairs >= kDispatchMultiPairs) {
    dispatch_multi_kernel<<<(unsigned)n_exp, kDispatchThreads, 0, stream>>>(ids, (int)n_pairs, (int)n_exp, offsets,
                                                                           sorted, active, n_active, units);
    return check_launch("dispatch_multi_kernel");
  }
  dispatch_kernel<<<1, kDispatchThreads, dispatch_lds_bytes((int)n_pairs, (int)n_exp), stream>>>(
      ids, (int)n_pairs, (int)n_exp, offsets, sorted, active, n_active, units);
  return check_launch("dispatch_kernel");
}

// Slices of the hidden dimension for the decode router: about 128
// workgroups, at most kRouterMaxSlices slices (the last workgroup of a token
// tile reads every slice of its expert tiles).
int64_t decode_router_slices(int64_t n_tok, int64_t hidden, int64_t n_exp) {
  const int64_t tiles = ((n_exp + kRouterTile - 1) / kRouterTile) * ((n_tok + kRouterTile - 1) / kRouterTile);
  const int64_t nchunk = (hidden + 31) / 32;
  int64_t ks = (kDecodeRouterWorkgroups + tiles - 1) / tiles;
  ks = ks < kRouterMaxSlices ? ks : kRouterMaxSlices;
  ks = ks < nchunk ? ks : nchunk;
  return ks > 1 ? ks : 1;
}

int64_t decode_router_counters(int64_t n_tok, int64_t /*n_exp*/) { return (n_tok + kRouterTile - 1) / kRouterTile + 1; }

int64_t decode_router_partial_bytes(int64_t n_tok, int64_t hidden, int64_t n_exp) {
  const int64_t tiles = ((n_exp + kRouterTile - 1) / kRouterTile) * ((n_tok + kRouterTile - 1) / kRouterTile);
  return tiles * decode_router_slices(n_tok, hidden, n_exp) * 256 * (int64_t)sizeof(double);
}

int launch_router_decode(const void* x, const void* w, const void* b, void* logits, int64_t n_tok, int64_t hidden,
                         int64_t n_exp, int64_t k, int32_t* ids, float* values, void* weights, int32_t* offsets,
                         int32_t* sorted, int32_t* active, int32_t* n_active, int32_t* units, uint32_t* counters,
                         double* partials, hipStream_t stream, int32_t* host_ids, void* host_weights,
                         uint32_t* host_tag, uint32_t tag_value) {
  const dim3 grid((unsigned)((n_exp + kRouterTile - 1) / kRouterTile), (unsigned)((n_tok + kRouterTile - 1) / kRouterTile),
                  (unsigned)decode_router_slices(n_tok, hidden, n_exp));
  size_t lds = 3 * 64 * 4 * sizeof(double);
  lds = std::max(lds, decode_rows_bytes((int)n_exp) + 4 * topk_tie_scratch_bytes((int)n_exp));
  lds = std::max(lds, dispatch_lds_bytes((int)(n_tok * k), (int)n_exp));
  const bool one = router_decode_one_wave(n_tok, n_exp);
  auto kernel = one ? router_decode_kernel<0, true> : router_decode_kernel<0, false>;
  switch (router_expert_class(n_exp, k)) {
    case 1: kernel = one ? router_decode_kernel<1, true> : router_decode_kernel<1, false>; break;
    case 2: kernel = one ? router_decode_kernel<2, true> : router_decode_kernel<2, false>; break;
    case 4: kernel = one ? router_decode_kernel<4, true> : router_decode_kernel<4, false>; break;
    default: break;
  }
  kernel<<<grid, 256, lds, stream>>>(
      static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), static_cast<const uint16_t*>(b),
      static_cast<uint16_t*>(logits), (int)n_tok, (int)hidden, (int)n_exp, (int)k, ids, values,
      static_cast<uint16_t*>(weights), offsets, sorted, active, n_active, units, counters, partials, host_ids,
      static_cast<uint16_t*>(host_weights), router_decode_one_wave(n_tok, n_exp) ? host_tag : nullptr, tag_value);
  return check_launch("router_decode_kernel");
}

int check_router_args(int64_t n_tok, int64_t hidden, int64_t n_exp) {
  KLC_REQUIRE(n_tok > 0 && hidden > 0 && n_exp > 0, KLC_ERR_ARGUMENT,
              "router: bad sizes n_tokens=%lld hidden=%lld n_experts=%lld", (long long)n_tok, (long long)hidden,
              (long long)n_exp);
  KLC_REQUIRE(hidden % 8 == 0, KLC_ERR_SHAPE, "router: hidden=%lld must be a multiple of 8", (long long)hidden);
  KLC_REQUIRE(n_tok <= (int64_t)65535 * kRouterTile && hidden <= (1 << 20) && n_exp <= 1024, KLC_ERR_UNSUPPORTED,
              "router: unsupported sizes n_tokens=%lld hidden=%lld n_experts=%lld (n_tokens <= %d, hidden <= "
              "1048576, n_experts <= 1024)", (long long)n_tok, (long long)hidden, (long long)n_exp, 65535 * kRouterTile);
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
  KLC_REQUIRE(n_pairs <= KLC_DISPATCH_MAX_PAIRS, KLC_ERR_UNSUPPORTED, "dispatch: n_pairs=%lld > %d",
              (long long)n_pairs, KLC_DISPATCH_MAX_PAIRS);
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
  return launch_topk(logits, ids, values, weights, n_tokens, n_experts, k, as_stream(stream), nullptr, nullptr);
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
