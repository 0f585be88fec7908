// Device helpers of the router: float64 MFMA logits tiles, torch-order
// top-k + softmax, the expert-sorted dispatch, and the workgroup hand-offs
// of the one-launch decode router (gfx950).  Included by klc_router.hip
// (kernels and launchers) and klc_decode.hip (the fused decode layer).
#pragma once

#include <algorithm>

#include "klc_common.h"
#include "klc_torch_order.h"

namespace klc {
namespace {
constexpr int kRouterTile = 16;    // experts and tokens per logits tile
constexpr int kRouterDepth = 4;    // 32-deep chunks per lane in flight
constexpr int kRouterMaxSlices = 8;  // hidden-dimension slices of the decode router
constexpr int kRouterMaxK = 32;      // experts per token (checked on the host)
#ifndef KLC_DECODE_ROUTER_WORKGROUPS
#define KLC_DECODE_ROUTER_WORKGROUPS 128
#endif
constexpr int kDecodeRouterWorkgroups = KLC_DECODE_ROUTER_WORKGROUPS;  // target grid size of the decode router
typedef double f64x4_t __attribute__((ext_vector_type(4)));

// Partial logits of the tile (experts e0.., tokens t0..) over the 32-deep
// hidden chunks [c_begin, c_end), by the 4 waves of the workgroup, each on a
// quarter of the range.  Per chunk lane l holds 8 consecutive weights of
// expert row l % 16 and 8 hidden values of token l % 16 (k = 32 c + 8 (l / 16)
// + i), converted to float64, and issues 8 v_mfma_f64_16x16x4_f64 (A lane l
// = row l % 16, k = l / 16; B lane l = column l % 16, same k; D lane l
// register i = row l / 16 + 4 i, column l % 16) on two accumulators.  The
// rows are read as raw buffers (the tile's rows, the chunk in the uniform
// offset): chunks or rows outside the matrices load zeros without a branch,
// so the loads of the next kRouterDepth chunks stay in flight while the
// current ones multiply.  The waves' sums are added through LDS in wave
// order; the result is valid in wave 0.  x_f32, when given, receives the
// float32 copy of the hidden rows the tile reads.
__device__ __forceinline__ f64x4_t router_block_dot(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, int n_tok,
                                    int hidden, int n_exp, int e0, int t0, int c_begin, int c_end,
                                    float* __restrict__ x_f32, double* red /* LDS [3][64][4] */) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int per = (c_end - c_begin + 3) >> 2;
  const int c0 = min(c_begin + wave * per, c_end);
  const int c1 = min(c0 + per, c_end);
  const int tok = t0 + r;
  const int row_bytes = hidden * 2;
  const __amdgpu_buffer_rsrc_t wbuf = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(w + (int64_t)e0 * hidden), (short)0, min(kRouterTile, n_exp - e0) * row_bytes, kBufferWord3);
  const __amdgpu_buffer_rsrc_t xbuf = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(x + (int64_t)t0 * hidden), (short)0, min(kRouterTile, n_tok - t0) * row_bytes, kBufferWord3);
  const uint32_t lane_off = (uint32_t)(r * row_bytes + g * 16);
  const bool w_ok = e0 + r < n_exp;
  const bool x_ok = tok < n_tok;
  f64x4_t acc0 = {0.0, 0.0, 0.0, 0.0}, acc1 = {0.0, 0.0, 0.0, 0.0};
  auto load = [&](int c, u32x4_t (&wv)[kRouterDepth], u32x4_t (&xv)[kRouterDepth]) {
#pragma unroll
    for (int i = 0; i < kRouterDepth; ++i) {
      // hidden % 8 == 0: a lane's 8 values are all inside the row or all past it
      const bool ok = c + i < c1 && (c + i) * 32 + g * 8 < hidden;
      wv[i] = __builtin_amdgcn_raw_buffer_load_b128(wbuf, ok && w_ok ? lane_off : kOutOfRange, (c + i) * 64, 0);
      xv[i] = __builtin_amdgcn_raw_buffer_load_b128(xbuf, ok && x_ok ? lane_off : kOutOfRange, (c + i) * 64, 0);
    }
  };
  u32x4_t wa[kRouterDepth], xa[kRouterDepth];
  load(c0, wa, xa);
  for (int c = c0; c < c1; c += kRouterDepth) {
    u32x4_t wb[kRouterDepth], xb[kRouterDepth];
    load(c + kRouterDepth, wb, xb);
#pragma unroll
    for (int i = 0; i < kRouterDepth; ++i) {
      if (x_f32 != nullptr && x_ok && c + i < c1 && (c + i) * 32 + g * 8 < hidden) {
        float4* dst = reinterpret_cast<float4*>(x_f32 + (int64_t)tok * hidden + (c + i) * 32 + g * 8);
        dst[0] = make_float4(__uint_as_float(xa[i].x << 16), __uint_as_float(xa[i].x & 0xffff0000u),
                             __uint_as_float(xa[i].y << 16), __uint_as_float(xa[i].y & 0xffff0000u));
        dst[1] = make_float4(__uint_as_float(xa[i].z << 16), __uint_as_float(xa[i].z & 0xffff0000u),
                             __uint_as_float(xa[i].w << 16), __uint_as_float(xa[i].w & 0xffff0000u));
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc0 = __builtin_amdgcn_mfma_f64_16x16x4f64((double)__uint_as_float(wa[i][q] << 16),
                                                     (double)__uint_as_float(xa[i][q] << 16), acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f64_16x16x4f64((double)__uint_as_float(wa[i][q] & 0xffff0000u),
                                                     (double)__uint_as_float(xa[i][q] & 0xffff0000u), acc1, 0, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < kRouterDepth; ++i) {
      wa[i] = wb[i];
      xa[i] = xb[i];
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
  }
  return acc;
}

// The router bias as a raw buffer of n_exp bfloat16 values.  load_bias_f32
// reads expert e's as float32 and 0 for e >= n_exp (out of range: no memory
// access), with no branch, so a tile's bias loads all go out together.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t bias_rsrc(const uint16_t* b, int n_exp) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)b, (short)0, n_exp * 2, kBufferWord3);
}
__device__ __forceinline__ float load_bias_f32(__amdgpu_buffer_rsrc_t bbuf, int e) {
  return bf16_to_f32((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(bbuf, (uint32_t)e * 2u, 0, 0));
}

// The calling wave rounds a tile's sums (its lanes holding them in the MFMA
// D layout) like F.linear in bfloat16: bf16(f32(sum) + b).  Optionally also
// into an LDS copy [16 tokens][n_exp] of the token tile's logits.
__device__ __forceinline__ void router_tile_store(f64x4_t acc, const float (&bias4)[4], uint16_t* logits, int n_tok,
                                                  int n_exp, int e0, int t0, uint16_t* lds_rows = nullptr) {
  const int lane = threadIdx.x & 63;
  const int tok = t0 + (lane & 15);
  if (tok >= n_tok) return;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = e0 + (lane >> 4) + 4 * i;
    if (e < n_exp) {
      const uint16_t v = (uint16_t)f32_to_bf16_rne((float)acc[i] + bias4[i]);
      logits[(int64_t)tok * n_exp + e] = v;
      if (lds_rows != nullptr) lds_rows[(lane & 15) * n_exp + e] = v;
    }
  }
}

// Selection key of a bfloat16 logit: its comparator key (order_key16: NaN
// largest, -0 == +0) above the inverted expert index, so the maximum of the
// keys is the largest value and, among equal values, the lower expert; 0 is
// below every real key.
__device__ __forceinline__ uint32_t sel_key(uint32_t bf16bits, int idx) {
  return (order_key16(bf16bits) << 16) | (uint32_t)(0xffff - idx);
}

constexpr int kTopkMaxPerLane = 16;  // n_experts <= 1024

// Cross-lane steps on the DPP network (VALU, no LDS round trip).  Lanes whose
// source is outside the row or masked off keep `old`.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t old, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, kCtrl, kRowMask, 0xf, false);
}
template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint32_t dpp_max_u32(uint32_t v) {
  const uint32_t o = dpp_u32<kCtrl, kRowMask>(v, v);
  return o > v ? o : v;
}

// Maximum of a 32-bit key over each 16-lane row, in every lane of the row:
// quad swaps, then half-row and row mirrors.
__device__ __forceinline__ uint32_t row_max_u32(uint32_t v) {
  v = dpp_max_u32<0xB1, 0xf>(v);   // quad_perm [1, 0, 3, 2]
  v = dpp_max_u32<0x4E, 0xf>(v);   // quad_perm [2, 3, 0, 1]
  v = dpp_max_u32<0x141, 0xf>(v);  // row_half_mirror
  return dpp_max_u32<0x140, 0xf>(v);  // row_mirror
}

// Wave-wide maximum of a 32-bit key, uniform: the row maxima, two row
// broadcasts carry them into row 3, and lane 63 is read back.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = row_max_u32(v);
  v = dpp_max_u32<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
  v = dpp_max_u32<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Lane r of the caller's 16-lane row, in every lane of the row (DPP row_newbcast).
template <int kR>
__device__ __forceinline__ float row_lane_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + kR, 0xf, 0xf, false));
}

// Workgroup barrier that orders LDS accesses only: unlike __syncthreads it
// does not wait for the workgroup's outstanding global stores.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Orders LDS accesses of the lanes of one wave (no instruction: a wave's
// LDS operations complete in order; this keeps the compiler from moving them).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// LDS bytes one wave needs for wave_torch_topk over n logits: the entries
// and the two stop-position lists of a partition step, and at least 64
// words past a row of n words (the register form's per-lane dummy words).
__host__ __device__ constexpr size_t topk_tie_scratch_bytes(int n) { return ((size_t)(n < 64 ? 64 : n) * 8 + 15) / 16 * 16; }

// LDS bytes of the decode router's bfloat16 logits rows of one token tile.
__host__ __device__ constexpr size_t decode_rows_bytes(int n_exp) {
  return ((size_t)kRouterTile * n_exp * sizeof(uint16_t) + 15) / 16 * 16;
}

// torch.topk(row.float(), k)'s CPU order (klc_torch_order.h) for one row of
// n bfloat16 logits, by one wave; leaves the k results in a[0 .. k)
// (entry = comparator key << 16 | expert).  scratch: topk_tie_scratch_bytes(n)
// bytes of LDS owned by the wave.  libstdc++'s introselect is followed step
// by step, but each __unguarded_partition runs as one wave step: with the
// pivot P at `first`, the left scan stops at the positions L holding a value
// not greater than P (ascending) and the right scan at the positions R
// holding a value not less than P (descending, then `first` itself); the
// i-th swap exchanges L[i] and R[i] while L[i] < R[i], and after m swaps the
// scan returns L[0] (m = 0), min(L[m], R[m - 1]) or, with L used up,
// R[m - 1].  Lane 0 runs the sequential pieces (median of three, insertion
// sorts, heap select, the final std::sort of k - 1 entries).
__device__ __forceinline__ void wave_torch_topk(const uint16_t* row, int n, int k, uint32_t* scratch) {
  const int lane = threadIdx.x & 63;
  uint32_t* a = scratch;
  uint16_t* lp = reinterpret_cast<uint16_t*>(scratch + n);
  uint16_t* rp = lp + n;
  for (int p = lane; p < n; p += kWave) a[p] = order_entry(row[p], p);
  wave_lds_sync();
  if (k * 64 <= n) {  // TopKImpl.h: std::partial_sort
    if (lane == 0) stl_partial_sort(a, 0, k, n);
    wave_lds_sync();
    return;
  }
  const int nth = k - 1;
  int first = 0, last = n;
  int depth = floor_log2(n) * 2;
  bool selected = false;
  while (last - first > 3) {
    if (depth == 0) {
      if (lane == 0) {
        stl_heap_select(a, first, nth + 1, last);
        entry_swap(a, first, nth);
      }
      selected = true;
      break;
    }
    --depth;
    if (lane == 0) stl_move_median_to_first(a, first, first + 1, first + (last - first) / 2, last - 1);
    wave_lds_sync();
    const uint32_t pk = a[first] >> 16;
    int cl = 0, cr = 0;
    for (int c = first + 1; c < last; c += kWave) {
      const int p = c + lane;
      const uint32_t key = p < last ? a[p] >> 16 : 0u;
      const bool fl = p < last && key <= pk;
      const bool fr = p < last && key >= pk;
      const uint64_t bl = __ballot(fl), br = __ballot(fr);
      const uint64_t below = (1ull << lane) - 1ull;
      if (fl) lp[cl + __popcll(bl & below)] = (uint16_t)p;
      if (fr) rp[cr + __popcll(br & below)] = (uint16_t)p;
      cl += __popcll(bl);
      cr += __popcll(br);
    }
    wave_lds_sync();
    // R descending: R[i] = rp[cr - 1 - i]; L[i] < R[i] holds for a prefix of i
    const int lim = min(cl, cr);
    int m = 0;
    for (int c = 0; c < lim; c += kWave) {
      const int i = c + lane;
      m += __popcll(__ballot(i < lim && lp[i] < rp[cr - 1 - i]));
    }
    int cut;
    if (m == 0) cut = lp[0];
    else if (m < cl) cut = min((int)lp[m], (int)rp[cr - m]);
    else cut = rp[cr - m];
    for (int c = 0; c < m; c += kWave) {
      const int i = c + lane;
      if (i < m) {
        const int x = lp[i], y = rp[cr - 1 - i];
        const uint32_t vx = a[x], vy = a[y];
        a[x] = vy;
        a[y] = vx;
      }
    }
    wave_lds_sync();
    if (cut <= nth) first = cut;
    else last = cut;
  }
  if (lane == 0) {
    if (!selected) stl_insertion_sort(a, first, last);
    stl_sort(a, 0, k - 1);
  }
  wave_lds_sync();
}

// Entry at wave-uniform position p of a row held in v[0 .. S) (position p in
// slot p / 64 of lane p % 64): the lane is read from every slot, then one is
// picked (a select between the slots' registers would turn into a run-time
// indexed array in scratch).
template <int S>
__device__ __forceinline__ uint32_t row_get(const uint32_t (&v)[S], int p) {
  const int slot = p >> 6, l = p & 63;
  uint32_t x = (uint32_t)__builtin_amdgcn_readlane((int)v[0], l);
#pragma unroll
  for (int i = 1; i < S; ++i) {
    const uint32_t y = (uint32_t)__builtin_amdgcn_readlane((int)v[i], l);
    x = slot == i ? y : x;
  }
  return x;
}

// Stable sort by key, descending, of the entries at positions [lo, hi) of
// slot 0 (hi <= 64): each lane's rank among them, then a scatter through LDS
// (dummy: one word per lane).  Equal keys keep their order, as libstdc++'s
// insertion sort leaves them.
__device__ __forceinline__ uint32_t lanes_stable_sort_desc(uint32_t v0, int lo, int hi, uint32_t* scratch,
                                                           uint32_t* dummy) {
  const int lane = threadIdx.x & 63;
  const uint32_t mk = v0 >> 16;
  int rank = 0;
  for (int i = lo; i < hi; ++i) {
    const uint32_t ki = (uint32_t)__builtin_amdgcn_readlane((int)v0, i) >> 16;
    rank += (ki > mk || (ki == mk && i < lane)) ? 1 : 0;
  }
  const bool in = lane >= lo && lane < hi;
  scratch[in ? lo + rank : (int)(dummy - scratch) + lane] = v0;
  wave_lds_sync();
  const uint32_t x = scratch[lane];
  wave_lds_sync();
  return in ? x : v0;
}

// One __unguarded_partition step of the introselect on positions [first,
// last) of a row held in v[0 .. S) (position p in slot p / 64 of lane
// p % 64), with the median of three moved to `first` as the pivot P.  The
// left scan stops at the positions L holding a value not greater than P
// (ascending), the right scan at the positions R holding a value not less
// than P (descending, then `first`).  The i-th left stop x swaps with the
// i-th right stop while x lies below it, i.e. while at least i + 1 right
// stops lie above x: m, the number of swaps, is the count of left stops
// with that property.  The m pairs exchange their entries through LDS
// (buf_l, buf_r: (n + 1) / 2 words each; dummy: one word per lane for
// lanes without a partner, so every lane stores and loads unconditionally).
// Returns the cut: L[0] (m = 0), min(L[m], R[m - 1]), or R[m - 1] once L is
// used up.
template <int S>
__device__ __forceinline__ int wave_partition_round(uint32_t (&v)[S], int first, int last, uint32_t* buf_l,
                                                    uint32_t* buf_r, uint32_t* dummy) {
  constexpr int kNone = 1 << 30;
  const int lane = threadIdx.x & 63;
  // __move_median_to_first(first, first + 1, mid, last - 1)
  const int pa = first + 1, pb = first + (last - first) / 2, pc = last - 1;
  const uint32_t va = row_get(v, pa), vb = row_get(v, pb), vc = row_get(v, pc), vf = row_get(v, first);
  int pick;
  uint32_t vm;
  if (entry_gt(va, vb)) {
    if (entry_gt(vb, vc)) { pick = pb; vm = vb; }
    else if (entry_gt(va, vc)) { pick = pc; vm = vc; }
    else { pick = pa; vm = va; }
  } else if (entry_gt(va, vc)) { pick = pa; vm = va; }
  else if (entry_gt(vb, vc)) { pick = pc; vm = vc; }
  else { pick = pb; vm = vb; }
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int p = s * kWave + lane;
    v[s] = p == first ? vm : (p == pick ? vf : v[s]);
  }
  const uint32_t pk = vm >> 16;
  // the scans' stops: L (left, ascending), R (right, descending).  Per lane
  // and slot: bl / br = left / right stops before the position, flags bit 0
  // = a left stop, bit 1 = a right stop (VGPRs: lane masks of every slot
  // kept live through the exchange would crowd the scalar registers)
  int bl[S], br[S];
  uint32_t flags[S];
  int cl = 0, cr = 0;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int p = s * kWave + lane;
    const bool in = p > first && p < last;
    const uint32_t key = v[s] >> 16;
    const bool is_l = in && key <= pk, is_r = in && key >= pk;
    const uint64_t lmask = __builtin_amdgcn_ballot_w64(is_l);
    const uint64_t rmask = __builtin_amdgcn_ballot_w64(is_r);
    bl[s] = __builtin_amdgcn_mbcnt_hi((uint32_t)(lmask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)lmask, (uint32_t)cl));
    br[s] = __builtin_amdgcn_mbcnt_hi((uint32_t)(rmask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)rmask, (uint32_t)cr));
    flags[s] = (is_l ? 1u : 0u) | (is_r ? 2u : 0u);
    cl += __popcll(lmask);
    cr += __popcll(rmask);
  }
  // swap count: the i-th left stop x swaps while at least i + 1 right stops
  // lie above x (cr - br - [x is a right stop] of them)
  int m = 0;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int above = cr - br[s] - (int)(flags[s] >> 1);
    m += __popcll(__builtin_amdgcn_ballot_w64((flags[s] & 1u) != 0u && above > bl[s]));
  }
  // exchange the m pairs' entries through LDS (every lane stores and loads;
  // no branch): the i-th left stop's entry goes to buf_l[i], the i-th right
  // stop's (counted from the top) to buf_r[i]
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int ir = cr - 1 - br[s];
    const bool sl = (flags[s] & 1u) != 0u && bl[s] < m;
    const bool sr = (flags[s] & 2u) != 0u && ir < m;
    const int dum = (int)(dummy - buf_l) + lane;
    buf_l[sl ? bl[s] : dum] = v[s];
    buf_l[sr ? (int)(buf_r - buf_l) + ir : dum] = v[s];
  }
  wave_lds_sync();
  uint32_t x[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int ir = cr - 1 - br[s];
    const bool sl = (flags[s] & 1u) != 0u && bl[s] < m;
    const bool sr = (flags[s] & 2u) != 0u && ir < m;
    // word offsets from buf_l (a select between LDS pointers put the row in scratch)
    const int at = sl ? (int)(buf_r - buf_l) + bl[s] : (sr ? ir : (int)(dummy - buf_l) + lane);
    x[s] = buf_l[at];
  }
  // where the left scan stopped (while the loads are in flight): L[0]
  // (m = 0), min(L[m], R[m - 1]), or R[m - 1] once L is used up
  int lm = kNone, rm1 = kNone;
#pragma unroll
  for (int s = S - 1; s >= 0; --s) {
    const uint64_t at_l = __builtin_amdgcn_ballot_w64((flags[s] & 1u) != 0u && bl[s] == m);
    const uint64_t at_r = __builtin_amdgcn_ballot_w64(m > 0 && (flags[s] & 2u) != 0u && cr - 1 - br[s] == m - 1);
    if (at_l) lm = s * kWave + __builtin_ctzll(at_l);
    if (at_r) rm1 = s * kWave + __builtin_ctzll(at_r);
  }
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int ir = cr - 1 - br[s];
    const bool swapped = ((flags[s] & 1u) != 0u && bl[s] < m) || ((flags[s] & 2u) != 0u && ir < m);
    v[s] = swapped ? x[s] : v[s];
  }
  wave_lds_sync();
  return min(lm, rm1);
}

// The register form of wave_torch_topk, for rows of n <= 64 * S entries in
// the introselect regime (k * 64 > n) with k <= 16: position p of the row
// lives in slot p / 64 of lane p % 64.  Each partition step is ballots and
// prefix counts (wave_partition_round); once the range [first, last) lies
// below position 64 (nth < 16 is always inside it) only slot 0 takes part.
// After the loop every position involved is below 19, so the two insertion
// sorts run as stable rank sorts of lanes of slot 0.  The rare depth-limit
// branch (heap select) spills the row to LDS and finishes sequentially in
// lane 0.  Returns, in lane out_lane_base + j (j < k), the expert of result
// j; other lanes get my_id back.  scratch: topk_tie_scratch_bytes(n) bytes.
template <int S>
__device__ __forceinline__ int wave_torch_topk_regs(const uint16_t* row, int n, int k, uint32_t* scratch,
                                                    int out_lane_base, int my_id) {
  const int lane = threadIdx.x & 63;
  uint32_t v[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int p = s * kWave + lane;
    v[s] = p < n ? order_entry(row[p], p) : 0u;
  }
  uint32_t* buf_l = scratch;
  uint32_t* buf_r = scratch + (n + 1) / 2;
  uint32_t* dummy = scratch + n;  // one word per lane for lanes without a partner
  const int nth = k - 1;
  int first = 0, last = n;
  int depth = floor_log2(n) * 2;
  bool spilled = false;
  while (last - first > 3) {
    if (depth == 0) {
#pragma unroll
      for (int s = 0; s < S; ++s)
        if (s * kWave + lane < n) scratch[s * kWave + lane] = v[s];
      wave_lds_sync();
      if (lane == 0) {
        stl_heap_select(scratch, first, nth + 1, last);
        entry_swap(scratch, first, nth);
        stl_sort(scratch, 0, k - 1);
      }
      wave_lds_sync();
      spilled = true;
      break;
    }
    --depth;
    int cut;
    if (S == 1 || last <= kWave) {
      // the range lies in slot 0: the other slots hold positions >= last, which no longer move
      uint32_t v0[1] = {v[0]};
      cut = wave_partition_round<1>(v0, first, last, buf_l, buf_r, dummy);
      v[0] = v0[0];
    } else {
      cut = wave_partition_round<S>(v, first, last, buf_l, buf_r, dummy);
    }
    if (cut <= nth) first = cut;
    else last = cut;
  }
  if (!spilled) {
    // std::__insertion_sort of [first, last), then std::sort of [0, k - 1) (<= 16 entries: insertion
    // sort): both stable for equal keys.  nth < 16 lies in [first, last), so every position involved
    // is below 19, in slot 0.
    v[0] = lanes_stable_sort_desc(v[0], first, last, scratch, dummy);
    v[0] = lanes_stable_sort_desc(v[0], 0, k - 1, scratch, dummy);
    const int j = lane - out_lane_base;
    const uint32_t id = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (j >= 0 && j < k ? j : 0), (int)(v[0] & 0xffffu));
    if (j >= 0 && j < k) my_id = (int)id;
  } else {
    if (lane >= out_lane_base && lane < out_lane_base + k) my_id = (int)(scratch[lane - out_lane_base] & 0xffffu);
    wave_lds_sync();
  }
  return my_id;
}

// Expert class of a router: 1, 2 or 4 when k <= 16, k * 64 > n_exp (torch's
// introselect regime) and n_exp <= 64, 128 or 256 -- the rows then take
// only the register and 4-tokens-per-wave forms of that size, so a kernel
// instantiated for the class compiles no other form (the decode router's
// code drops from ~38,700 to ~12,000 instructions, which shortens its
// workgroups' start); 0 otherwise (every form compiled, chosen per call).
__host__ __device__ constexpr int router_expert_class(int64_t n_exp, int64_t k) {
  return (k > 16 || k * 64 <= n_exp || n_exp > 256) ? 0 : n_exp <= 64 ? 1 : n_exp <= 128 ? 2 : 4;
}

// torch's order for one tie row by the whole wave: the register form for
// the rows the 4-tokens-per-wave kernel takes (n <= 256, k <= 16) in the
// introselect regime, the LDS form otherwise.  Returns the expert of result
// j in lane out_lane_base + j.  kCls: router_expert_class(n, k), or 0.
template <int kCls = 0>
__device__ __forceinline__ int wave_torch_topk_lanes(const uint16_t* row, int n, int k, uint32_t* scratch, int out_lane_base,
                                     int my_id) {
  if constexpr (kCls > 0) return wave_torch_topk_regs<kCls>(row, n, k, scratch, out_lane_base, my_id);
  if (k * 64 > n && k <= 16) {
    if (n <= 64) return wave_torch_topk_regs<1>(row, n, k, scratch, out_lane_base, my_id);
    if (n <= 128) return wave_torch_topk_regs<2>(row, n, k, scratch, out_lane_base, my_id);
    if (n <= 256) return wave_torch_topk_regs<4>(row, n, k, scratch, out_lane_base, my_id);
  }
  wave_torch_topk(row, n, k, scratch);
  const int lane = threadIdx.x & 63;
  if (lane >= out_lane_base && lane < out_lane_base + k) my_id = (int)(scratch[lane - out_lane_base] & 0xffffu);
  wave_lds_sync();
  return my_id;
}

// torch's CPU softmax (klc_torch_order.h) of the k values held by lanes
// 0 .. k - 1 of the wave (lane r holds slot r), evaluated by every lane:
// the maximum in slot order, exp(v - max), the sum left to right, one
// reciprocal; returns the bfloat16 weight of the calling lane's slot.  The
// slot values are read with readlane (no LDS round trip).
__device__ __forceinline__ uint32_t torch_softmax_bf16(float v, int k) {
#pragma clang fp contract(off)
  float mx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  for (int r = 1; r < k; ++r) mx = torch_vec_max(mx, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), r)));
  const float e = sleef_expf_u10(v - mx);
  float sum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), 0));
  for (int r = 1; r < k; ++r) sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), r));
  const float inv = 1.0f / sum;
  return f32_to_bf16_rne(e * inv);
}

// The same softmax per 16-lane row: lane r < k of each row holds that row's
// slot r (k <= 16); the values are broadcast inside the row by DPP.
__device__ __forceinline__ uint32_t torch_softmax_bf16_row(float v, int k) {
#pragma clang fp contract(off)
  float mx = row_lane_f32<0>(v);
#pragma unroll
  for (int r = 1; r < 16; ++r) {
    float x;
    switch (r) {
      case 1: x = row_lane_f32<1>(v); break;
      case 2: x = row_lane_f32<2>(v); break;
      case 3: x = row_lane_f32<3>(v); break;
      case 4: x = row_lane_f32<4>(v); break;
      case 5: x = row_lane_f32<5>(v); break;
      case 6: x = row_lane_f32<6>(v); break;
      case 7: x = row_lane_f32<7>(v); break;
      case 8: x = row_lane_f32<8>(v); break;
      case 9: x = row_lane_f32<9>(v); break;
      case 10: x = row_lane_f32<10>(v); break;
      case 11: x = row_lane_f32<11>(v); break;
      case 12: x = row_lane_f32<12>(v); break;
      case 13: x = row_lane_f32<13>(v); break;
      case 14: x = row_lane_f32<14>(v); break;
      default: x = row_lane_f32<15>(v); break;
    }
    if (r < k) mx = torch_vec_max(mx, x);
  }
  const float e = sleef_expf_u10(v - mx);
  float sum = row_lane_f32<0>(e);
#pragma unroll
  for (int r = 1; r < 16; ++r) {
    float x;
    switch (r) {
      case 1: x = row_lane_f32<1>(e); break;
      case 2: x = row_lane_f32<2>(e); break;
      case 3: x = row_lane_f32<3>(e); break;
      case 4: x = row_lane_f32<4>(e); break;
      case 5: x = row_lane_f32<5>(e); break;
      case 6: x = row_lane_f32<6>(e); break;
      case 7: x = row_lane_f32<7>(e); break;
      case 8: x = row_lane_f32<8>(e); break;
      case 9: x = row_lane_f32<9>(e); break;
      case 10: x = row_lane_f32<10>(e); break;
      case 11: x = row_lane_f32<11>(e); break;
      case 12: x = row_lane_f32<12>(e); break;
      case 13: x = row_lane_f32<13>(e); break;
      case 14: x = row_lane_f32<14>(e); break;
      default: x = row_lane_f32<15>(e); break;
    }
    if (r < k) sum = sum + x;
  }
  const float inv = 1.0f / sum;
  return f32_to_bf16_rne(e * inv);
}

// Where a token's selection goes: ids (agent-scope stores: the decode
// router's final dispatch may run in another workgroup), the float32 values
// (optional), the bf16 weights, a second copy of the ids in LDS (optional,
// same indices) and copies of ids and weights in a host record (pinned host
// memory mapped into the device; optional), fenced at system scope so that
// an event recorded after the kernel finds them in host memory.
struct SelectionOut {
  int32_t* ids;
  float* values;
  uint16_t* weights;
  int32_t* lds_ids;
  int32_t* host_ids;
  uint16_t* host_weights;

  __device__ __forceinline__ void put(int64_t o, int id, float v, uint32_t w) const {
    __hip_atomic_store(ids + o, id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (lds_ids != nullptr) lds_ids[o] = id;
    if (values != nullptr) values[o] = v;
    weights[o] = (uint16_t)w;
    if (host_ids != nullptr) {
      host_ids[o] = id;
      host_weights[o] = (uint16_t)w;
      __threadfence_system();
    }
  }
};

// Top-k + softmax of one token's logits row by one wave, kSlots keys per
// lane.  The keys order values (NaN largest, -0 == +0), then lower expert
// index first; k + 1 rounds of wave maxima give the k largest and the next
// value.  If no two of those k + 1 values are equal, torch's order is that
// descending order; otherwise the wave replays torch's order
// (wave_torch_topk, tie_scratch: topk_tie_scratch_bytes(n_exp) bytes of
// the wave's LDS).  kCls: router_expert_class(n_exp, k), or 0.
template <int kSlots, int kCls = 0>
__device__ __forceinline__ void topk_softmax_row_n(const uint16_t* row, int n_exp, int k, int64_t t,
                                                   const SelectionOut& out, uint32_t* tie_scratch) {
  const int lane = threadIdx.x & 63;
  uint32_t keys[kSlots];
#pragma unroll
  for (int s = 0; s < kSlots; ++s) {
    const int idx = lane + s * kWave;
    keys[s] = idx < n_exp ? sel_key(row[idx], idx) : 0u;  // a real key is never 0
  }
  // lane r keeps the r-th selection
  int my_id = 0;
  bool tie = false;
  uint32_t prev = 0;
  const int rounds = k < n_exp ? k + 1 : k;
  for (int r = 0; r < rounds; ++r) {
    uint32_t best = keys[0];
#pragma unroll
    for (int s = 1; s < kSlots; ++s) best = keys[s] > best ? keys[s] : best;
    best = wave_max_u32(best);
#pragma unroll
    for (int s = 0; s < kSlots; ++s)
      if (keys[s] == best) keys[s] = 0u;
    const uint32_t value_key = best >> 16;
    tie |= r > 0 && value_key == prev;
    prev = value_key;
    if (lane == r) my_id = (int)(0xffffu - (best & 0xffffu));
  }
  if (tie) my_id = wave_torch_topk_lanes<kCls>(row, n_exp, k, tie_scratch, 0, my_id);  // uniform: the same maxima
  const float my_val = bf16_to_f32(row[lane < k ? my_id : 0]);
  const uint32_t w = torch_softmax_bf16(my_val, k);
  if (lane < k) out.put(t * k + lane, my_id, my_val, w);
}

template <int kCls = 0>
__device__ __forceinline__ void topk_softmax_row(const uint16_t* row, int n_exp, int k, int64_t t,
                                                 const SelectionOut& out, uint32_t* tie_scratch) {
  if constexpr (kCls > 0) {
    topk_softmax_row_n<kCls, kCls>(row, n_exp, k, t, out, tie_scratch);
    return;
  }
  const int slots = (n_exp + kWave - 1) / kWave;  // <= kTopkMaxPerLane (checked on the host)
  if (slots <= 1) topk_softmax_row_n<1>(row, n_exp, k, t, out, tie_scratch);
  else if (slots <= 2) topk_softmax_row_n<2>(row, n_exp, k, t, out, tie_scratch);
  else if (slots <= 4) topk_softmax_row_n<4>(row, n_exp, k, t, out, tie_scratch);
  else if (slots <= 8) topk_softmax_row_n<8>(row, n_exp, k, t, out, tie_scratch);
  else topk_softmax_row_n<kTopkMaxPerLane>(row, n_exp, k, t, out, tie_scratch);
}

// Top-k + softmax of up to 16 tokens by one 256-thread workgroup; tokens
// 4 w .. 4 w + 3 go to wave w, whose 16 lanes of row q (lanes 16 q ..
// 16 q + 15) take token 4 w + q, lane r of the row holding the keys of
// experts r + 16 s.  Each round's maximum comes from the lane's own keys and
// 4 DPP steps inside the row (quad swaps, half-row and row mirrors), so a
// wave's 4 selections run side by side: k + 1 rounds give the k largest
// and the next value.  Rows without equal values among those k + 1 are
// finished at once (torch's order is the descending order); rows with ties
// go to a workgroup list, and the 4 waves replay them in turn
// (wave_torch_topk_lanes), so a workgroup's ties are spread over its waves.
// rows(t) gives local token t's logits row; n_block <= 16 tokens; token t
// is written at t_base + t.  n_exp <= 16 kSlots, k <= 16.  Every thread of
// the workgroup must call this (it synchronises the workgroup).
// tie_scratch: the calling wave's topk_tie_scratch_bytes(n_exp) bytes of
// LDS; tie_list: 17 ints of LDS shared by the workgroup.  kCls:
// router_expert_class(n_exp, k), or 0.
template <int kSlots, int kCls, typename RowFn>
__device__ __forceinline__ void topk_softmax_block_quad(RowFn rows, int n_block, int n_exp, int k, int64_t t_base,
                                                        const SelectionOut& out, uint32_t* tie_scratch,
                                                        int* tie_list) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int q = lane >> 4;
  const int r = lane & 15;
  const int n_valid = min(max(n_block - 4 * wave, 0), 4);
  if (threadIdx.x == 0) tie_list[16] = 0;
  lds_barrier();
  if (n_valid > 0) {
    const uint16_t* row = rows(4 * wave + min(q, n_valid - 1));
    uint32_t keys[kSlots];
#pragma unroll
    for (int s = 0; s < kSlots; ++s) {
      const int idx = r + s * 16;
      keys[s] = idx < n_exp ? sel_key(row[idx], idx) : 0u;  // a real key is never 0
    }
    int my_id = 0;
    bool tie = false;
    uint32_t prev = 0;
    const int rounds = k < n_exp ? k + 1 : k;
    for (int rd = 0; rd < rounds; ++rd) {
      uint32_t best = keys[0];
#pragma unroll
      for (int s = 1; s < kSlots; ++s) best = keys[s] > best ? keys[s] : best;
      best = row_max_u32(best);  // every lane of the row holds its maximum
#pragma unroll
      for (int s = 0; s < kSlots; ++s)
        if (keys[s] == best) keys[s] = 0u;
      const uint32_t value_key = best >> 16;
      tie |= rd > 0 && value_key == prev;
      prev = value_key;
      if (r == rd) my_id = (int)(0xffffu - (best & 0xffffu));
    }
    // every row's softmax is evaluated (the row's lanes exchange values); tie rows' results are dropped
    const float my_val = bf16_to_f32(row[r < k ? my_id : 0]);
    const uint32_t w = torch_softmax_bf16_row(my_val, k);
    if (q < n_valid) {
      if (tie) {
        if (r == 0) tie_list[atomicAdd(&tie_list[16], 1)] = 4 * wave + q;
      } else if (r < k) {
        out.put((t_base + 4 * wave + q) * k + r, my_id, my_val, w);
      }
    }
  }
  lds_barrier();
  const int n_ties = tie_list[16];
  for (int i = wave; i < n_ties; i += 4) {
    const int t = tie_list[i];
    const uint16_t* row = rows(t);
    const int id = wave_torch_topk_lanes<kCls>(row, n_exp, k, tie_scratch, 0, 0);
    const float v = bf16_to_f32(row[lane < k ? id : 0]);
    const uint32_t w = torch_softmax_bf16(v, k);
    if (lane < k) out.put((t_base + t) * k + lane, id, v, w);
  }
}

// Top-k + softmax of up to 16 tokens (local t < n_block, written at
// t_base + t) by one 256-thread workgroup: the 4-tokens-per-wave form when a
// row fits (n_exp <= 256, k <= 16), else token by token, 4 per wave.
// out: where the selections go (SelectionOut).  tie_scratch: the wave's
// topk_tie_scratch_bytes(n_exp) bytes of LDS; tie_list: 17 ints of LDS.
// Called by every thread of the workgroup.  kCls: router_expert_class(n_exp,
// k), or 0.
template <int kCls = 0, typename RowFn>
__device__ __forceinline__ void topk_softmax_block(RowFn rows, int n_block, int n_exp, int k, int64_t t_base,
                                                   const SelectionOut& out, uint32_t* tie_scratch, int* tie_list) {
  if constexpr (kCls > 0) {
    topk_softmax_block_quad<4 * kCls, kCls>(rows, n_block, n_exp, k, t_base, out, tie_scratch, tie_list);
    return;
  }
  if (k <= 16 && n_exp <= 256) {
    if (n_exp <= 64)
      topk_softmax_block_quad<4, 0>(rows, n_block, n_exp, k, t_base, out, tie_scratch, tie_list);
    else if (n_exp <= 128)
      topk_softmax_block_quad<8, 0>(rows, n_block, n_exp, k, t_base, out, tie_scratch, tie_list);
    else
      topk_softmax_block_quad<16, 0>(rows, n_block, n_exp, k, t_base, out, tie_scratch, tie_list);
  } else {
    const int wave = threadIdx.x >> 6;
    for (int q = 4 * wave; q < min(n_block, 4 * wave + 4); ++q)
      topk_softmax_row(rows(q), n_exp, k, t_base + q, out, tie_scratch);
  }
}

constexpr int kDispatchThreads = 256;
constexpr int kDispatchMaxExperts = 256;

// Inclusive prefix sum over the wave on the DPP network: shifts by 1, 2, 4
// and 8 within each 16-lane row, then two row broadcasts.
__device__ __forceinline__ int32_t wave_inclusive_scan(int32_t v) {
  uint32_t s = (uint32_t)v;
  s += dpp_u32<0x111, 0xf>(0u, s);  // row_shr:1
  s += dpp_u32<0x112, 0xf>(0u, s);  // row_shr:2
  s += dpp_u32<0x114, 0xf>(0u, s);  // row_shr:4
  s += dpp_u32<0x118, 0xf>(0u, s);  // row_shr:8
  s += dpp_u32<0x142, 0xa>(0u, s);  // row_bcast:15 into rows 1 and 3
  s += dpp_u32<0x143, 0xc>(0u, s);  // row_bcast:31 into rows 2 and 3
  return (int32_t)s;
}

// Exclusive prefix sum of LDS array `v[n]` (n <= 256) by the calling wave;
// total written to *total.  4 entries per lane.
__device__ __forceinline__ void wave_exclusive_scan_256(int32_t* v, int n, int32_t* total, int lane) {
  int32_t local[4];
  int32_t s = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = lane * 4 + i;
    local[i] = idx < n ? v[idx] : 0;
    s += local[i];
  }
  const int32_t incl = wave_inclusive_scan(s);
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
constexpr int kDispatchDirectPairs = 1024;  // up to this many pairs each expert's thread writes its units
constexpr int kDispatchWaves = kDispatchThreads / kWave;

__host__ __device__ constexpr int dispatch_chunks(int n_pairs) { return (n_pairs + kDispatchChunk - 1) / kDispatchChunk; }

// LDS bytes block_dispatch needs for n_pairs pairs: the pairs' experts and
// ranks (uint16 each), per-wave counts and five per-expert arrays.
__host__ __device__ constexpr size_t dispatch_lds_bytes(int n_pairs, int /*n_exp*/) {
  return 2 * (((size_t)n_pairs * sizeof(uint16_t) + 15) / 16 * 16) +
         (kDispatchWaves + 5) * kDispatchMaxExperts * sizeof(int32_t) + 8 * sizeof(int32_t);
}

// Largest n_pairs whose staging fits in 160 KiB of LDS (block_dispatch's
// limit; the decode router and the dispatch below 1024 pairs stay far under it).
constexpr int kDispatchLdsMaxPairs = 38648;
static_assert(dispatch_lds_bytes(kDispatchLdsMaxPairs, kDispatchMaxExperts) <= 160 * 1024, "dispatch LDS");
static_assert(dispatch_lds_bytes(kDispatchLdsMaxPairs + 8, kDispatchMaxExperts) > 160 * 1024, "dispatch LDS");

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
// chunks), so no step is serial over pairs.  get_id(p) returns pair p's
// expert id; lds holds dispatch_lds_bytes(n_pairs, n_exp) bytes.  The steps
// hand over LDS only, so the barriers between them do not wait for earlier
// global stores.
template <typename IdFn>
__device__ __forceinline__ void block_dispatch(IdFn get_id, int n_pairs, int n_exp, int32_t* __restrict__ offsets,
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
    for (int j = 0; j < 8; ++j) v[j] = get_id(min(p0 + j * kDispatchThreads + tid, n_pairs - 1));
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int p = p0 + j * kDispatchThreads + tid;
      if (p < n_pairs) sid[p] = (v[j] >= 0 && v[j] < n_exp) ? (uint16_t)v[j] : (uint16_t)0xffffu;
    }
  }
  lds_barrier();
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
  lds_barrier();
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
  lds_barrier();
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
  lds_barrier();
  // 3. scatter
  for (int p = tid; p < n_pairs; p += kDispatchThreads) {
    const uint32_t e = sid[p];
    if (e < (uint32_t)n_exp) {
      const int w = (p / kDispatchChunk) / cpw;
      sorted[total[e] + cnt[w * kDispatchMaxExperts + e] + rank[p]] = p;
    }
  }
  // 4. unit lists
  {
    const int n_gu = sums[2], n_dn = sums[3], n_all = sums[2] + sums[3] + sums[4];
    int32_t* const gu_list = units + kUnitHeader;
    int32_t* const dn_list = units + units_offset_down(n_pairs, n_exp);
    int32_t* const gm_list = units + units_offset_gemm(n_pairs, n_exp);
    // small batches: each expert's thread writes its own units (a few each)
    if (n_pairs <= kDispatchDirectPairs) {
      for (int e = tid; e < n_exp; e += kDispatchThreads) {
        const int cnt = (e + 1 < n_exp ? total[e + 1] : sums[0]) - total[e];
        for (int j = 0; j * kUnitTokensGateUp < cnt; ++j) gu_list[ugu[e] + j] = make_unit(e, j);
        for (int j = 0; j * kUnitTokensDown < cnt; ++j) dn_list[udn[e] + j] = make_unit(e, j);
        for (int j = 0; j * kUnitTokensGemm < cnt; ++j) gm_list[ugm[e] + j] = make_unit(e, j);
      }
    }
    // large batches: all three lists as one index space, 4 units per thread
    // at a time: a unit's expert is the last one whose first unit is <= the
    // unit (experts without units share the next one's first unit), found
    // by 8 bisection steps run in lockstep
    for (int u0 = tid; n_pairs > kDispatchDirectPairs && u0 < n_all; u0 += 4 * kDispatchThreads) {
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

// Last-arriver election among `expected` workgroups on *ctr.  Everything
// the workgroups hand over (partial logits, ids) is stored and loaded at
// agent scope (sc1: stores write through the XCD's L2, loads miss in the
// non-coherent caches), so no fence is needed: every wave waits for its own
// stores to complete, then thread 0 counts the arrival, and the last
// workgroup resets the counter for the next launch.  (An agent-scope fence
// would write back and invalidate the whole L2.)  Returns the same value in
// every thread.
__device__ __forceinline__ bool arrive_last(uint32_t* ctr, uint32_t expected, uint32_t* flag) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t last = prev == expected - 1u ? 1u : 0u;
    if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = last;
  }
  __syncthreads();
  return *flag != 0u;
}

// block_dispatch's outputs for at most 64 pairs (one token tile), by one
// wave: pair p sits in lane p; its rank among the earlier pairs of its
// expert comes from the key ballots (wave_peers), the per-expert counts from
// LDS atomics, and the offsets, active-list positions and the three lists'
// first units from five scans of the wave, with no workgroup barrier.
// ids: the pairs' experts in LDS; lds: 5 * 256 + 8 ints.
__device__ __forceinline__ void wave_dispatch(const int32_t* ids, int n_pairs, int n_exp,
                                              int32_t* __restrict__ offsets, int32_t* __restrict__ sorted,
                                              int32_t* __restrict__ active, int32_t* __restrict__ n_active,
                                              int32_t* __restrict__ units, int32_t* lds) {
  const int lane = threadIdx.x & 63;
  int32_t* cnt = lds;                          // counts, then offsets
  int32_t* flags = cnt + kDispatchMaxExperts;  // expert has pairs, then its active-list position
  int32_t* ugu = flags + kDispatchMaxExperts;  // units per expert, then the first one (gate_up)
  int32_t* udn = ugu + kDispatchMaxExperts;    // same for down
  int32_t* ugm = udn + kDispatchMaxExperts;    // same for the GEMM
  int32_t* sums = ugm + kDispatchMaxExperts;
  const int id = lane < n_pairs ? ids[lane] : -1;
  const bool valid = id >= 0 && id < n_exp;
  uint32_t key[1] = {valid ? (uint32_t)id : 511u};
  uint64_t peers[1];
  wave_peers(key, peers);
  const int rank = __popcll(peers[0] & ((1ull << lane) - 1ull));
  for (int e = lane; e < n_exp; e += kWave) cnt[e] = 0;
  wave_lds_sync();
  if (valid) atomicAdd(&cnt[id], 1);
  wave_lds_sync();
  for (int e = lane; e < n_exp; e += kWave) {
    const int32_t c = cnt[e];
    flags[e] = c > 0 ? 1 : 0;
    ugu[e] = (c + kUnitTokensGateUp - 1) / kUnitTokensGateUp;
    udn[e] = (c + kUnitTokensDown - 1) / kUnitTokensDown;
    ugm[e] = (c + kUnitTokensGemm - 1) / kUnitTokensGemm;
  }
  wave_lds_sync();
  wave_exclusive_scan_256(cnt, n_exp, &sums[0], lane);
  wave_exclusive_scan_256(flags, n_exp, &sums[1], lane);
  wave_exclusive_scan_256(ugu, n_exp, &sums[2], lane);
  wave_exclusive_scan_256(udn, n_exp, &sums[3], lane);
  wave_exclusive_scan_256(ugm, n_exp, &sums[4], lane);
  wave_lds_sync();
  if (valid) sorted[cnt[id] + rank] = lane;
  int32_t* const gu_list = units + kUnitHeader;
  int32_t* const dn_list = units + units_offset_down(n_pairs, n_exp);
  int32_t* const gm_list = units + units_offset_gemm(n_pairs, n_exp);
  for (int e = lane; e < n_exp; e += kWave) {
    const int c = (e + 1 < n_exp ? cnt[e + 1] : sums[0]) - cnt[e];
    offsets[e] = cnt[e];
    if (c > 0) active[flags[e]] = e;
    if (e >= sums[1]) active[e] = -1;
    for (int j = 0; j * kUnitTokensGateUp < c; ++j) gu_list[ugu[e] + j] = make_unit(e, j);
    for (int j = 0; j * kUnitTokensDown < c; ++j) dn_list[udn[e] + j] = make_unit(e, j);
    for (int j = 0; j * kUnitTokensGemm < c; ++j) gm_list[ugm[e] + j] = make_unit(e, j);
  }
  if (lane == 0) {
    offsets[n_exp] = sums[0];
    *n_active = sums[1];
    units[0] = sums[2];
    units[1] = sums[3];
    units[2] = sums[4];
    units[3] = 0;
  }
}

// The dispatch (block_dispatch's outputs) of one token's k pairs, by one
// wave: the experts tile_ids[0 .. k) are distinct (a top-k), so pair j's
// position among the expert-sorted pairs is the number of its experts below
// its own, every expert has at most one pair, and each list's r-th unit is
// pass 0 of the r-th expert in ascending order.
__device__ __forceinline__ void single_token_dispatch(const int32_t* tile_ids, int n_exp, int k,
                                                      int32_t* __restrict__ offsets, int32_t* __restrict__ sorted,
                                                      int32_t* __restrict__ active, int32_t* __restrict__ n_active,
                                                      int32_t* __restrict__ units) {
  const int lane = threadIdx.x & 63;
  const int n_pairs = k;
  const int my = lane < k ? tile_ids[lane] : 0x7fffffff;
  int rank = 0;
  for (int i = 0; i < k; ++i) rank += __builtin_amdgcn_readlane(my, i) < my ? 1 : 0;
  int32_t* const gu_list = units + kUnitHeader;
  int32_t* const dn_list = units + units_offset_down(n_pairs, n_exp);
  int32_t* const gm_list = units + units_offset_gemm(n_pairs, n_exp);
  if (lane < k) {
    sorted[rank] = lane;
    active[rank] = my;
    gu_list[rank] = make_unit(my, 0);
    dn_list[rank] = make_unit(my, 0);
    gm_list[rank] = make_unit(my, 0);
  }
  for (int e = lane; e <= n_exp; e += kWave) {
    int c = 0;
    for (int i = 0; i < k; ++i) c += __builtin_amdgcn_readlane(my, i) < e ? 1 : 0;
    offsets[e] = c;
  }
  for (int e = k + lane; e < n_exp; e += kWave) active[e] = -1;
  if (lane == 0) {
    *n_active = k;
    units[0] = k;
    units[1] = k;
    units[2] = k;
    units[3] = 0;
  }
}

}  // namespace
}  // namespace klc
