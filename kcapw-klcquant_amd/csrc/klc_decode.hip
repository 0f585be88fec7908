// The MoE layer of a small decode batch in one launch (gfx950):
// router logits -> top-k + softmax -> dispatch -> gate_up/SwiGLU -> down ->
// combine, for batches of at most 16 tokens (at most 64 token-slot pairs).
//
// Why one launch.  At these batch sizes each kernel of the multi-launch layer
// is mostly its own start-up and tail (a launch of a tiny kernel costs about
// 3 us between dispatch and completion on MI355X), and the router's
// cross-workgroup hand-offs cost more than its arithmetic.  Here every
// workgroup of a persistent grid (no more workgroups than the GPU holds at
// once) stays resident for the whole layer:
//
// 1. Router.  Workgroup e (e < n_experts) computes expert e's logits for all
//    tokens: float64 sums of the exact bfloat16 products, rounded once like
//    F.linear in bfloat16 (bf16(f32(sum) + bias)).  It stores each as a
//    64-bit word (the launch's tag above the 16 logit bits) at agent scope.
// 2. Routing.  Every workgroup polls those words until all carry this
//    launch's tag, then selects the top-k (torch's CPU order), the softmax
//    weights and the expert-sorted dispatch itself, in LDS.  No workgroup
//    waits for another's routing result, and no atomic is used: same-address
//    atomics from hundreds of workgroups serialise (about 5 us for one
//    counter that 512 workgroups poll and 128 increment).
// 3. Work items, taken round-robin by workgroup index: the gate_up items
//    (unit, tile group), then the down items, then the combine items (one
//    per down tile group, all tokens).  A finished gate_up or down item
//    stores its outputs at agent scope (write-through), waits for them to
//    complete, and stores the launch's tag into its flag word.  A down item starts
//    its weight stream first and then waits for the flags of the gate_up
//    unit that produced its inputs; a combine item waits for the flags of
//    its tile group's down items.  Every item waits only for items of lower
//    index, which workgroups that are already resident take before any
//    higher one, so every wait ends.
//
// The tag is a per-launch 64-bit number chosen on the host: a 52-bit launch
// count (36 bits in the logit words) under the high bits 0x7FB, a pattern no
// float or bfloat16 result has (as float32 or bfloat16 it is a signalling
// NaN, as float64 a value near 2^1020), so neither words and flags left by
// earlier launches nor other data left in scratch memory match it.  Nothing
// needs resetting and the layer leaves no state behind.  A launch inside HIP
// graph capture would replay one tag, so captured calls use the multi-launch
// layer.  Every wait is bounded: a wait that runs out (which
// needs a GPU shared with kernels that hold its compute units) sets a sticky
// status bit, records the launch's tag and goes on, so the launch always
// ends; the launch then poisons what it writes after that point (ids -1,
// NaN weights, NaN outputs), so the failure shows without a host sync.
//
// Numerics are the multi-launch layer's: the GEMVs are the same device code
// (klc_gemv.h) and the combine performs the same operations in the same
// order, so outputs are bit-identical given the same routing.  The router's
// float64 sums are exact for bfloat16 products short of a 2^53 spread of
// magnitudes, so the logits are the correctly rounded ones, as there.
#include <atomic>
#include <cstdlib>
#include <mutex>

#include "klc_gemv.h"
#include "klc_router_dev.h"

namespace klc {
namespace {

constexpr int kFusedMaxTokens = 16;  // one router token tile
constexpr int kFusedMaxPairs = 64;   // one wave dispatches
constexpr int kFusedMaxExperts = 256;
constexpr int kFusedMaxK = 16;
constexpr int kFusedThreads = 256;
constexpr int kSpinLimit = 1 << 18;  // polls of a wait before it gives up (each poll is a memory round trip)
constexpr int kCombineSlots = 4;     // slots whose expert-output loads are in flight together
#ifndef KLC_FUSED_RING_UP
#define KLC_FUSED_RING_UP 8
#endif
#ifndef KLC_FUSED_RING_DN
#define KLC_FUSED_RING_DN 8
#endif
constexpr int kRingUp = KLC_FUSED_RING_UP, kRingDn = KLC_FUSED_RING_DN;

// Launch tags: 0x7FB in the top 12 bits, the launch count below.  A logit
// word holds the tag's high 48 bits (the count's low 36 bits) above the
// logit's 16 bfloat16 bits.
constexpr uint64_t kTagHigh = 0x7FBull << 52;
__host__ __device__ constexpr uint64_t launch_tag(uint64_t count) { return kTagHigh | (count & ((1ull << 52) - 1)); }
__host__ __device__ constexpr uint64_t word_tag(uint64_t tag) {
  return ((tag & ~((1ull << 52) - 1)) | ((tag & ((1ull << 36) - 1)) << 16));
}

struct FusedArgs {
  const uint16_t* x;               // [n_tok][hidden] bfloat16
  const uint16_t* router_w;        // [n_exp][hidden]
  const uint16_t* router_b;        // [n_exp]
  const uint8_t* const* w_up;      // [n_exp] packed gate_up matrices
  const uint16_t* b_up;            // [n_exp][2 inter]
  const uint8_t* const* w_dn;      // [n_exp] packed down matrices
  const uint16_t* b_dn;            // [n_exp][hidden]
  const uint16_t* residual;        // [n_tok][hidden] or null
  uint16_t* out;                   // [n_tok][hidden]
  int32_t* ids;                    // [n_tok][k]
  uint16_t* weights;               // [n_tok][k] bfloat16
  float* values;                   // [n_tok][k] selected logits as float32
  uint16_t* logits;                // [n_tok][n_exp]
  uint64_t* words;                 // [n_exp][n_tok] tagged logits
  uint64_t* flags;                 // [max_up_items + max_dn_items] tags of finished items
  uint16_t* gated;                 // hi/lo planes [2][pairs][inter]
  float* eo;                       // [pairs][hidden]
  uint32_t* status;                // bit 0: a wait ran out (sticky: never cleared by a launch)
  uint64_t* fail_tag;              // the tag of the last launch in which a wait ran out
  int spin_limit;                  // polls of a wait before it gives up; < 0: give up at once
  int n_tok, hidden, inter, n_exp, k, precision;
  float limit;
  uint64_t tag;                    // the launch's flag value; tag_word(tag) tags the logit words
  int max_up_items;                // flag index of the first down item
};

// LDS: the routing state kept for the whole launch, then one area shared by
// the routing scratch and the GEMV's staged activation rows.
constexpr int kUnitsMax = kUnitHeader + 3 * kFusedMaxPairs;  // units_size(<= 64 pairs, any n_exp)
struct RoutingLds {
  int32_t sorted[kFusedMaxPairs];
  int32_t offsets[kFusedMaxExperts + 4];
  int32_t units[kUnitsMax];
  int32_t ids[kFusedMaxPairs];
  uint16_t wts[kFusedMaxPairs];
};
constexpr size_t kRoutingLdsBytes = (sizeof(RoutingLds) + 15) / 16 * 16;

// routing scratch inside the shared area: logits rows, per-wave tie
// scratch, the dispatch's counters, the active list and the values
struct ScratchLayout {
  size_t rows, tie, disp, active, values, red, total;
};
__host__ __device__ constexpr ScratchLayout scratch_layout(int n_exp) {
  ScratchLayout s{};
  size_t o = 0;
  s.rows = o;   o += decode_rows_bytes(n_exp);
  s.tie = o;    o += 4 * topk_tie_scratch_bytes(n_exp);
  s.disp = o;   o += ((5 * kDispatchMaxExperts + 8) * 4 + 15) / 16 * 16;
  s.active = o; o += (kFusedMaxExperts + 4) * 4;
  s.values = o; o += kFusedMaxPairs * 4;
  s.red = o;    o += (kFusedMaxTokens + 4) * 8;
  s.total = o;
  return s;
}

__host__ __device__ constexpr size_t fused_lds_bytes(int steps, int n_exp) {
  const size_t a = gemv_lds_bytes(steps), b = scratch_layout(n_exp).total;
  return kRoutingLdsBytes + (a > b ? a : b);
}

// Sum of v over the 16 lanes of each DPP row, in every lane of the row.
// Each step adds the partner's value (commutative, so the partners agree
// bit for bit and every lane ends with the same sum).
template <int kCtrl, int kRowMask>
__device__ __forceinline__ double dpp_add_f64(double v) {
  const uint64_t u = __double_as_longlong(v);
  const uint32_t lo = dpp_u32<kCtrl, kRowMask>(0u, (uint32_t)u);
  const uint32_t hi = dpp_u32<kCtrl, kRowMask>(0u, (uint32_t)(u >> 32));
  return v + __longlong_as_double((int64_t)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ double row_sum_f64(double v) {
  v = dpp_add_f64<0xB1, 0xf>(v);   // quad_perm [1, 0, 3, 2]
  v = dpp_add_f64<0x4E, 0xf>(v);   // quad_perm [2, 3, 0, 1]
  v = dpp_add_f64<0x141, 0xf>(v);  // row_half_mirror
  v = dpp_add_f64<0x140, 0xf>(v);  // row_mirror
  return v;
}
// Sum over the wave, valid in lane 63: row sums, then row_bcast:15 into
// rows 1 and 3 and row_bcast:31 into rows 2 and 3.
__device__ __forceinline__ double wave_sum_f64(double v) {
  v = row_sum_f64(v);
  v = dpp_add_f64<0x142, 0xa>(v);
  v = dpp_add_f64<0x143, 0xc>(v);
  return v;
}

// Logits of expert e for every token, stored as tagged words.  Each token
// gets lpt = 256 / (its power-of-two token count, at least 16) lanes, which
// take its 16-byte chunks lane, lane + lpt, ...; a lane issues up to
// kRouterLoads chunks' weight and hidden loads before it uses any, so one
// expert costs one or two memory round trips.  Per lane a float64
// accumulator; then DPP sums over a row (16 lanes), two rows, or the wave
// (lane 63), and for 128 or 256 lanes per token the waves' sums in wave
// order through LDS.
constexpr int kRouterLoads = 8;
__device__ __forceinline__ void router_expert(const FusedArgs& a, int e, double* red) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int n_tok = a.n_tok, hidden = a.hidden;
  const int lpt = n_tok == 1 ? 256 : n_tok == 2 ? 128 : n_tok <= 4 ? 64 : n_tok <= 8 ? 32 : 16;
  const int tok = tid / lpt;
  const int sub = tid - tok * lpt;
  const int nchunk = hidden >> 3;
  double acc = 0.0;
  if (tok < n_tok) {
    const uint16_t* wrow = a.router_w + (int64_t)e * hidden;
    const uint16_t* xrow = a.x + (int64_t)tok * hidden;
    for (int c0 = sub; c0 < nchunk; c0 += kRouterLoads * lpt) {
      u32x4_t wv[kRouterLoads], xv[kRouterLoads];
#pragma unroll
      for (int i = 0; i < kRouterLoads; ++i) {
        const int c = min(c0 + i * lpt, nchunk - 1);
        wv[i] = *reinterpret_cast<const u32x4_t*>(wrow + c * 8);
        xv[i] = *reinterpret_cast<const u32x4_t*>(xrow + c * 8);
      }
#pragma unroll
      for (int i = 0; i < kRouterLoads; ++i) {
        if (c0 + i * lpt < nchunk) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            acc += (double)__uint_as_float(wv[i][q] << 16) * (double)__uint_as_float(xv[i][q] << 16);
            acc += (double)__uint_as_float(wv[i][q] & 0xffff0000u) * (double)__uint_as_float(xv[i][q] & 0xffff0000u);
          }
        }
      }
    }
  }
  double* wsum = red + kFusedMaxTokens;  // [4] wave sums
  if (lpt == 16) {
    acc = row_sum_f64(acc);
    if ((lane & 15) == 15 && tok < n_tok) red[tok] = acc;
  } else if (lpt == 32) {
    acc = row_sum_f64(acc);
    acc = dpp_add_f64<0x142, 0xa>(acc);  // row_bcast:15: rows 1 and 3 add rows 0 and 2
    if ((lane & 31) == 31 && tok < n_tok) red[tok] = acc;
  } else {
    acc = wave_sum_f64(acc);
    if (lane == 63) wsum[wave] = acc;
  }
  lds_barrier();
  if (tid < n_tok) {
    const int t = tid;
    double sum;
    if (lpt == 256) sum = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
    else if (lpt == 128) sum = wsum[2 * t] + wsum[2 * t + 1];
    else if (lpt == 64) sum = wsum[t];
    else sum = red[t];
    const float bias = bf16_to_f32(a.router_b[e]);
    const uint64_t logit = f32_to_bf16_rne((float)sum + bias);
    __hip_atomic_store(a.words + (int64_t)e * n_tok + t, word_tag(a.tag) | logit, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
}

// A wait that ran out: the sticky status bit for the host, and the launch's
// tag for this launch's workgroups (their outputs are then poisoned).
// The stores complete before the wave goes on, so the workgroup's other
// waves (after its next barrier) and the consumers of its later flags see them.
__device__ __forceinline__ void ran_out(uint32_t* status, uint64_t* fail_tag, uint64_t tag) {
  __hip_atomic_fetch_or(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(fail_tag, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);
}
__device__ __forceinline__ bool launch_failed(const FusedArgs& a) {
  return __hip_atomic_load(a.fail_tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == a.tag;
}

// The calling wave polls n flag words until all hold `tag`, at most
// `limit` times (limit < 0: none).  A wait that runs out reports it (ran_out).
__device__ __forceinline__ void wait_flags(const uint64_t* flags, int n, uint64_t tag, uint32_t* status,
                                           uint64_t* fail_tag, int limit) {
  const int lane = threadIdx.x & 63;
  for (int it = 0;; ++it) {
    bool done = limit >= 0;
    for (int i = lane; done && i < n; i += kWave)
      done &= __hip_atomic_load(flags + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == tag;
    if (__ballot(!done) == 0) return;
    if (it >= limit) {
      if (lane == 0) ran_out(status, fail_tag, tag);
      return;
    }
    __builtin_amdgcn_s_sleep(2);
  }
}

// Every wave waits for its own outputs to complete, then thread 0 stores
// the tag into the item's flag.  The barrier also ends the item's use of LDS.
__device__ __forceinline__ void publish(uint64_t* flag, uint64_t tag) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_store(flag, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Tiles per work item: two (gate_up) or three (down) 64-row tiles once the
// items outnumber the workgroups enough, else one.
__device__ __forceinline__ int tiles_per_item(int total_tiles, int grid, int max_tpw) {
  int tpw = total_tiles / (2 * grid);
  return tpw < 1 ? 1 : (tpw > max_tpw ? max_tpw : tpw);
}

template <int kSteps>
#ifndef KLC_FUSED_WAVES_PER_EU
#define KLC_FUSED_WAVES_PER_EU 3
#endif
__global__ __launch_bounds__(kFusedThreads, KLC_FUSED_WAVES_PER_EU) void moe_decode_fused_kernel(FusedArgs a) {
  extern __shared__ __align__(16) char lds[];
  __shared__ int tie_list[17];
  RoutingLds& R = *reinterpret_cast<RoutingLds*>(lds);
  char* area = lds + kRoutingLdsBytes;
  const int n_tok = a.n_tok, n_exp = a.n_exp, k = a.k;
  const int n_pairs = n_tok * k;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const ScratchLayout sl = scratch_layout(n_exp);
  uint16_t* rows = reinterpret_cast<uint16_t*>(area + sl.rows);

  // ---- 1. router: expert e's logits for every token ----
  for (int e = blockIdx.x; e < n_exp; e += gridDim.x) {
    router_expert(a, e, reinterpret_cast<double*>(area + sl.red));
    lds_barrier();
  }

  // ---- 2. routing, in every workgroup ----
  {
    const int total = n_exp * n_tok;
    const uint64_t wtag = word_tag(a.tag);
    if (wave == 0) {
      // every poll writes the logits it read into the rows [16][n_exp]: once
      // all words carry the tag, the rows hold this launch's logits
      for (int it = 0;; ++it) {
        bool done = a.spin_limit >= 0;  // a negative limit gives up after the first read
        for (int i = lane; i < total; i += kWave) {
          const uint64_t wd = __hip_atomic_load(a.words + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          done &= (wd & ~0xffffull) == wtag;
          const int e = i / n_tok, t = i - e * n_tok;
          rows[t * n_exp + e] = (uint16_t)(wd & 0xffffu);
        }
        if (__ballot(!done) == 0) break;
        if (it >= a.spin_limit) {
          if (lane == 0) ran_out(a.status, a.fail_tag, a.tag);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    }
    lds_barrier();
    uint32_t* tie = reinterpret_cast<uint32_t*>(area + sl.tie + wave * topk_tie_scratch_bytes(n_exp));
    float* values = reinterpret_cast<float*>(area + sl.values);
    int32_t* active = reinterpret_cast<int32_t*>(area + sl.active);
    const SelectionOut sel{R.ids, values, R.wts, nullptr, nullptr, nullptr};
    if (n_tok == 1) {
      if (wave == 0) {
        topk_softmax_row(rows, n_exp, k, 0, sel, tie);
        wave_lds_sync();
        single_token_dispatch(R.ids, n_exp, k, R.offsets, R.sorted, active, active + kFusedMaxExperts + 2, R.units);
      }
    } else {
      topk_softmax_block([&](int t) { return rows + t * n_exp; }, n_tok, n_exp, k, 0, sel, tie, tie_list);
      lds_barrier();
      if (wave == 0)
        wave_dispatch(R.ids, n_pairs, n_exp, R.offsets, R.sorted, active, active + kFusedMaxExperts + 2, R.units,
                      reinterpret_cast<int32_t*>(area + sl.disp));
    }
    lds_barrier();
    if (blockIdx.x == 0) {
      // a routing wait of this launch that ran out (here or in another
      // workgroup so far) poisons the routing outputs: ids -1, NaN weights
      // and values
      const bool failed = launch_failed(a);
      for (int i = threadIdx.x; i < n_pairs; i += kFusedThreads) {
        a.ids[i] = failed ? -1 : R.ids[i];
        a.weights[i] = failed ? (uint16_t)0x7fc0u : R.wts[i];
        a.values[i] = failed ? __uint_as_float(0x7fc00000u) : values[i];
      }
      for (int i = threadIdx.x; i < n_tok * n_exp; i += kFusedThreads) a.logits[i] = rows[i];
    }
    lds_barrier();  // the routing scratch is dead from here on: the area holds staged rows
  }

  // ---- 3. work items ----
  // values read from LDS are the same in every lane: readfirstlane keeps
  // them (and the addresses and buffer descriptors built from them) scalar
  const int n_up_units = __builtin_amdgcn_readfirstlane(R.units[0]);
  const int n_dn_units = __builtin_amdgcn_readfirstlane(R.units[1]);
  const int32_t* gu_list = R.units + kUnitHeader;
  const int32_t* dn_list = R.units + units_offset_down(n_pairs, n_exp);
  const int up_rows = 2 * a.inter, dn_rows = a.hidden;
  const int tiles_up = up_rows / kTileRows, tiles_dn = dn_rows / kTileRows;
  const int tpw_up = tiles_per_item(n_up_units * tiles_up, gridDim.x, 2);
  const int tpw_dn = tiles_per_item(n_dn_units * tiles_dn, gridDim.x, 3);
  const int tg_up = (tiles_up + tpw_up - 1) / tpw_up, tg_dn = (tiles_dn + tpw_dn - 1) / tpw_dn;
  const int n_up = n_up_units * tg_up, n_dn = n_dn_units * tg_dn;
  const int n_items = n_up + n_dn + tg_dn;
  const int64_t plane = (int64_t)n_pairs * a.inter;
  uint16_t* xs = reinterpret_cast<uint16_t*>(area);

  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    if (item < n_up) {
      const int u = item / tg_up, j = item - u * tg_up;
      const int32_t unit = __builtin_amdgcn_readfirstlane(gu_list[u]);
      const int e = unit_expert(unit);
      const int pb = __builtin_amdgcn_readfirstlane(R.offsets[e]);
      const int tc = unit_pass(unit) * kUnitTokensGateUp;
      const int nt = min(kUnitTokensGateUp, __builtin_amdgcn_readfirstlane(R.offsets[e + 1]) - pb - tc);
      const int tile0 = j * tpw_up;
      gemv_unit<false, kSteps, true, kRingUp>(a.w_up[e], a.b_up, e, a.x, 0, nullptr, a.gated, plane, nullptr,
                                     R.sorted + pb + tc, nt, up_rows, a.hidden / 32, k, a.limit, a.precision, tile0,
                                     min(tpw_up, tiles_up - tile0), xs, NoWait{});
      publish(a.flags + item, a.tag);
    } else if (item < n_up + n_dn) {
      const int d = item - n_up;
      const int u = d / tg_dn, j = d - u * tg_dn;
      const int32_t unit = __builtin_amdgcn_readfirstlane(dn_list[u]);
      const int e = unit_expert(unit);
      const int pb = __builtin_amdgcn_readfirstlane(R.offsets[e]);
      const int tc = unit_pass(unit) * kUnitTokensDown;
      const int nt = min(kUnitTokensDown, __builtin_amdgcn_readfirstlane(R.offsets[e + 1]) - pb - tc);
      // the gate_up unit whose 8 tokens hold these 4
      const int32_t want = make_unit(e, unit_pass(unit) >> 1);
      const uint64_t hit = __ballot(lane < n_up_units && gu_list[min(lane, kFusedMaxPairs - 1)] == want);
      const int ug = __builtin_amdgcn_readfirstlane(hit ? __ffsll((unsigned long long)hit) - 1 : 0);
      const uint64_t* need = a.flags + ug * tg_up;
      const int tile0 = j * tpw_dn;
      auto wait_inputs = [&]() {
        if (wave == 0) wait_flags(need, tg_up, a.tag, a.status, a.fail_tag, a.spin_limit);
        lds_barrier();
      };
      gemv_unit<true, kSteps, true, kRingDn>(a.w_dn[e], a.b_dn, e, a.gated, plane, a.eo, nullptr, 0, nullptr,
                                    R.sorted + pb + tc, nt, dn_rows, a.inter / 32, 1, 0.0f, a.precision, tile0,
                                    min(tpw_dn, tiles_dn - tile0), xs, wait_inputs);
      publish(a.flags + a.max_up_items + d, a.tag);
    } else {
      // combine of rows [r0, r1) for every token, once this tile group's
      // down items are done: the multi-launch combine's operations, in its order
      const int j = item - n_up - n_dn;
      if (wave == 0) {
        const uint64_t* base = a.flags + a.max_up_items;
        const int lim = a.spin_limit;
        for (int it = 0;; ++it) {
          const bool done = lim >= 0 && (lane >= n_dn_units ||
                                         __hip_atomic_load(base + lane * tg_dn + j, __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT) == a.tag);
          if (__ballot(!done) == 0) break;
          if (it >= lim) {
            if (lane == 0) ran_out(a.status, a.fail_tag, a.tag);
            break;
          }
          __builtin_amdgcn_s_sleep(2);
        }
      }
      lds_barrier();
      // a wait of this launch that ran out before this point (the workgroup
      // that ran out records it before it publishes its flag) poisons this
      // tile group's outputs: NaN, with or without the residual
      const bool failed = launch_failed(a);
      const int r0 = j * tpw_dn * kTileRows;
      const int nq = (min(a.hidden, r0 + tpw_dn * kTileRows) - r0) >> 2;  // 4-output groups per token
      const __amdgpu_buffer_rsrc_t ebuf =
          __builtin_amdgcn_make_buffer_rsrc((void*)a.eo, (short)0, 0x7fffffff, kBufferWord3);
      for (int i = threadIdx.x; i < n_tok * nq; i += kFusedThreads) {
        const int t = i / nq;
        const int h = r0 + 4 * (i - t * nq);
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int j0 = 0; j0 < k; j0 += kCombineSlots) {
          // every slot's 16-byte load is in flight before the first is used
          u32x4_t v[kCombineSlots];
#pragma unroll
          for (int q = 0; q < kCombineSlots; ++q) {
            const int64_t p = (int64_t)t * k + min(j0 + q, k - 1);
            v[q] = __builtin_amdgcn_raw_buffer_load_b128(ebuf, (uint32_t)((p * a.hidden + h) * 4), 0, kAgentScope);
          }
#pragma unroll
          for (int q = 0; q < kCombineSlots; ++q) {
            if (j0 + q < k) {
              const float wj = bf16_to_f32(R.wts[t * k + j0 + q]);
#pragma unroll
              for (int r = 0; r < 4; ++r)
                acc[r] = round_bf16(acc[r] + round_bf16(round_bf16(__uint_as_float(v[q][r])) * wj));
            }
          }
        }
        if (a.residual != nullptr) {
          const uint2 rv = *reinterpret_cast<const uint2*>(a.residual + (int64_t)t * a.hidden + h);
          acc[0] = bf16_to_f32(rv.x & 0xffffu) + acc[0];
          acc[1] = bf16_to_f32(rv.x >> 16) + acc[1];
          acc[2] = bf16_to_f32(rv.y & 0xffffu) + acc[2];
          acc[3] = bf16_to_f32(rv.y >> 16) + acc[3];
        }
        const uint2 o = failed ? make_uint2(0x7fc07fc0u, 0x7fc07fc0u)
                               : make_uint2(f32_to_bf16_rne(acc[0]) | (f32_to_bf16_rne(acc[1]) << 16),
                                            f32_to_bf16_rne(acc[2]) | (f32_to_bf16_rne(acc[3]) << 16));
        *reinterpret_cast<uint2*>(a.out + (int64_t)t * a.hidden + h) = o;
      }
    }
  }
}

using FusedKernel = void (*)(FusedArgs);

FusedKernel fused_kernel_for(int steps) {
  switch (steps) {
    case 1: return moe_decode_fused_kernel<1>;
    case 2: return moe_decode_fused_kernel<2>;
    case 4: return moe_decode_fused_kernel<4>;
    case 8: return moe_decode_fused_kernel<8>;
    case 24: return moe_decode_fused_kernel<24>;
    default: return nullptr;
  }
}

// Resident workgroups of each instantiation, per device (the grid size).
constexpr int kMaxDevices = 64;
std::mutex g_grid_mutex;
int g_grid[kMaxDevices][25][2];  // [device][steps][n_exp > 128]

std::atomic<uint64_t> g_launches{0};

int fused_steps(int64_t hidden, int64_t inter) {
  const int su = gemv_steps((int)(hidden / 32)), sd = gemv_steps((int)(inter / 32));
  return su > sd ? su : sd;
}

}  // namespace

// Whether klc_moe_layer can run this batch as one launch: at most 16
// tokens, 64 pairs, 256 experts and k <= 16, 8-byte aligned out/residual,
// and a stream that is not capturing a graph.
bool fused_decode_supported(int64_t n_tok, int64_t hidden, int64_t inter, int64_t n_exp, int64_t k, const void* out,
                            const void* residual) {
  if (n_tok < 1 || n_tok > kFusedMaxTokens || n_tok * k > kFusedMaxPairs || n_exp > kFusedMaxExperts ||
      k > kFusedMaxK)
    return false;
  if (((uintptr_t)out & 7) != 0 || ((uintptr_t)residual & 7) != 0) return false;
  const int s = fused_steps(hidden, inter);
  return s > 0 && fused_kernel_for(s) != nullptr && hidden % 8 == 0;
}

// Workspace bytes of the fused layer's logit words, item flags and status word.
int64_t fused_decode_scratch_bytes(int64_t n_tok, int64_t hidden, int64_t inter, int64_t n_exp, int64_t k) {
  const int64_t pairs = n_tok * k;
  const int64_t words = n_exp * n_tok * 8;
  const int64_t flags = (units_capacity(pairs, n_exp, kUnitTokensGateUp) * (2 * inter / kTileRows) +
                         units_capacity(pairs, n_exp, kUnitTokensDown) * (hidden / kTileRows)) * 8;
  // flags, then the status word, 4 spare bytes and the failed launch's tag
  return ((words + 255) & ~(int64_t)255) + ((flags + 16 + 255) & ~(int64_t)255);
}

int launch_moe_decode_fused(const void* x, const void* router_w, const void* router_b, const void* const* w_gate_up,
                            const void* gate_up_bias, const void* const* w_down, const void* down_bias,
                            int64_t n_tok, int64_t hidden, int64_t inter, int64_t n_exp, int64_t k, float limit,
                            int precision, char* fused_ws, void* logits, int32_t* ids, float* values, void* weights,
                            void* gated, float* eo, void* out, const void* residual, hipStream_t stream) {
  const int steps = fused_steps(hidden, inter);
  const FusedKernel kern = fused_kernel_for(steps);
  KLC_REQUIRE(kern != nullptr, KLC_ERR_UNSUPPORTED, "fused decode: no kernel for %d steps", steps);
  const size_t lds = fused_lds_bytes(steps, (int)n_exp);
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  KLC_REQUIRE(err == hipSuccess && dev >= 0 && dev < kMaxDevices, KLC_ERR_HIP, "fused decode: hipGetDevice: %s",
              hipGetErrorString(err));
  int grid = 0;
  {
    std::lock_guard<std::mutex> lock(g_grid_mutex);
    int& g = g_grid[dev][steps][n_exp > 128 ? 1 : 0];
    if (g == 0) {
      int per_cu = 0, cus = 0;
      err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kern), kFusedThreads,
                                                         fused_lds_bytes(steps, n_exp > 128 ? kFusedMaxExperts : 128));
      KLC_REQUIRE(err == hipSuccess, KLC_ERR_HIP, "fused decode: occupancy: %s", hipGetErrorString(err));
      err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
      KLC_REQUIRE(err == hipSuccess, KLC_ERR_HIP, "fused decode: CU count: %s", hipGetErrorString(err));
      KLC_REQUIRE(per_cu >= 1 && cus >= 1, KLC_ERR_UNSUPPORTED, "fused decode: kernel does not fit a CU");
      g = per_cu * cus;
    }
    grid = g;
  }
  KLC_REQUIRE(grid >= 1, KLC_ERR_UNSUPPORTED, "fused decode: empty grid");
  const uint64_t tag = launch_tag(g_launches.fetch_add(1, std::memory_order_relaxed) + 1);

  const int64_t pairs = n_tok * k;
  const int64_t words_bytes = ((n_exp * n_tok * 8) + 255) & ~(int64_t)255;
  FusedArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.router_w = static_cast<const uint16_t*>(router_w);
  a.router_b = static_cast<const uint16_t*>(router_b);
  a.w_up = reinterpret_cast<const uint8_t* const*>(w_gate_up);
  a.b_up = static_cast<const uint16_t*>(gate_up_bias);
  a.w_dn = reinterpret_cast<const uint8_t* const*>(w_down);
  a.b_dn = static_cast<const uint16_t*>(down_bias);
  a.residual = static_cast<const uint16_t*>(residual);
  a.out = static_cast<uint16_t*>(out);
  a.ids = ids;
  a.weights = static_cast<uint16_t*>(weights);
  a.values = values;
  a.logits = static_cast<uint16_t*>(logits);
  a.words = reinterpret_cast<uint64_t*>(fused_ws);
  a.flags = reinterpret_cast<uint64_t*>(fused_ws + words_bytes);
  a.max_up_items = (int)(units_capacity(pairs, n_exp, kUnitTokensGateUp) * (2 * inter / kTileRows));
  const int64_t max_dn_items = units_capacity(pairs, n_exp, kUnitTokensDown) * (hidden / kTileRows);
  a.status = reinterpret_cast<uint32_t*>(a.flags + a.max_up_items + max_dn_items);
  a.fail_tag = reinterpret_cast<uint64_t*>(a.status + 2);
  a.gated = static_cast<uint16_t*>(gated);
  a.eo = eo;
  a.n_tok = (int)n_tok;
  a.hidden = (int)hidden;
  a.inter = (int)inter;
  a.n_exp = (int)n_exp;
  a.k = (int)k;
  a.precision = precision;
  a.limit = limit;
  a.tag = tag;
  // KLC_FUSED_SPIN_LIMIT overrides the polls a wait makes before it gives
  // up (a negative value: none; for tests of the failure path)
  a.spin_limit = kSpinLimit;
  if (const char* env = getenv("KLC_FUSED_SPIN_LIMIT")) a.spin_limit = atoi(env);
  kern<<<grid, kFusedThreads, lds, stream>>>(a);
  return check_launch("moe_decode_fused_kernel");
}

// Byte offset of the status word in the fused scratch: bit 0 set means a
// wait of some launch on this scratch ran out.
int64_t fused_decode_status_offset(int64_t n_tok, int64_t hidden, int64_t inter, int64_t n_exp, int64_t k) {
  const int64_t pairs = n_tok * k;
  const int64_t words_bytes = ((n_exp * n_tok * 8) + 255) & ~(int64_t)255;
  const int64_t flags = units_capacity(pairs, n_exp, kUnitTokensGateUp) * (2 * inter / kTileRows) +
                        units_capacity(pairs, n_exp, kUnitTokensDown) * (hidden / kTileRows);
  return words_bytes + flags * 8;
}

}  // namespace klc
