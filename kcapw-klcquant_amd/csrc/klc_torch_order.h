// Exact torch CPU semantics of the router's selection and weights (gfx950 and
// host).
//
// The reference picks experts with torch.topk(logits.float(), k) and weights
// them with torch.softmax(values).to(bf16) (streamed_moe_router.py:271-273,
// 281-282).  On the CPU, torch's top-k (ATen/native/TopKImpl.h,
// topk_impl_loop) orders (value, index) pairs with the comparator "greater,
// NaN largest" using libstdc++: std::nth_element at k - 1 then std::sort of
// the first k - 1 pairs, or std::partial_sort when k * 64 <= n.  Equal
// values therefore come out in whatever order those algorithms leave them.
// This header restates the algorithms (GCC libstdc++ bits/stl_algo.h and
// bits/stl_heap.h: introselect with median-of-three pivots and the unguarded
// Hoare partition, insertion sort, introsort, heap select / sort_heap) on an
// array of 32-bit entries (comparator key << 16 | index), sequentially; the
// router's kernel runs the partition steps of the introselect wave-parallel
// and these sequential pieces in one lane, on the rare rows with ties.
//
// torch's softmax over the last dimension (_vec_softmax_lastdim) is float32:
// max by sequential vec::maximum (NaN propagates), exp(x - max) by
// Vectorized<float>::exp (SLEEF's 1.0-ulp expf, restated in sleef_expf_u10),
// the sum accumulated left to right, one reciprocal, one multiply each.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace klc {

// Comparator key of a bfloat16 logit: larger key = larger value; every NaN is
// the largest and NaNs equal each other; -0 equals +0.
__host__ __device__ __forceinline__ uint32_t order_key16(uint32_t bf16) {
  const uint32_t mag = bf16 & 0x7fffu;
  if (mag > 0x7f80u) return 0xffffu;
  if (mag == 0u) return 0x8000u;
  return (bf16 & 0x8000u) ? 0x8000u - mag : 0x8000u + mag;
}
__host__ __device__ __forceinline__ uint32_t order_entry(uint32_t bf16, int idx) {
  return (order_key16(bf16) << 16) | (uint32_t)idx;
}
// comp(x, y) of TopKImpl.h for largest = true
__host__ __device__ __forceinline__ bool entry_gt(uint32_t x, uint32_t y) { return (x >> 16) > (y >> 16); }
__host__ __device__ __forceinline__ void entry_swap(uint32_t* a, int i, int j) {
  const uint32_t t = a[i];
  a[i] = a[j];
  a[j] = t;
}

__host__ __device__ __forceinline__ int floor_log2(int n) {
  int l = 0;
  while (n > 1) {
    n >>= 1;
    ++l;
  }
  return l;
}

// __move_median_to_first(result, a, b, c)
__host__ __device__ __forceinline__ void stl_move_median_to_first(uint32_t* v, int result, int a, int b, int c) {
  if (entry_gt(v[a], v[b])) {
    if (entry_gt(v[b], v[c])) entry_swap(v, result, b);
    else if (entry_gt(v[a], v[c])) entry_swap(v, result, c);
    else entry_swap(v, result, a);
  } else if (entry_gt(v[a], v[c])) {
    entry_swap(v, result, a);
  } else if (entry_gt(v[b], v[c])) {
    entry_swap(v, result, c);
  } else {
    entry_swap(v, result, b);
  }
}

// __unguarded_partition(first, last, pivot)
__host__ __device__ __forceinline__ int stl_unguarded_partition(uint32_t* v, int first, int last, int pivot) {
  const uint32_t p = v[pivot];
  while (true) {
    while (entry_gt(v[first], p)) ++first;
    --last;
    while (entry_gt(p, v[last])) --last;
    if (!(first < last)) return first;
    entry_swap(v, first, last);
    ++first;
  }
}

__host__ __device__ __forceinline__ int stl_unguarded_partition_pivot(uint32_t* v, int first, int last) {
  const int mid = first + (last - first) / 2;
  stl_move_median_to_first(v, first, first + 1, mid, last - 1);
  return stl_unguarded_partition(v, first + 1, last, first);
}

__host__ __device__ __forceinline__ void stl_unguarded_linear_insert(uint32_t* v, int last) {
  const uint32_t val = v[last];
  int next = last - 1;
  while (entry_gt(val, v[next])) {
    v[last] = v[next];
    last = next;
    --next;
  }
  v[last] = val;
}

__host__ __device__ __forceinline__ void stl_insertion_sort(uint32_t* v, int first, int last) {
  if (first == last) return;
  for (int i = first + 1; i < last; ++i) {
    if (entry_gt(v[i], v[first])) {
      const uint32_t val = v[i];
      for (int j = i; j > first; --j) v[j] = v[j - 1];  // move_backward
      v[first] = val;
    } else {
      stl_unguarded_linear_insert(v, i);
    }
  }
}

// heap algorithms on v[base .. base + len)
__host__ __device__ __forceinline__ void stl_push_heap(uint32_t* v, int base, int hole, int top, uint32_t value) {
  int parent = (hole - 1) / 2;
  while (hole > top && entry_gt(v[base + parent], value)) {
    v[base + hole] = v[base + parent];
    hole = parent;
    parent = (hole - 1) / 2;
  }
  v[base + hole] = value;
}

__host__ __device__ __forceinline__ void stl_adjust_heap(uint32_t* v, int base, int hole, int len, uint32_t value) {
  const int top = hole;
  int child = hole;
  while (child < (len - 1) / 2) {
    child = 2 * (child + 1);
    if (entry_gt(v[base + child], v[base + child - 1])) --child;
    v[base + hole] = v[base + child];
    hole = child;
  }
  if ((len & 1) == 0 && child == (len - 2) / 2) {
    child = 2 * (child + 1);
    v[base + hole] = v[base + child - 1];
    hole = child - 1;
  }
  stl_push_heap(v, base, hole, top, value);
}

__host__ __device__ __forceinline__ void stl_make_heap(uint32_t* v, int first, int last) {
  const int len = last - first;
  if (len < 2) return;
  for (int parent = (len - 2) / 2;; --parent) {
    stl_adjust_heap(v, first, parent, len, v[first + parent]);
    if (parent == 0) return;
  }
}

__host__ __device__ __forceinline__ void stl_pop_heap(uint32_t* v, int first, int last, int result) {
  const uint32_t value = v[result];
  v[result] = v[first];
  stl_adjust_heap(v, first, 0, last - first, value);
}

__host__ __device__ __forceinline__ void stl_heap_select(uint32_t* v, int first, int middle, int last) {
  stl_make_heap(v, first, middle);
  for (int i = middle; i < last; ++i)
    if (entry_gt(v[i], v[first])) stl_pop_heap(v, first, middle, i);
}

__host__ __device__ __forceinline__ void stl_partial_sort(uint32_t* v, int first, int middle, int last) {
  stl_heap_select(v, first, middle, last);
  for (int l = middle; l - first > 1;) {  // __sort_heap
    --l;
    stl_pop_heap(v, first, l, l);
  }
}

// std::sort (introsort + final insertion sort, threshold 16) for ranges of
// at most 33 entries (the router sorts k - 1 <= 31).  __introsort_loop
// partitions [f, l) at `cut`, recurses into [cut, l) and loops on [f, cut)
// with the same depth budget; the two ranges are disjoint, and for at most
// 33 entries only one of them can hold more than 16, so following that one
// alone does what the recursion does, without a stack.
__host__ __device__ __forceinline__ void stl_sort(uint32_t* v, int first, int last) {
  if (first == last) return;
  constexpr int kThreshold = 16;
  int f = first, l = last, d = floor_log2(last - first) * 2;
  while (l - f > kThreshold) {
    if (d == 0) {
      stl_partial_sort(v, f, l, l);
      break;
    }
    --d;
    const int cut = stl_unguarded_partition_pivot(v, f, l);
    if (l - cut > kThreshold) f = cut;
    else l = cut;
  }
  if (last - first > kThreshold) {
    stl_insertion_sort(v, first, first + kThreshold);
    for (int i = first + kThreshold; i < last; ++i) stl_unguarded_linear_insert(v, i);
  } else {
    stl_insertion_sort(v, first, last);
  }
}

// std::nth_element(first, nth, last), sequential (the host restatement of
// what the router kernel runs with its partitions spread over a wave).
__host__ __device__ __forceinline__ void stl_nth_element(uint32_t* v, int first, int nth, int last) {
  if (first == last || nth == last) return;
  int depth = floor_log2(last - first) * 2;
  while (last - first > 3) {
    if (depth == 0) {
      stl_heap_select(v, first, nth + 1, last);
      entry_swap(v, first, nth);
      return;
    }
    --depth;
    const int cut = stl_unguarded_partition_pivot(v, first, last);
    if (cut <= nth) first = cut;
    else last = cut;
  }
  stl_insertion_sort(v, first, last);
}

// torch.topk(x, k) (largest, sorted) on CPU: v[0 .. k) ends as the result.
__host__ __device__ __forceinline__ void torch_topk_order(uint32_t* v, int n, int k) {
  if (k <= 0) return;
  if (k * 64 <= n) {
    stl_partial_sort(v, 0, k, n);
  } else {
    stl_nth_element(v, 0, k - 1, n);
    stl_sort(v, 0, k - 1);
  }
}

// ---- softmax ---------------------------------------------------------------

// SLEEF expf, 1.0-ulp variant (xexpf of sleefsimdsp.c, as
// Vectorized<float>::exp evaluates it with FMA): q = rint(d / ln 2); s = d -
// q ln 2 in two FMA steps (ln 2 split as 0.693145751953125 +
// 1.428606765330187045e-06); a degree-6 polynomial in s by FMA;
// u = 1 + (s^2 u + s); scaled by 2^(q >> 1) and 2^(q - (q >> 1)).
__host__ __device__ __forceinline__ float pow2i_f32(int q) {
  const uint32_t bits = (uint32_t)(q + 0x7f) << 23;
  float f;
  __builtin_memcpy(&f, &bits, 4);
  return f;
}

__host__ __device__ __forceinline__ float sleef_expf_u10(float d) {
#pragma clang fp contract(off)
  float q = __builtin_rintf(d * 1.442695040888963407359924681001892137426645954152985934135449406931f);
  q = q > 200.0f ? 200.0f : (q < -200.0f ? -200.0f : q);  // NaN stays NaN; outside this range d is saturated below
  const int qi = q == q ? (int)q : 0;
  float s = __builtin_fmaf(q, -0.693145751953125f, d);
  s = __builtin_fmaf(q, -1.428606765330187045e-06f, s);
  float u = 0.000198527617612853646278381f;
  u = __builtin_fmaf(u, s, 0.00139304355252534151077271f);
  u = __builtin_fmaf(u, s, 0.00833336077630519866943359f);
  u = __builtin_fmaf(u, s, 0.0416664853692054748535156f);
  u = __builtin_fmaf(u, s, 0.166666671633720397949219f);
  u = __builtin_fmaf(u, s, 0.5f);
  const float ss = s * s;
  u = 1.0f + __builtin_fmaf(ss, u, s);
  u = u * pow2i_f32(qi >> 1);
  u = u * pow2i_f32(qi - (qi >> 1));
  if (d < -104.0f) u = 0.0f;
  if (100.0f < d) u = __builtin_inff();
  if (d != d) u = d;
  return u;
}

// vec::maximum: NaN if either operand is NaN, else the larger.
__host__ __device__ __forceinline__ float torch_vec_max(float a, float b) {
  if (a != a || b != b) return __builtin_nanf("");
  return a > b ? a : b;
}

}  // namespace klc
