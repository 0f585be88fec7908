"""torch CPU kernels behind the reference's router — TEST INFRASTRUCTURE ONLY.

The reference selects experts with ``torch.topk(logits.float(), k)`` and
weights them with ``torch.softmax(fp32 scores).to(bf16)``
(streamed_moe_router.py:271-273, 281-282).  Both are torch CPU kernels whose
exact results (tie order, last-bit rounding) are not fixed by any
specification, so they are restated here step for step:

* ``topk_order`` — torch's CPU top-k loop (``topk_impl_loop``,
  ``torch/include/ATen/native/TopKImpl.h``, torch 2.10): (value, index)
  pairs are ordered with the comparator "greater, NaN largest"; for
  ``k * 64 <= n`` with ``std::partial_sort``, otherwise with
  ``std::nth_element`` at ``k - 1`` followed by ``std::sort`` of the first
  ``k - 1`` pairs.  torch is built with GCC 11's libstdc++; its algorithms
  (``bits/stl_algo.h``: ``__introselect``, ``__unguarded_partition_pivot``,
  ``__move_median_to_first``, ``__unguarded_partition``,
  ``__insertion_sort``, ``__introsort_loop``, ``__final_insertion_sort``,
  ``__heap_select``; ``bits/stl_heap.h``: ``__make_heap``, ``__adjust_heap``,
  ``__push_heap``, ``__pop_heap``, ``__sort_heap``) are restated below in the
  order they move elements, which is what decides the order of equal values.
* ``softmax_f32`` — torch's CPU softmax over the last dimension
  (``_vec_softmax_lastdim``): the maximum by sequential ``vec::maximum``
  (NaN propagates), ``exp(x - max)`` by ``Vectorized<float>::exp`` (SLEEF's
  ``expf`` with a 1.0-ulp bound, ``Sleef_expf16_u10``; restated in
  ``sleef_expf_u10``), the sum accumulated left to right in float32, one
  float32 reciprocal, and a float32 multiply per element.

Pinned in tests/test_oracle_torch_cpu.py directly against ``torch.topk`` and
``torch.softmax`` (torch is the reference's dependency and is importable in
the test environment) on tie-heavy and random inputs, and against the
committed golden vectors of tests/golden/.
"""

from __future__ import annotations

import numpy as np

# ---------------------------------------------------------------------------
# libstdc++ algorithms on a list `a` with a strict weak order `gt` ("greater")


def _lg(n: int) -> int:
    """std::__lg: floor(log2(n)) for n > 0."""
    return n.bit_length() - 1


def _move_median_to_first(a, result, i, j, m, gt):
    # __move_median_to_first(result, a=i, b=j, c=m)
    if gt(a[i], a[j]):
        if gt(a[j], a[m]):
            a[result], a[j] = a[j], a[result]
        elif gt(a[i], a[m]):
            a[result], a[m] = a[m], a[result]
        else:
            a[result], a[i] = a[i], a[result]
    elif gt(a[i], a[m]):
        a[result], a[i] = a[i], a[result]
    elif gt(a[j], a[m]):
        a[result], a[m] = a[m], a[result]
    else:
        a[result], a[j] = a[j], a[result]


def _unguarded_partition(a, first, last, pivot, gt):
    while True:
        while gt(a[first], a[pivot]):
            first += 1
        last -= 1
        while gt(a[pivot], a[last]):
            last -= 1
        if not first < last:
            return first
        a[first], a[last] = a[last], a[first]
        first += 1


def _unguarded_partition_pivot(a, first, last, gt):
    mid = first + (last - first) // 2
    _move_median_to_first(a, first, first + 1, mid, last - 1, gt)
    return _unguarded_partition(a, first + 1, last, first, gt)


def _unguarded_linear_insert(a, last, gt):
    val = a[last]
    nxt = last - 1
    while gt(val, a[nxt]):
        a[last] = a[nxt]
        last = nxt
        nxt -= 1
    a[last] = val


def _insertion_sort(a, first, last, gt):
    if first == last:
        return
    for i in range(first + 1, last):
        if gt(a[i], a[first]):
            val = a[i]
            a[first + 1:i + 1] = a[first:i]  # move_backward
            a[first] = val
        else:
            _unguarded_linear_insert(a, i, gt)


def _push_heap(a, base, hole, top, value, gt):
    parent = (hole - 1) // 2
    while hole > top and gt(a[base + parent], value):
        a[base + hole] = a[base + parent]
        hole = parent
        parent = (hole - 1) // 2
    a[base + hole] = value


def _adjust_heap(a, base, hole, length, value, gt):
    top = hole
    child = hole
    while child < (length - 1) // 2:
        child = 2 * (child + 1)
        if gt(a[base + child], a[base + child - 1]):
            child -= 1
        a[base + hole] = a[base + child]
        hole = child
    if (length & 1) == 0 and child == (length - 2) // 2:
        child = 2 * (child + 1)
        a[base + hole] = a[base + child - 1]
        hole = child - 1
    _push_heap(a, base, hole, top, value, gt)


def _make_heap(a, first, last, gt):
    length = last - first
    if length < 2:
        return
    parent = (length - 2) // 2
    while True:
        _adjust_heap(a, first, parent, length, a[first + parent], gt)
        if parent == 0:
            return
        parent -= 1


def _pop_heap(a, first, last, result, gt):
    value = a[result]
    a[result] = a[first]
    _adjust_heap(a, first, 0, last - first, value, gt)


def _sort_heap(a, first, last, gt):
    while last - first > 1:
        last -= 1
        _pop_heap(a, first, last, last, gt)


def _heap_select(a, first, middle, last, gt):
    _make_heap(a, first, middle, gt)
    for i in range(middle, last):
        if gt(a[i], a[first]):
            _pop_heap(a, first, middle, i, gt)


def stl_partial_sort(a, first, middle, last, gt):
    _heap_select(a, first, middle, last, gt)
    _sort_heap(a, first, middle, gt)


def stl_nth_element(a, first, nth, last, gt):
    if first == last or nth == last:
        return
    depth = _lg(last - first) * 2
    while last - first > 3:
        if depth == 0:
            _heap_select(a, first, nth + 1, last, gt)
            a[first], a[nth] = a[nth], a[first]
            return
        depth -= 1
        cut = _unguarded_partition_pivot(a, first, last, gt)
        if cut <= nth:
            first = cut
        else:
            last = cut
    _insertion_sort(a, first, last, gt)


_THRESHOLD = 16  # libstdc++ _S_threshold


def _introsort_loop(a, first, last, depth, gt):
    while last - first > _THRESHOLD:
        if depth == 0:
            stl_partial_sort(a, first, last, last, gt)
            return
        depth -= 1
        cut = _unguarded_partition_pivot(a, first, last, gt)
        _introsort_loop(a, cut, last, depth, gt)
        last = cut


def stl_sort(a, first, last, gt):
    if first == last:
        return
    _introsort_loop(a, first, last, _lg(last - first) * 2, gt)
    if last - first > _THRESHOLD:
        _insertion_sort(a, first, first + _THRESHOLD, gt)
        for i in range(first + _THRESHOLD, last):
            _unguarded_linear_insert(a, i, gt)
    else:
        _insertion_sort(a, first, last, gt)


# ---------------------------------------------------------------------------
# torch.topk on CPU


def order_key_bf16(bits) -> np.ndarray:
    """bfloat16 patterns -> integer keys with torch.topk's CPU comparator order.

    Larger key = "greater"; every NaN is the largest and NaNs are equal to one
    another; -0 equals +0.  (The comparator compares float values:
    ``isnan(x) && !isnan(y) || x > y``.)
    """
    u = np.asarray(bits, dtype=np.uint16).astype(np.int64)
    mag = u & 0x7FFF
    key = np.where(u & 0x8000, 0x8000 - mag, 0x8000 + mag)
    key = np.where(mag == 0, 0x8000, key)
    return np.where(mag > 0x7F80, 0x10000, key)


def topk_order(keys, k: int) -> list[int]:
    """Indices torch.topk(x, k) (largest, sorted) returns on CPU for one row.

    ``keys`` are comparator-ordered integers (``order_key_bf16``); ties keep
    whatever order libstdc++'s algorithms leave them in (TopKImpl.h).
    """
    n = len(keys)
    k = int(k)
    if k == 0:
        return []
    q = [(int(keys[j]), j) for j in range(n)]

    def gt(x, y):
        return x[0] > y[0]

    if k * 64 <= n:
        stl_partial_sort(q, 0, k, n, gt)
    else:
        stl_nth_element(q, 0, k - 1, n, gt)
        stl_sort(q, 0, k - 1, gt)
    return [q[j][1] for j in range(k)]


# ---------------------------------------------------------------------------
# float32 arithmetic with one rounding, and torch's CPU softmax


def fma_f32(a, b, c) -> np.ndarray:
    """Correctly rounded float32 a * b + c (IEEE fusedMultiplyAdd).

    The float32 product is exact in float64; the float64 sum ``s`` and its
    exact error ``e`` (TwoSum) give a * b + c = s + e exactly.  Rounding ``s``
    to float32 is then correct unless ``s`` lies exactly halfway between two
    float32 values, where the sign of ``e`` decides.
    """
    a = np.asarray(a, np.float32).astype(np.float64)
    b = np.asarray(b, np.float32).astype(np.float64)
    c = np.asarray(c, np.float32).astype(np.float64)
    p = a * b
    s = p + c
    bb = s - p
    e = (p - (s - bb)) + (c - bb)
    with np.errstate(over="ignore", invalid="ignore"):
        r = s.astype(np.float32)
        r64 = r.astype(np.float64)
        up = np.nextafter(r, np.float32(np.inf))
        down = np.nextafter(r, np.float32(-np.inf))
        hi = np.where(r64 < s, up, r)  # the float32 neighbours of s
        lo = np.where(r64 < s, r, down)
        halfway = np.isfinite(s) & (s != r64) & ((s - lo.astype(np.float64)) == (hi.astype(np.float64) - s))
        r = np.where(halfway & (e > 0), hi, np.where(halfway & (e < 0), lo, r))
    return np.where(np.isfinite(s), r, s.astype(np.float32)).astype(np.float32)


# SLEEF single-precision exp, 1.0-ulp variant (Sleef_expf_u10; sleefsimdsp.c
# xexpf): Cody-Waite reduction by ln 2 in two parts, a degree-6 polynomial
# evaluated with FMA, and a scale by 2^q in two halves.
_R_LN2F = np.float32(1.442695040888963407359924681001892137426645954152985934135449406931)
_L2UF = np.float32(0.693145751953125)
_L2LF = np.float32(1.428606765330187045e-06)
_EXPF_POLY = [np.float32(v) for v in (
    0.000198527617612853646278381,
    0.00139304355252534151077271,
    0.00833336077630519866943359,
    0.0416664853692054748535156,
    0.166666671633720397949219,
    0.5,
)]


def _pow2i(q: np.ndarray) -> np.ndarray:
    return ((q.astype(np.int64) + 0x7F) << 23).astype(np.uint32).view(np.float32)


def sleef_expf_u10(d) -> np.ndarray:
    d = np.asarray(d, dtype=np.float32)
    with np.errstate(over="ignore", invalid="ignore", under="ignore"):
        q = np.rint(d * _R_LN2F).astype(np.float32)
        q = np.where(np.isfinite(q), q, np.float32(0))
        qi = q.astype(np.int64)
        s = fma_f32(q, -_L2UF, d)
        s = fma_f32(q, -_L2LF, s)
        u = np.full_like(d, _EXPF_POLY[0])
        for c in _EXPF_POLY[1:]:
            u = fma_f32(u, s, c)
        u = np.float32(1.0) + fma_f32((s * s).astype(np.float32), u, s)
        u = (u * _pow2i(qi >> 1)).astype(np.float32)
        u = (u * _pow2i(qi - (qi >> 1))).astype(np.float32)
        u = np.where(d < np.float32(-104), np.float32(0), u)
        u = np.where(np.float32(100) < d, np.float32(np.inf), u)
        u = np.where(np.isnan(d), np.float32(np.nan), u)
    return u.astype(np.float32)


def softmax_f32(values) -> np.ndarray:
    """torch.softmax(x, dim=-1) for float32 rows on CPU (_vec_softmax_lastdim)."""
    v = np.atleast_2d(np.asarray(values, dtype=np.float32))
    out = np.empty_like(v)
    for r in range(v.shape[0]):
        row = v[r]
        mx = row[0]
        for x in row[1:]:
            mx = np.float32(np.nan) if (np.isnan(mx) or np.isnan(x)) else max(mx, x)
        with np.errstate(invalid="ignore", over="ignore"):
            e = sleef_expf_u10((row - mx).astype(np.float32))
            s = e[0]
            for x in e[1:]:
                s = np.float32(s + x)
            inv = np.float32(np.float32(1.0) / s)
            out[r] = (e * inv).astype(np.float32)
    return out
