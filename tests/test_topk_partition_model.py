"""The router kernel's wave-parallel form of libstdc++'s partition step.

csrc/klc_router.hip runs each ``__unguarded_partition`` of the
introselect as one wave step instead of two scanning pointers: with pivot
``P`` at ``first`` and the range ``[first + 1, last)``, the left scan stops
at the positions ``L`` holding a value not greater than ``P`` (ascending),
the right scan at the positions ``R`` holding a value not less than ``P``
(descending, then ``first`` itself).  The i-th swap exchanges ``L[i]`` and
``R[i]`` while ``L[i] < R[i]``; with ``m`` swaps the returned cut is
``L[0]`` if ``m == 0``, else ``min(L[m], R[m - 1])`` (``R[m - 1]`` if ``L``
is used up).  This model of that rule must leave every array exactly as the
sequential restatement of libstdc++ (oracle/torch_cpu.py) does.
"""

from __future__ import annotations

import numpy as np

from oracle import torch_cpu


def gt(x, y):
    return x[0] > y[0]


def wave_partition(a, first, last):
    """The list form of __unguarded_partition(first + 1, last, pivot=first)."""
    p = a[first][0]
    pos = range(first + 1, last)
    L = [q for q in pos if not a[q][0] > p]
    R = [q for q in reversed(pos) if not p > a[q][0]] + [first]
    m = 0
    while m < min(len(L), len(R)) and L[m] < R[m]:
        m += 1
    for i in range(m):
        a[L[i]], a[R[i]] = a[R[i]], a[L[i]]
    if m == 0:
        return L[0]
    if m < len(L):
        return min(L[m], R[m - 1])
    return R[m - 1]


def wave_nth_element(a, nth):
    first, last = 0, len(a)
    depth = torch_cpu._lg(last) * 2
    while last - first > 3:
        if depth == 0:
            torch_cpu._heap_select(a, first, nth + 1, last, gt)
            a[first], a[nth] = a[nth], a[first]
            return
        depth -= 1
        mid = first + (last - first) // 2
        torch_cpu._move_median_to_first(a, first, first + 1, mid, last - 1, gt)
        cut = wave_partition(a, first, last)
        if cut <= nth:
            first = cut
        else:
            last = cut
    torch_cpu._insertion_sort(a, first, last, gt)


def test_wave_partition_equals_sequential_partition():
    rng = np.random.default_rng(21)
    for _ in range(4000):
        n = int(rng.integers(4, 200))
        vals = rng.integers(0, int(rng.integers(1, 12)), n)
        a = [(int(v), j) for j, v in enumerate(vals)]
        b = list(a)
        mid = n // 2
        torch_cpu._move_median_to_first(a, 0, 1, mid, n - 1, gt)
        torch_cpu._move_median_to_first(b, 0, 1, mid, n - 1, gt)
        cut_seq = torch_cpu._unguarded_partition(a, 1, n, 0, gt)
        cut_wave = wave_partition(b, 0, n)
        assert cut_seq == cut_wave and a == b


def test_wave_nth_element_equals_libstdcxx():
    rng = np.random.default_rng(22)
    for _ in range(3000):
        n = int(rng.integers(1, 300))
        k = int(rng.integers(1, min(n, 32) + 1))
        vals = rng.integers(0, int(rng.integers(1, 10)), n)
        a = [(int(v), j) for j, v in enumerate(vals)]
        b = list(a)
        torch_cpu.stl_nth_element(a, 0, k - 1, n, gt)
        if n > 0:
            wave_nth_element(b, k - 1)
        assert a == b


def test_swap_count_from_prefix_counts():
    """The kernel finds the swap count without building the lists: with A(q) the left stops below
    position q and B(q) the right stops at or above q (pivot excluded), m = max over q of
    min(A(q), B(q)); the cut and the partner of each stop follow from the ranks."""
    rng = np.random.default_rng(23)
    for _ in range(4000):
        n = int(rng.integers(4, 260))
        vals = rng.integers(0, int(rng.integers(1, 12)), n)
        first = 0
        p = vals[first]
        pos = range(first + 1, n)
        L = [q for q in pos if not vals[q] > p]
        R = [q for q in reversed(pos) if not p > vals[q]]
        m_lists = 0
        while m_lists < min(len(L), len(R)) and L[m_lists] < R[m_lists]:
            m_lists += 1
        a = [sum(1 for x in L if x < q) for q in range(n + 1)]
        b = [sum(1 for x in R if x >= q) for q in range(n + 1)]
        assert max(min(a[q], b[q]) for q in range(first + 1, n + 1)) == m_lists


def test_swap_count_from_right_stops_above():
    """The kernel's form: the i-th left stop x (ascending) swaps while at least i + 1 right stops lie
    strictly above x, so m is the number of left stops with that property (they form a prefix)."""
    rng = np.random.default_rng(24)
    for _ in range(4000):
        n = int(rng.integers(4, 260))
        vals = rng.integers(0, int(rng.integers(1, 12)), n)
        p = vals[0]
        pos = range(1, n)
        L = [q for q in pos if not vals[q] > p]
        R = [q for q in reversed(pos) if not p > vals[q]]
        m_lists = 0
        while m_lists < min(len(L), len(R)) and L[m_lists] < R[m_lists]:
            m_lists += 1
        flags = [sum(1 for y in R if y > x) >= i + 1 for i, x in enumerate(L)]
        assert sum(flags) == m_lists
        assert flags == sorted(flags, reverse=True)  # a prefix of L
