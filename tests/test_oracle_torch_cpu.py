"""Pins oracle/torch_cpu.py against the torch CPU kernels it restates.

torch is the reference's own dependency for this arithmetic
(streamed_moe_router.py:271-273, 281-282) and is importable on the CPU, so
``torch.topk`` and ``torch.softmax`` themselves are the checkers here.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

from oracle import router, torch_cpu
from oracle.numerics import f32_to_bf16

torch = pytest.importorskip("torch")


def torch_topk(vals_f32: np.ndarray, k: int) -> list[int]:
    return torch.topk(torch.from_numpy(np.ascontiguousarray(vals_f32, np.float32)), k).indices.tolist()


def bf16_rows(vals: np.ndarray) -> np.ndarray:
    return f32_to_bf16(np.asarray(vals, np.float32))


def test_topk_matches_torch_on_tie_heavy_rows():
    rng = np.random.default_rng(7)
    for _ in range(1500):
        n = int(rng.integers(1, 260))
        k = int(rng.integers(1, min(n, 32) + 1))
        vals = rng.integers(0, int(rng.integers(1, 9)), n).astype(np.float32) - 3.0
        if rng.random() < 0.25:
            vals[rng.integers(0, n, 3)] = np.nan
        if rng.random() < 0.25:
            vals[rng.integers(0, n, 4)] = rng.choice([0.0, -0.0])
        bits = bf16_rows(vals)
        assert torch_cpu.topk_order(torch_cpu.order_key_bf16(bits), k) == torch_topk(vals, k), (n, k, vals.tolist())


def test_topk_matches_torch_in_the_partial_sort_regime():
    # k * 64 <= n switches torch to std::partial_sort (heap select + sort_heap)
    rng = np.random.default_rng(8)
    for n in (64, 128, 256, 300, 512, 1024):
        for k in (1, 2, 4, 8, 16):
            if k * 64 > n:
                continue
            for levels in (2, 5, 40):
                vals = rng.integers(0, levels, n).astype(np.float32)
                vals[rng.integers(0, n, 2)] = np.nan
                assert torch_cpu.topk_order(torch_cpu.order_key_bf16(bf16_rows(vals)), k) == torch_topk(vals, k)


def test_topk_matches_torch_on_router_like_rows():
    # bf16 logits of N(0, 0.3): ties at the top-k boundary are common
    rng = np.random.default_rng(9)
    for n in (32, 128, 256):
        vals = (rng.standard_normal((400, n)) * 0.3).astype(np.float32)
        bits = bf16_rows(vals)
        f = (bits.astype(np.uint32) << 16).view(np.float32)
        ids, _ = router.topk(bits, 4)
        for r in range(vals.shape[0]):
            assert ids[r].tolist() == torch_topk(f[r], 4)


def _mcilroy_killer(n: int, nth: int) -> np.ndarray:
    """Values that drive libstdc++'s introselect to its depth limit (McIlroy's
    adaptive adversary: undecided values are "gas" and are frozen, smallest
    first, only as comparisons force it)."""
    gas = n
    val = [gas] * n
    state = {"solid": 0, "cand": -1}

    def freeze(i):
        val[i] = state["solid"]
        state["solid"] += 1

    def gt(x, y):
        i, j = x[1], y[1]
        if val[i] == gas and val[j] == gas:
            freeze(i if i == state["cand"] else j)
        if val[i] == gas:
            state["cand"] = i
        elif val[j] == gas:
            state["cand"] = j
        return val[i] > val[j]

    q = [(0, j) for j in range(n)]
    torch_cpu.stl_nth_element(q, 0, nth, n, gt)
    out = np.array(val, dtype=np.float64)
    out[out == gas] = n + np.arange(int((out == gas).sum()))
    return out


def test_topk_matches_torch_past_the_introselect_depth_limit():
    hit = 0
    for n in (40, 100, 128, 200):
        base = _mcilroy_killer(n, 3)
        for coarse in (1, 2, 3):
            bits = bf16_rows(np.floor(base / coarse))
            vals = (bits.astype(np.uint32) << 16).view(np.float32)  # the bf16 values both sides see
            keys = torch_cpu.order_key_bf16(bits)
            # does the oracle reach __heap_select?  (count it through a wrapped helper)
            calls = []
            orig = torch_cpu._heap_select
            torch_cpu._heap_select = lambda *a, **kw: (calls.append(1), orig(*a, **kw))
            try:
                got = torch_cpu.topk_order(keys, 4)
            finally:
                torch_cpu._heap_select = orig
            hit += bool(calls)
            assert got == torch_topk(vals, 4), (n, coarse)
    assert hit >= 4  # the adversarial rows do take the heap-select branch


def test_softmax_matches_torch_bit_for_bit():
    rng = np.random.default_rng(10)
    rows = []
    for _ in range(3000):
        k = int(rng.integers(1, 9))
        rows.append((rng.standard_normal(k) * rng.choice([0.05, 0.5, 2.0, 20.0])).astype(np.float32))
    for row in rows:
        want = torch.softmax(torch.from_numpy(row), dim=-1).numpy()
        got = torch_cpu.softmax_f32(row)[0]
        assert np.array_equal(want.view(np.uint32), got.view(np.uint32)), row
    # a float64 softmax rounded once differs from torch's float32 kernel in the last bit often:
    # the test above discriminates between the two
    v = np.stack([r for r in rows if r.size == 4])
    v64 = v.astype(np.float64)
    e = np.exp(v64 - v64.max(1, keepdims=True))
    alt = (e / e.sum(1, keepdims=True)).astype(np.float32)
    assert np.count_nonzero(alt != torch_cpu.softmax_f32(v)) > v.size // 10


def test_softmax_special_values_match_torch():
    cases = [[0.0], [np.nan, 1.0], [np.inf, 1.0], [-np.inf, 0.0, 1.0], [-200.0, 0.0], [88.0, -88.0, 0.0, 3.0],
             [-110.0, 0.0], [1e-30, -1e-30]]
    for c in cases:
        row = np.array(c, np.float32)
        want = torch.softmax(torch.from_numpy(row), dim=-1).numpy()
        got = torch_cpu.softmax_f32(row)[0]
        assert np.array_equal(np.isnan(want), np.isnan(got)), c
        assert np.array_equal(np.nan_to_num(want).view(np.uint32), np.nan_to_num(got).view(np.uint32)), c


def test_fma_f32_is_correctly_rounded():
    rng = np.random.default_rng(11)
    a = rng.standard_normal(400).astype(np.float32)
    b = rng.standard_normal(400).astype(np.float32)
    c = rng.standard_normal(400).astype(np.float32) * np.float32(1e-3)
    # halfway cases: a*b lands exactly between two float32 values and c nudges it
    a[:50] = np.float32(1.0 + 2.0 ** -12)
    b[:50] = np.float32(1.0 + 2.0 ** -12)  # exact product 1 + 2^-11 + 2^-24: a float32 midpoint
    c[:25] = np.float32(2.0 ** -60)
    c[25:50] = np.float32(-(2.0 ** -60))
    got = torch_cpu.fma_f32(a, b, c)
    for i in range(a.size):
        exact = Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i]))
        lo = np.float32(float(exact))  # a candidate; compare distances exactly
        cands = [np.nextafter(lo, np.float32(-np.inf)), lo, np.nextafter(lo, np.float32(np.inf))]
        dists = [abs(Fraction(float(x)) - exact) for x in cands]
        best = min(dists)
        winners = [x for x, d in zip(cands, dists) if d == best]
        if len(winners) > 1:  # exact tie: even significand
            winners = [x for x in winners if (int(np.float32(x).view(np.uint32)) & 1) == 0]
        assert got[i] == winners[0], i
