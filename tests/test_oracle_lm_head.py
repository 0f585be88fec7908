"""The lm_head oracle pinned without restating it: exact integer cases, the
float32 error bound of any summation order, and torch's own nan_to_num and
argmax (the functions the reference's callers use) on crafted vectors."""

from __future__ import annotations

import numpy as np
import torch

from oracle import lm_head as olm
from oracle.numerics import f32_to_bf16


def test_integer_dot_products_are_exact():
    rng = np.random.default_rng(1)
    w = rng.integers(-8, 9, (300, 64)).astype(np.float32)
    x = rng.integers(-100, 101, 64).astype(np.float32)
    got = olm.logits(f32_to_bf16(w), x, chunk_rows=128)
    assert np.array_equal(got, (w.astype(np.int64) @ x.astype(np.int64)).astype(np.float32))


def test_within_float32_summation_bound_of_torch():
    """Any float32 summation order lies within H * 2^-24 * sum|w x| of the
    exact dot product; the oracle is the exact value rounded once."""
    rng = np.random.default_rng(2)
    wf = rng.standard_normal((513, 2880)).astype(np.float32)
    w_bits = f32_to_bf16(wf)
    x = rng.standard_normal(2880).astype(np.float32)
    got = olm.logits(w_bits, x, chunk_rows=100)
    wt = torch.from_numpy(w_bits.view(np.int16)).view(torch.bfloat16)
    ref = torch.matmul(wt.float(), torch.from_numpy(x)).numpy()
    wd = np.asarray(wt.float().numpy(), dtype=np.float64)
    bound = 2880 * 2.0 ** -24 * (np.abs(wd) @ np.abs(x.astype(np.float64)))
    assert (np.abs(got.astype(np.float64) - ref) <= bound).all()
    exact = wd @ x.astype(np.float64)
    assert (np.abs(got.astype(np.float64) - exact) <= np.spacing(np.abs(got)).astype(np.float64) / 2 * 1.0001).all()


def test_nan_to_num_and_first_index_argmax_match_torch():
    cases = [
        np.array([1.0, 3.0, 3.0, -2.0], np.float32),                    # tie: first index
        np.array([np.nan, -5e9, -1e9, -2e9], np.float32),               # nan -> -1e9 ties with -1e9 (index 0 first)
        np.array([2e9, np.inf, 5.0], np.float32),                       # +inf -> 1e9 ranks below 2e9
        np.array([-np.inf, -np.inf, np.nan], np.float32),               # all map to -1e9: index 0
        np.array([-0.0, 0.0, -0.0], np.float32),                        # signed zeros compare equal
        np.array([np.float32(-3.4e38), np.float32(-3.3e38)], np.float32),
    ]
    for v in cases:
        t = torch.nan_to_num(torch.from_numpy(v), nan=-1e9, posinf=1e9, neginf=-1e9)
        assert np.array_equal(olm.nan_to_num(v), t.numpy())
        assert olm.greedy_token(v) == int(torch.argmax(t).item())
