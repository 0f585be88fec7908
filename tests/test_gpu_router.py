"""GPU parity: router logits, top-k/softmax and dispatch against the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor
from klcquant_amd import ops, synth
from oracle import router as orr
from oracle.numerics import f32_to_bf16

pytestmark = pytest.mark.gpu


def router_inputs(seed, n_tok, hidden, n_exp):
    x = synth.random_normal_bf16(seed + 1, n_tok * hidden).reshape(n_tok, hidden)
    w = synth.random_normal_bf16(seed + 2, n_exp * hidden, 0.0, 0.02).reshape(n_exp, hidden)
    b = synth.random_normal_bf16(seed + 3, n_exp, 0.0, 0.01)
    return x, w, b


@pytest.mark.parametrize("n_tok,hidden,n_exp", [(1, 2880, 32), (64, 2880, 128), (13, 2880, 128), (5, 104, 7),
                                                (9, 64, 1024), (17, 4096, 5)])
def test_logits_bit_exact(gpu, n_tok, hidden, n_exp):
    x, w, b = router_inputs(100 + n_tok, n_tok, hidden, n_exp)
    logits, x_f32 = ops.router_logits(bf16_tensor(x, gpu), bf16_tensor(w, gpu), bf16_tensor(b, gpu), want_f32=True)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(logits), orr.router_logits(x, w, b))
    assert np.array_equal(x_f32.cpu().numpy(), (x.astype(np.uint32) << 16).view(np.float32))


def test_topk_on_gpu_logits_bit_exact_and_softmax(gpu):
    n_tok, hidden, n_exp, k = 2048, 2880, 128, 4
    x, w, b = router_inputs(7, n_tok, hidden, n_exp)
    logits = ops.router_logits(bf16_tensor(x, gpu), bf16_tensor(w, gpu), bf16_tensor(b, gpu))
    ids, values, weights = ops.topk_softmax(logits, k)
    torch.cuda.synchronize()
    lb = bf16_bits(logits)
    want_ids, want_vals = orr.topk(lb, k)
    assert np.array_equal(ids.cpu().numpy(), want_ids)
    assert np.array_equal(values.cpu().numpy(), want_vals)
    assert np.array_equal(bf16_bits(weights), orr.softmax_weights(want_vals))
    # this input has boundary ties (4th == 5th logit); the tie rule decides them
    srt = -np.sort(-(lb.astype(np.uint32) << 16).view(np.float32), axis=1)
    assert (srt[:, k - 1] == srt[:, k]).sum() > 0


def test_topk_ties_nan_and_signed_zero(gpu):
    f = np.array([[0, 2, 1, 2, 2, 3, 2, 0, 0, 0],
                  [-0.0, 0.0, -1, -1, -2, -3, -4, -5, -6, -7],
                  [1, np.nan, 5, 5, 0, 0, 0, 0, 0, np.nan],
                  [-np.inf, -np.inf, -np.inf, -np.inf, -np.inf, -np.inf, -np.inf, -np.inf, -np.inf, 7]],
                 dtype=np.float32)
    bits = f32_to_bf16(f)
    ids, values, weights = ops.topk_softmax(bf16_tensor(bits, gpu), 3)
    torch.cuda.synchronize()
    # torch.topk's CPU order of these rows (torch 2.10)
    assert ids.cpu().numpy().tolist() == [[5, 4, 1], [1, 0, 3], [1, 9, 3], [9, 6, 5]]
    want_ids, want_vals = orr.topk(bits, 3)
    assert np.array_equal(ids.cpu().numpy(), want_ids)
    w = bf16_bits(weights)
    ow = orr.softmax_weights(want_vals)
    gn = (w & 0x7FFF) > 0x7F80
    assert np.array_equal(gn, (ow & 0x7FFF) > 0x7F80)
    assert np.array_equal(w[~gn], ow[~gn])


def tie_heavy_logits(seed, n_tok, n_exp):
    """bf16 logits with few distinct values per row (ties everywhere), some NaN and signed zeros."""
    rng = np.random.default_rng(seed)
    levels = rng.integers(1, 9, size=(n_tok, 1))
    f = (rng.integers(0, 1 << 20, size=(n_tok, n_exp)) % levels).astype(np.float32) - 2.0
    nan_rows = rng.random(n_tok) < 0.1
    f[nan_rows, rng.integers(0, n_exp, int(nan_rows.sum()))] = np.nan
    zero_rows = rng.random(n_tok) < 0.2
    f[zero_rows, rng.integers(0, n_exp, int(zero_rows.sum()))] = -0.0
    return f32_to_bf16(f)


@pytest.mark.parametrize("n_exp,k", [(5, 3), (32, 4), (64, 4), (128, 4), (128, 16), (200, 7), (256, 4), (256, 16),
                                     (300, 4), (1024, 4), (1024, 16), (1024, 32), (100, 32), (128, 1)])
def test_topk_torch_order_on_tie_heavy_rows(gpu, n_exp, k):
    """Rows full of equal values take the replay of torch's libstdc++ order (nth_element + sort, or
    partial_sort when k * 64 <= n_exp), in the 4-tokens-per-wave and the wave-per-token kernels."""
    n_tok = 203
    bits = tie_heavy_logits(n_exp * 100 + k, n_tok, n_exp)
    ids, values, weights = ops.topk_softmax(bf16_tensor(bits, gpu), k)
    torch.cuda.synchronize()
    want_ids, want_vals = orr.topk(bits, k)
    assert np.array_equal(ids.cpu().numpy(), want_ids)
    w = bf16_bits(weights)
    ow = orr.softmax_weights(want_vals)
    nan = (ow & 0x7FFF) > 0x7F80
    assert np.array_equal((w & 0x7FFF) > 0x7F80, nan)
    assert np.array_equal(w[~nan], ow[~nan])


def test_topk_torch_order_past_the_introselect_depth_limit(gpu):
    """Adversarial rows (McIlroy's adversary against median-of-three) drive libstdc++'s introselect
    to its heap-select fallback; the kernel replays that branch too."""
    from test_oracle_torch_cpu import _mcilroy_killer

    rows = []
    for n in (128,):
        for coarse in (1, 2, 3):
            rows.append(f32_to_bf16(np.floor(_mcilroy_killer(n, 3) / coarse)))
    bits = np.stack(rows)
    ids, _, _ = ops.topk_softmax(bf16_tensor(bits, gpu), 4)
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy(), orr.topk(bits, 4)[0])


@pytest.mark.parametrize("n_tok,k,n_exp", [(1, 4, 128), (64, 4, 128), (2048, 4, 128), (7, 3, 5), (300, 2, 256),
                                           (64, 4, 32), (255, 4, 128), (256, 4, 128), (1031, 1, 256),
                                           (600, 2, 1)])
def test_dispatch_matches_stable_counting_sort(gpu, n_tok, k, n_exp):
    """Below 1024 pairs one workgroup sorts; from 1024 on one workgroup per expert does (both give these
    outputs)."""
    rng_ids = synth.random_ints(900 + n_tok, n_tok * k, 0, n_exp - 1).reshape(n_tok, k).astype(np.int32)
    disp = ops.dispatch(torch.from_numpy(rng_ids).to(gpu), n_exp)
    torch.cuda.synchronize()
    counts, w_off, w_order, w_active = orr.dispatch(rng_ids, n_exp)
    assert np.array_equal(disp.offsets.cpu().numpy(), w_off)
    assert np.array_equal(disp.sorted_pairs.cpu().numpy(), w_order)
    na = int(disp.n_active.item())
    assert na == len(w_active)
    a = disp.active.cpu().numpy()
    assert np.array_equal(a[:na], w_active)
    assert (a[na:] == -1).all()
    # work units: every (expert, run of 8 / 4 tokens) once, experts ascending (the ABI's documented layout)
    u = disp.units.cpu().numpy()
    n_pairs = n_tok * k
    caps = {m: (n_pairs + (m - 1) * min(n_pairs, n_exp)) // m for m in (8, 4, 64)}
    assert u.size == 4 + caps[8] + caps[4] + caps[64]
    starts = {8: 4, 4: 4 + caps[8], 64: 4 + caps[8] + caps[4]}
    for slot, per in enumerate((8, 4, 64)):
        n = int(u[slot])
        want = [e | (j << 10) for e in range(n_exp) for j in range(-(-int(counts[e]) // per))]
        assert u[starts[per]:starts[per] + n].tolist() == want
        assert n <= caps[per]


def check_dispatch(gpu, ids, n_exp):
    disp = ops.dispatch(torch.from_numpy(ids).to(gpu), n_exp)
    torch.cuda.synchronize()
    counts, w_off, w_order, w_active = orr.dispatch(ids, n_exp)
    assert np.array_equal(disp.offsets.cpu().numpy(), w_off)
    assert np.array_equal(disp.sorted_pairs.cpu().numpy(), w_order)
    assert int(disp.n_active.item()) == len(w_active)
    u = disp.units.cpu().numpy()
    n_pairs = ids.size
    caps = {m: (n_pairs + (m - 1) * min(n_pairs, n_exp)) // m for m in (8, 4, 64)}
    starts = {8: 4, 4: 4 + caps[8], 64: 4 + caps[8] + caps[4]}
    for slot, per in enumerate((8, 4, 64)):
        want = np.concatenate([e | (np.arange(-(-int(counts[e]) // per), dtype=np.int64) << 10)
                               for e in range(n_exp)])
        assert int(u[slot]) == want.size
        assert np.array_equal(u[starts[per]:starts[per] + want.size], want)


@pytest.mark.parametrize("n_tok,n_exp", [(2048, 128), (9662, 128), (4001, 256), (5000, 3), (40000, 128)])
def test_dispatch_skewed_loads(gpu, n_tok, n_exp):
    """Hot experts take most pairs (one expert > 64 pairs per load, runs across the waves' ranges);
    40000 x 4 = 160000 pairs is past the 38648 a one-workgroup LDS staging could hold."""
    rng = np.random.default_rng(n_tok)
    hot = rng.random((n_tok, 4))
    ids = np.where(hot < 0.3, 7 % n_exp, np.where(hot < 0.45, (n_exp - 1), rng.integers(0, n_exp, (n_tok, 4))))
    check_dispatch(gpu, ids.astype(np.int32), n_exp)


def test_dispatch_rejects_too_many_pairs(gpu):
    from klcquant_amd._native import KlcError
    from klcquant_amd import _native as nat
    ids = torch.zeros((nat.DISPATCH_MAX_PAIRS + 1,), dtype=torch.int32, device=gpu)
    with pytest.raises(KlcError, match="n_pairs"):
        ops.dispatch(ids.view(-1, 1), 128)


def test_router_rejects_bad_shapes(gpu):
    x = torch.zeros((2, 64), dtype=torch.bfloat16, device=gpu)
    w = torch.zeros((8, 32), dtype=torch.bfloat16, device=gpu)
    b = torch.zeros(8, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError):
        ops.router_logits(x, w, b)
    from klcquant_amd._native import KlcError
    x2 = torch.zeros((2, 100), dtype=torch.bfloat16, device=gpu)
    w2 = torch.zeros((8, 100), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(KlcError, match="multiple of 8"):
        ops.router_logits(x2, w2, b)
    with pytest.raises(Exception):
        ops.topk_softmax(torch.zeros((2, 8), dtype=torch.bfloat16, device=gpu), 9)


def test_softmax_weights_of_host_chosen_scores(gpu):
    """klc_moe_softmax_weights: unordered scores, a NaN row, k = 1 and a wide k."""
    for n_tok, k in [(300, 4), (3, 1), (2, 40)]:
        vals = synth.random_normal_f32(90 + k, n_tok * k, 0.0, 3.0).reshape(n_tok, k)
        if k > 1:
            vals[1, 1] = np.nan
        got = ops.softmax_weights(torch.from_numpy(vals).to(gpu))
        torch.cuda.synchronize()
        want = orr.softmax_weights(vals)
        assert np.array_equal(bf16_bits(got), want) or k > 1 and np.array_equal(
            np.delete(bf16_bits(got), 1, axis=0), np.delete(want, 1, axis=0))
        if k > 1:
            assert np.isnan(got[1].float().cpu().numpy()).all()
