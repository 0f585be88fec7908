"""GPU: the one-launch decode layer (path "fused", batches of at most 16 tokens).

The one-launch layer runs the multi-launch layer's GEMV device code and the
same combine operations in the same order, and its router rounds the same
float64 sums, so for the same inputs its outputs, expert ids and routing
weights are bit-identical to the multi-launch GEMV layer's (path "gemv").
Each case checks exactly that; test_fused_120b_against_oracle also checks
the routing and outputs against the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor
from klcquant_amd import moe
from test_gpu_experts import oracle_layer

pytestmark = pytest.mark.gpu


def run(layer, xt, residual=None):
    n_tok = xt.shape[0]
    ids = torch.empty((n_tok, layer.k), dtype=torch.int32, device=xt.device)
    w = torch.empty((n_tok, layer.k), dtype=torch.bfloat16, device=xt.device)
    out = layer.forward(xt, ids=ids, weights=w, residual=residual)
    return out, ids, w


def compare_paths(gpu, workload, hidden, inter, n_exp, k, n_tok, precision="fp32", residual=False, step=0):
    dev_w = moe.MoELayerWeights.synthetic(workload, 0, hidden, inter, n_exp, gpu)
    x = moe.synthetic_hidden(workload, n_tok, hidden, step)
    xt = bf16_tensor(x, gpu)
    res = bf16_tensor(moe.synthetic_hidden(workload + 1, n_tok, hidden, step), gpu) if residual else None
    fused = moe.MoELayer(dev_w, k, precision=precision, path="fused")
    gemv = moe.MoELayer(dev_w, k, precision=precision, path="gemv")
    assert fused.layer_path(n_tok) == "fused"
    assert gemv.layer_path(n_tok) == "gemv"
    print(f"[fused] workload={workload} H={hidden} I={inter} E={n_exp} k={k} B={n_tok} {precision} "
          f"residual={residual}", flush=True)
    of, idf, wf = run(fused, xt, res)
    og, idg, wg = run(gemv, xt, res)
    torch.cuda.synchronize()
    assert np.array_equal(idf.cpu().numpy(), idg.cpu().numpy()), "expert ids differ from the multi-launch layer"
    assert np.array_equal(bf16_bits(wf), bf16_bits(wg)), "routing weights differ from the multi-launch layer"
    diff = np.flatnonzero(bf16_bits(of) != bf16_bits(og))
    assert diff.size == 0, f"{diff.size} outputs differ from the multi-launch layer (first at {diff[:4]})"
    assert fused.fused_status(n_tok) == 0, "a wait of the one-launch layer ran out"
    return dev_w, x, idf, wf, of


@pytest.mark.parametrize("n_tok", [1, 2, 3, 4, 5, 8, 13, 16])
def test_fused_small_layer_batches(gpu, n_tok):
    compare_paths(gpu, 61, 256, 128, 16, 4, n_tok)


@pytest.mark.parametrize("case", [
    (62, 512, 256, 128, 4, 1),
    (62, 512, 256, 128, 4, 16),
    (63, 256, 128, 256, 4, 16),   # 256 experts, 64 pairs
    (64, 256, 128, 64, 8, 8),     # k = 8, 64 pairs
    (65, 256, 128, 16, 1, 7),     # k = 1
    (66, 192, 96, 16, 4, 6),      # inputs that do not fill the last 128-deep step
    (67, 256, 128, 3, 2, 9),      # more tokens than experts: several tokens per unit
])
def test_fused_shapes(gpu, case):
    compare_paths(gpu, *case)


@pytest.mark.parametrize("n_tok", [1, 8, 16])
def test_fused_120b_shape(gpu, n_tok):
    """gpt-oss-120B shape (H = I = 2880, 128 experts, top-4): the benchmark's decode batches."""
    compare_paths(gpu, 68, 2880, 2880, 128, 4, n_tok)


def test_fused_120b_against_oracle(gpu):
    """B = 8 at the 120B shape: routing bit-exact and outputs within tolerance of the oracle."""
    from klcquant_amd import moe as m
    host = m.synthetic_host_layer(69, 0, 2880, 2880, 128)
    dev_w, x, ids, w, out = compare_paths(gpu, 69, 2880, 2880, 128, 4, 8)
    ref = oracle_layer(host, x, 4)
    assert np.array_equal(ids.cpu().numpy(), ref["ids"])
    assert np.array_equal(bf16_bits(w), ref["weights"])
    from oracle.numerics import bf16_to_f32
    got = bf16_to_f32(bf16_bits(out)).astype(np.float64)
    want = bf16_to_f32(ref["out"]).astype(np.float64)
    wf = bf16_to_f32(ref["weights"])
    slack = 2.0 ** -7 * np.sum(np.abs(wf[:, :, None] * ref["expert_out"]), axis=1)
    err = np.abs(got - want)
    assert (err <= 1e-2 + 2e-2 * np.abs(want) + slack).all(), f"worst {err.max():.3e}"


def test_fused_20b_shape_bf16_and_residual(gpu):
    compare_paths(gpu, 70, 2880, 2880, 32, 4, 4, precision="bf16")
    compare_paths(gpu, 71, 2880, 2880, 32, 4, 3, residual=True)


def test_fused_back_to_back_calls(gpu):
    """Consecutive launches on one workspace (no synchronisation between them): each launch's tag
    marks its own words and flags, so none reads a previous launch's."""
    hidden, inter, n_exp, k, n_tok = 512, 256, 64, 4, 8
    dev_w = moe.MoELayerWeights.synthetic(72, 0, hidden, inter, n_exp, gpu)
    fused = moe.MoELayer(dev_w, k, path="fused")
    gemv = moe.MoELayer(dev_w, k, path="gemv")
    xs = [bf16_tensor(moe.synthetic_hidden(72, n_tok, hidden, s), gpu) for s in range(6)]
    outs = [fused.forward(x) for x in xs]
    refs = [gemv.forward(x) for x in xs]
    torch.cuda.synchronize()
    for s, (o, r) in enumerate(zip(outs, refs)):
        assert np.array_equal(bf16_bits(o), bf16_bits(r)), f"call {s} differs"


def test_fused_batch_sizes_share_nothing(gpu):
    """Alternating batch sizes (each with its own workspace) and the static scratch."""
    hidden, inter, n_exp, k = 256, 128, 32, 4
    dev_w = moe.MoELayerWeights.synthetic(73, 0, hidden, inter, n_exp, gpu)
    fused = moe.MoELayer(dev_w, k, path="fused")
    gemv = moe.MoELayer(dev_w, k, path="gemv")
    for rnd in range(2):
        for n_tok in (1, 16, 5):
            xt = bf16_tensor(moe.synthetic_hidden(73, n_tok, hidden, rnd), gpu)
            a = fused.forward(xt)
            b = fused.forward_static_scratch(xt)
            c = gemv.forward(xt)
            torch.cuda.synchronize()
            assert np.array_equal(bf16_bits(a), bf16_bits(c))
            assert np.array_equal(bf16_bits(b), bf16_bits(c))


def test_fused_refusals(gpu):
    from klcquant_amd import _native as nat
    dev_w = moe.MoELayerWeights.synthetic(74, 0, 256, 128, 16, gpu)
    fused = moe.MoELayer(dev_w, 4, path="fused")
    xt = bf16_tensor(moe.synthetic_hidden(74, 17, 256), gpu)
    with pytest.raises(nat.KlcError, match="KLC_PATH_FUSED"):
        fused.forward(xt)
    assert moe.MoELayer(dev_w, 4).layer_path(17) == "gemv"
    assert moe.MoELayer(dev_w, 4).layer_path(16) == "gemv"  # the default keeps the multi-launch layer
    assert fused.layer_path(16) == "fused"


def test_fused_wait_that_runs_out_poisons_outputs(gpu, monkeypatch):
    """KLC_FUSED_SPIN_LIMIT=-1 makes every wait of the one-launch layer give up at once, from the host (no
    kernel spins or faults; every workgroup still ends).  That launch's outputs are NaN and its ids -1, so the
    failure shows without a sync, and the layer raises on the host.  A fresh layer computes normally again."""
    hidden, inter, n_exp, k, n_tok = 256, 128, 16, 4, 4
    dev_w = moe.MoELayerWeights.synthetic(75, 0, hidden, inter, n_exp, gpu)
    xt = bf16_tensor(moe.synthetic_hidden(75, n_tok, hidden), gpu)
    layer = moe.MoELayer(dev_w, k, path="fused")
    monkeypatch.setenv("KLC_FUSED_SPIN_LIMIT", "-1")
    out, ids, w = run(layer, xt)
    torch.cuda.synchronize()
    assert np.isnan(out.float().cpu().numpy()).all()
    assert (ids.cpu().numpy() == -1).all()
    assert np.isnan(w.float().cpu().numpy()).all()
    with pytest.raises(RuntimeError, match="ran out"):
        layer.check_fused_status()
    assert layer.fused_status(n_tok) & 1
    monkeypatch.delenv("KLC_FUSED_SPIN_LIMIT")
    fresh = moe.MoELayer(dev_w, k, path="fused")
    a = fresh.forward(xt)
    b = moe.MoELayer(dev_w, k, path="gemv").forward(xt)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(a), bf16_bits(b))
    fresh.check_fused_status()
    assert fresh.fused_status(n_tok) == 0
