"""klc_moe_layer_static_scratch (the layer without a workspace argument) against klc_moe_layer."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor
from klcquant_amd import moe, synth
from klcquant_amd._native import KlcError

pytestmark = pytest.mark.gpu


def run_both(layer, x):
    n = x.shape[0]
    k = layer.k
    out_ws = torch.empty_like(x)
    ids_ws = torch.empty((n, k), dtype=torch.int32, device=x.device)
    w_ws = torch.empty((n, k), dtype=torch.bfloat16, device=x.device)
    layer.forward(x, out=out_ws, ids=ids_ws, weights=w_ws)
    out_st = torch.full_like(x, float("nan"))
    ids_st = torch.full((n, k), -1, dtype=torch.int32, device=x.device)
    w_st = torch.full((n, k), float("nan"), dtype=torch.bfloat16, device=x.device)
    layer.forward_static_scratch(x, out=out_st, ids=ids_st, weights=w_st)
    torch.cuda.synchronize()
    return (bf16_bits(out_ws), ids_ws.cpu().numpy(), bf16_bits(w_ws)), (bf16_bits(out_st), ids_st.cpu().numpy(),
                                                                        bf16_bits(w_st))


@pytest.mark.parametrize("hidden,inter,n_exp,batches", [(2880, 2880, 128, (64, 5)), (256, 128, 16, (200, 1))])
def test_static_scratch_equals_workspace_path(gpu, hidden, inter, n_exp, batches):
    """Two calls in a row on the shared scratch, the second with fewer tokens (decode router; 200 tokens take
    the separate router, top-k and dispatch kernels and the grouped GEMM)."""
    layer = moe.MoELayer(moe.MoELayerWeights.synthetic(7, 0, hidden, inter, n_exp, gpu), 4)
    for i, n in enumerate(batches):
        x = bf16_tensor(synth.random_normal_bf16(700 + 10 * i + n, n * hidden).reshape(n, hidden), gpu)
        want, got = run_both(layer, x)
        for a, b in zip(want, got):
            assert np.array_equal(a, b), (n, i)


def test_static_scratch_residual_and_repeat(gpu):
    """Residual add in place, and a third call after a larger one: the counters stay consistent."""
    hidden, inter, n_exp = 256, 128, 32
    layer = moe.MoELayer(moe.MoELayerWeights.synthetic(8, 0, hidden, inter, n_exp, gpu), 4)
    for n in (100, 3, 17):
        x = bf16_tensor(synth.random_normal_bf16(800 + n, n * hidden).reshape(n, hidden), gpu)
        r = bf16_tensor(synth.random_normal_bf16(900 + n, n * hidden).reshape(n, hidden), gpu)
        r2 = r.clone()
        layer.forward(x, out=r, residual=r)
        layer.forward_static_scratch(x, out=r2, residual=r2)
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(r), bf16_bits(r2)), n


def test_static_scratch_refuses_batches_beyond_its_size(gpu):
    hidden, inter, n_exp = 2880, 2880, 128
    layer = moe.MoELayer(moe.MoELayerWeights.synthetic(7, 0, hidden, inter, n_exp, gpu), 4)
    x = torch.zeros((1024, hidden), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(KlcError, match="static scratch"):
        layer.forward_static_scratch(x)


def test_static_scratch_allocates_nothing(gpu):
    """After a first call (which looks the scratch up), repeated calls with preallocated out, ids and
    weights leave the device's free memory and torch's reserved memory unchanged."""
    hidden, inter, n_exp, n = 2880, 2880, 128, 8
    layer = moe.MoELayer(moe.MoELayerWeights.synthetic(9, 0, hidden, inter, n_exp, gpu), 4)
    x = bf16_tensor(synth.random_normal_bf16(950, n * hidden).reshape(n, hidden), gpu)
    out = torch.empty_like(x)
    ids = torch.empty((n, 4), dtype=torch.int32, device=gpu)
    w = torch.empty((n, 4), dtype=torch.bfloat16, device=gpu)
    layer.forward_static_scratch(x, out=out, ids=ids, weights=w)
    torch.cuda.synchronize()
    free0, reserved0 = torch.cuda.mem_get_info(gpu)[0], torch.cuda.memory_reserved(gpu)
    for _ in range(20):
        layer.forward_static_scratch(x, out=out, ids=ids, weights=w)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info(gpu)[0] == free0
    assert torch.cuda.memory_reserved(gpu) == reserved0
