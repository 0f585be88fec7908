"""MoE layers replayed from HIP graphs against eager calls (moe.MoELayer.capture_graph).

Each graph is replayed several times with eager work and synchronisations
between replays, and every replay is checked against the eager result, bit
for bit: the layer records no memset and its completion counters reset
themselves, so a replay must equal the first run.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor
from klcquant_amd import moe, synth

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("hidden,inter,n_exp,n_tok", [(2880, 2880, 128, 1), (2880, 2880, 128, 64),
                                                      (256, 128, 16, 300)])
def test_graph_replays_equal_eager(gpu, hidden, inter, n_exp, n_tok):
    layer = moe.MoELayer(moe.MoELayerWeights.synthetic(31, 0, hidden, inter, n_exp, gpu), 4)
    xs = [bf16_tensor(synth.random_normal_bf16(3100 + i, n_tok * hidden).reshape(n_tok, hidden), gpu)
          for i in range(3)]
    want = []
    for x in xs:
        ids = torch.empty((n_tok, 4), dtype=torch.int32, device=gpu)
        want.append((bf16_bits(layer.forward(x, ids=ids)), ids.cpu().numpy()))
    x_static = xs[0].clone()
    out = torch.empty_like(x_static)
    ids = torch.empty((n_tok, 4), dtype=torch.int32, device=gpu)
    graph = layer.capture_graph(x_static, out, ids=ids)
    for rep in range(6):
        i = rep % 3
        x_static.copy_(xs[i])
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(out), want[i][0]), rep
        assert np.array_equal(ids.cpu().numpy(), want[i][1]), rep
        # eager work between replays, on the same layer and scratch
        layer.forward_static_scratch(xs[(i + 1) % 3])
        torch.cuda.synchronize()


def test_graph_of_a_stack_step_with_residual(gpu):
    """Three layers' static-scratch calls with the residual added in place, captured as one graph."""
    hidden, inter, n_exp, n_tok = 256, 128, 16, 8
    layers = [moe.MoELayer(moe.MoELayerWeights.synthetic(32, l, hidden, inter, n_exp, gpu), 4) for l in range(3)]
    x0 = bf16_tensor(synth.random_normal_bf16(3200, n_tok * hidden).reshape(n_tok, hidden), gpu)
    h = x0.clone()
    for layer in layers:
        layer.forward(h, out=h, residual=h)
    want = bf16_bits(h)
    h2 = x0.clone()
    for layer in layers:  # first calls outside capture
        layer.forward_static_scratch(h2, out=h2, residual=h2)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for layer in layers:
            layer.forward_static_scratch(h2, out=h2, residual=h2)
    for _ in range(3):
        h2.copy_(x0)
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(h2), want)
