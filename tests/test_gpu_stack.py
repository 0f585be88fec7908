"""GPU parity of the stacked decode pieces: RMSNorm (bit-exact), the combine
with residual add (bit-exact given the GPU's expert outputs), and a short
MoE stack checked layer by layer against the oracle.

The stack check feeds the GPU's own hidden state after layer L-1 to the
oracle's layer L, so each layer is judged on identical inputs (a last-bit
difference in one layer's output could otherwise flip a near-tied top-k
choice in the next).  Layer outputs use the final-output tolerance of
test_gpu_experts plus one bfloat16 rounding of the residual sum.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor
from klcquant_amd import moe, ops, synth
from oracle import experts as oex
from oracle.numerics import bf16_to_f32, f32_to_bf16
from oracle.rmsnorm import residual_add, rms_norm
from test_gpu_experts import ATOL, RTOL, oracle_layer

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n_tok,hidden", [(1, 2880), (64, 2880), (7, 256), (3, 8)])
def test_rms_norm_bit_exact(gpu, n_tok, hidden):
    x = synth.random_normal_bf16(70 + n_tok, n_tok * hidden, 0.0, 3.0).reshape(n_tok, hidden)
    w = synth.random_normal_bf16(71, hidden, 1.0, 0.05)
    if n_tok > 2:
        x[2] = 0  # all-zero row: rsqrt(eps) times zeros
    got = ops.rms_norm(bf16_tensor(x, gpu), bf16_tensor(w, gpu))
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(got), rms_norm(x, w))


@pytest.mark.parametrize("n_tok,k,hidden,misaligned", [
    (9, 4, 256, False),   # 4 outputs per thread, all slots' loads in flight together
    (5, 2, 256, False),
    (7, 6, 2880, False),  # more slots than one batch of loads
    (6, 4, 30, False),    # hidden % 4 != 0: one output per thread
    (4, 3, 256, True),    # expert outputs not 16-byte aligned: one output per thread
])
def test_combine_with_residual_bit_exact(gpu, n_tok, k, hidden, misaligned):
    eo = synth.random_normal_f32(80, n_tok * k * hidden, 0.0, 50.0).reshape(n_tok * k, hidden)
    wts = f32_to_bf16(np.abs(synth.random_normal_f32(81, n_tok * k)).reshape(n_tok, k) / 4)
    res = synth.random_normal_bf16(82, n_tok * hidden, 0.0, 20.0).reshape(n_tok, hidden)
    res_t = bf16_tensor(res, gpu)
    eo_t = torch.from_numpy(eo).to(gpu)
    if misaligned:
        buf = torch.empty(eo.size + 1, dtype=torch.float32, device=gpu)
        buf[1:] = eo_t.reshape(-1)
        eo_t = buf[1:].reshape(n_tok * k, hidden)
    got = ops.combine(eo_t, bf16_tensor(wts, gpu), n_tok, k, residual=res_t)
    torch.cuda.synchronize()
    want = residual_add(res, oex.combine(eo.reshape(n_tok, k, hidden), wts))
    assert np.array_equal(bf16_bits(got), want)


@pytest.mark.parametrize("precision", ["fp32"])
def test_stack_layer_by_layer(gpu, precision):
    n_layers, hidden, inter, n_exp, n_tok, k = 3, 256, 128, 16, 6, 4
    workload = 91
    stack = moe.MoEStack.synthetic(workload, n_layers, hidden, inter, n_exp, gpu, precision=precision)
    x = moe.synthetic_hidden(workload, n_tok, hidden)
    trace: list = []
    ids = [torch.empty((n_tok, k), dtype=torch.int32, device=gpu) for _ in range(n_layers)]
    out = stack(bf16_tensor(x, gpu), trace=trace, ids=ids)
    torch.cuda.synchronize()
    assert torch.equal(out, trace[-1])
    h_in = x
    for layer in range(n_layers):
        host = moe.synthetic_host_layer(workload, layer, hidden, inter, n_exp)
        normed = rms_norm(h_in, moe.synthetic_norm_weight(workload, layer, hidden))
        ref = oracle_layer(host, normed, k, precision)
        assert np.array_equal(ids[layer].cpu().numpy(), ref["ids"]), f"layer {layer} routing"
        want = bf16_to_f32(residual_add(h_in, ref["out"])).astype(np.float64)
        got_bits = bf16_bits(trace[layer])
        got = bf16_to_f32(got_bits).astype(np.float64)
        w = bf16_to_f32(ref["weights"])
        slack = 2.0 ** -7 * np.sum(np.abs(w[:, :, None] * ref["expert_out"]), axis=1) + 2.0 ** -8 * np.abs(want)
        err = np.abs(got - want)
        assert (err <= ATOL + RTOL * np.abs(want) + slack).all(), f"layer {layer}: worst error {err.max():.3e}"
        h_in = got_bits
