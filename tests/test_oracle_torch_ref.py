"""The torch-CPU restatement of the reference path (the CPU baseline) against the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from klcquant_amd import moe, synth
from oracle import layer as olayer
from oracle import mxfp4 as omx
from oracle import torch_ref
from oracle.numerics import bf16_to_f32


def t_bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16)).view(torch.bfloat16)


def test_dequantize_equals_oracle_on_every_code_and_scale():
    codes = np.arange(256, dtype=np.uint8)
    blocks = np.tile(codes.reshape(16, 1, 16), (256, 1, 1, 1)).reshape(256 * 16, 1, 16)
    scales = np.repeat(np.arange(256, dtype=np.uint8), 16).reshape(256 * 16, 1)
    got = torch_ref.dequantize(torch.from_numpy(blocks), torch.from_numpy(scales), torch.float32).numpy()
    want = omx.dequantize(blocks, scales, "f32")
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.nan_to_num(got).view(np.uint32), np.nan_to_num(want).view(np.uint32))
    got16 = torch_ref.dequantize(torch.from_numpy(blocks), torch.from_numpy(scales)).view(torch.int16).numpy()
    want16 = omx.dequantize(blocks, scales, "bf16")
    nan = (want16 & 0x7FFF) > 0x7F80
    assert np.array_equal((got16.view(np.uint16) & 0x7FFF) > 0x7F80, nan)
    assert np.array_equal(got16.view(np.uint16)[~nan], want16[~nan])


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_route_matches_the_oracle_layer(precision):
    hidden, inter, n_exp, n_tok, k = 256, 128, 16, 6, 4
    host = moe.synthetic_host_layer(17, 0, hidden, inter, n_exp)
    x = moe.synthetic_hidden(17, n_tok, hidden)
    experts = {e: tuple(torch.from_numpy(host[n][e]) for n in ("gate_up_blocks", "gate_up_scales", "down_blocks",
                                                               "down_scales")) for e in range(n_exp)}
    layer = torch_ref.Layer(t_bf16(host["router_weight"]), t_bf16(host["router_bias"]), t_bf16(host["gate_up_bias"]),
                            t_bf16(host["down_bias"]), experts, k)
    ref = olayer.moe_layer(x, host["router_weight"], host["router_bias"], host["gate_up_blocks"],
                           host["gate_up_scales"], host["gate_up_bias"], host["down_blocks"], host["down_scales"],
                           host["down_bias"], k=k, precision=precision)
    for warm in (False, True):
        for t in range(n_tok):
            out, ids = layer.route(t_bf16(x[t]), warm, precision)
            assert ids == ref["ids"][t].tolist()
            got = out.float().numpy().astype(np.float64)
            want = bf16_to_f32(ref["out"][t]).astype(np.float64)
            w = bf16_to_f32(ref["weights"][t])
            slack = 2.0 ** -7 * np.sum(np.abs(w[:, None] * ref["expert_out"][t]), axis=0)
            if precision == "bf16":  # matmul results rounded to bf16 on both sides
                slack = slack + 2.0 ** -8 * np.sum(np.abs(w[:, None]) * np.abs(ref["expert_out"][t]), axis=0)
            assert (np.abs(got - want) <= 1e-2 + 2e-2 * np.abs(want) + slack).all()
    assert len(layer.cache) > 0
