"""GPU parity of the prefill path (expert-grouped GEMM) against the oracle.

Tolerances are those of the decode GEMVs (test_gpu_experts): routing (logits,
ids, weights) bit-exact; SwiGLU and expert outputs |gpu - ref| <= 1e-2 +
2e-2 |ref| (exact products, float32 sums; the down input as hi + lo bfloat16,
relative residual 2^-17); final outputs add the bfloat16 combine slack.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor
from klcquant_amd import moe
from test_gpu_experts import assert_close, assert_final_close, build, oracle_layer

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n_tok,k,n_exp,precision", [(256, 4, 16, "fp32"), (40, 4, 8, "fp32"), (130, 2, 4, "bf16"),
                                                      (256, 4, 16, "bf16"), (75, 4, 8, "bf16")])
def test_gemm_layer_matches_oracle(gpu, n_tok, k, n_exp, precision):
    host, dev_w, x = build(gpu, 400 + n_tok, 256, 128, n_exp, n_tok)
    layer = moe.MoELayer(dev_w, experts_per_token=k, precision=precision, path="gemm")
    xt = bf16_tensor(x, gpu)
    det = layer.forward_detailed(xt)
    fused = layer.forward(xt)
    torch.cuda.synchronize()
    ref = oracle_layer(host, x, k, precision)
    assert np.array_equal(bf16_bits(det["logits"]), ref["logits"])
    assert np.array_equal(det["ids"].cpu().numpy(), ref["ids"])
    assert np.array_equal(bf16_bits(det["weights"]), ref["weights"])
    gated = det["gated"].cpu().numpy().reshape(n_tok, k, -1)
    eo = det["expert_out"].cpu().numpy().reshape(n_tok, k, -1)
    assert_close(gated, ref["gated"], "SwiGLU output", precision)
    assert_close(eo, ref["expert_out"], "expert output", precision)
    assert np.array_equal(bf16_bits(fused), bf16_bits(det["out"]))
    assert_final_close(bf16_bits(det["out"]), ref, precision)


@pytest.mark.parametrize("hidden,inter,precision", [(1024, 2048, "fp32"), (1024, 2048, "bf16"), (896, 960, "bf16"),
                                                   (3072, 3072, "fp32")])
def test_gemm_step_counts(gpu, hidden, inter, precision):
    """Inputs whose 128-wide step counts leave the step loop's padding past
    the scale records (8 and 16 steps), a 7-step and 7.5-step pair, and the
    widest supported input (24 steps)."""
    n_tok, k, n_exp = 72, 4, 8
    host, dev_w, x = build(gpu, 430 + hidden + inter, hidden, inter, n_exp, n_tok)
    layer = moe.MoELayer(dev_w, experts_per_token=k, precision=precision, path="gemm")
    det = layer.forward_detailed(bf16_tensor(x, gpu))
    torch.cuda.synchronize()
    ref = oracle_layer(host, x, k, precision)
    assert np.array_equal(det["ids"].cpu().numpy(), ref["ids"])
    assert_close(det["gated"].cpu().numpy().reshape(n_tok, k, -1), ref["gated"], "SwiGLU output", precision)
    assert_close(det["expert_out"].cpu().numpy().reshape(n_tok, k, -1), ref["expert_out"], "expert output", precision)
    assert_final_close(bf16_bits(det["out"]), ref, precision)


def test_gemm_units_span_hot_experts(gpu):
    """Router bias sends every token to the same 4 experts: 300 tokens per expert = 5 GEMM units each."""
    n_exp, n_tok = 8, 300
    bias = np.full(n_exp, 0xC2C8, dtype=np.uint16)  # -100.0
    bias[[0, 2, 5, 7]] = 0x42C8  # +100.0
    host, dev_w, x = build(gpu, 77, 128, 64, n_exp, n_tok, bias_override=bias)
    layer = moe.MoELayer(dev_w, 4, path="gemm")
    det = layer.forward_detailed(bf16_tensor(x, gpu))
    torch.cuda.synchronize()
    ref = oracle_layer(host, x, 4)
    assert set(np.unique(ref["ids"])) == {0, 2, 5, 7}
    assert int(det["units"][2]) == 4 * 5
    assert_close(det["expert_out"].cpu().numpy().reshape(n_tok, 4, -1), ref["expert_out"], "expert output")
    assert_final_close(bf16_bits(det["out"]), ref)


def test_gemm_and_gemv_paths_agree(gpu):
    host, dev_w, x = build(gpu, 55, 256, 128, 16, 24)
    xt = bf16_tensor(x, gpu)
    a = moe.MoELayer(dev_w, 4, path="gemm").forward_detailed(xt)
    b = moe.MoELayer(dev_w, 4, path="gemv").forward_detailed(xt)
    torch.cuda.synchronize()
    ref = oracle_layer(host, x, 4)
    for det in (a, b):
        assert_close(det["expert_out"].cpu().numpy().reshape(24, 4, -1), ref["expert_out"], "expert output")
    assert torch.equal(a["ids"], b["ids"])


def test_gpt_oss_120b_shape_prefill_chunk(gpu):
    """120B shape, 256 tokens: 1024 pairs over 128 experts takes the GEMM path automatically."""
    host, dev_w, x = build(gpu, 3, 2880, 2880, 128, 256)
    layer = moe.MoELayer(dev_w, 4)
    assert layer.uses_gemm(256)
    xt = bf16_tensor(x, gpu)
    det = layer.forward_detailed(xt)
    fused = layer.forward(xt)
    torch.cuda.synchronize()
    ref = oracle_layer(host, x, 4)
    assert np.array_equal(det["ids"].cpu().numpy(), ref["ids"])
    assert_close(det["expert_out"].cpu().numpy().reshape(256, 4, -1), ref["expert_out"], "expert output")
    assert np.array_equal(bf16_bits(fused), bf16_bits(det["out"]))
    assert_final_close(bf16_bits(det["out"]), ref)
