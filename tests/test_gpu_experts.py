"""GPU parity: gate_up/SwiGLU/down/combine and the fused layer against the oracle.

Tolerances (expert outputs, float32): |gpu - ref| <= 1e-2 + 2e-2 * |ref|
elementwise.  The bfloat16 combine is checked bit-exactly against the oracle's
combine applied to the GPU's own float32 expert outputs; the final output
against the oracle's final output allows, on top of 1e-2 + 2e-2 * |ref|, one
bfloat16 rounding step of the running sum (2**-7 * sum_j |w_j * out_j|),
because a last-bit difference in an expert output can flip one rounding of the
sequential bfloat16 accumulation.

Under expert_matmul_precision="bf16" the reference rounds both matmul inputs
and outputs to bfloat16 (streamed_moe_router.py:503, 507-509), so two valid
float32 accumulation orders already differ by a bfloat16 rounding of the
gate_up result, which the down matmul spreads over a whole output row (the
CPU oracle with float32 instead of float64 accumulation differs from itself by
0.023 at outputs of magnitude 0.3).  That mode adds 2**-8 * rms(row) to the
absolute tolerance.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor
from klcquant_amd import moe, ops
from oracle import experts as oex
from oracle import layer as olayer
from oracle.numerics import bf16_to_f32

pytestmark = pytest.mark.gpu

RTOL, ATOL = 2e-2, 1e-2


def build(gpu, workload, hidden, inter, n_exp, n_tok, step=0, bias_override=None):
    host = moe.synthetic_host_layer(workload, 0, hidden, inter, n_exp, bias_override)
    dev_w = moe.MoELayerWeights.synthetic(workload, 0, hidden, inter, n_exp, gpu, bias_override)
    x = moe.synthetic_hidden(workload, n_tok, hidden, step)
    return host, dev_w, x


def oracle_layer(host, x, k, precision="fp32"):
    return olayer.moe_layer(x, host["router_weight"], host["router_bias"], host["gate_up_blocks"],
                            host["gate_up_scales"], host["gate_up_bias"], host["down_blocks"], host["down_scales"],
                            host["down_bias"], k=k, precision=precision)


def assert_close(got, want, what, precision="fp32"):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    err = np.abs(got - want)
    tol = ATOL + RTOL * np.abs(want)
    if precision == "bf16":
        tol = tol + 2.0 ** -8 * np.sqrt(np.mean(want ** 2, axis=-1, keepdims=True))
    bad = np.argwhere(err > tol)
    assert bad.size == 0, f"{what}: {bad.shape[0]} elements out of tolerance, worst {err.max():.3e}"


def check_layer(gpu, host, dev_w, x, k, precision, path="auto"):
    layer = moe.MoELayer(dev_w, experts_per_token=k, precision=precision, path=path)
    xt = bf16_tensor(x, gpu)
    det = layer.forward_detailed(xt)
    fused_ids = torch.empty((x.shape[0], k), dtype=torch.int32, device=gpu)
    fused_w = torch.empty((x.shape[0], k), dtype=torch.bfloat16, device=gpu)
    fused = layer.forward(xt, ids=fused_ids, weights=fused_w)
    torch.cuda.synchronize()
    ref = oracle_layer(host, x, k, precision)

    ids = det["ids"].cpu().numpy()
    assert np.array_equal(bf16_bits(det["logits"]), ref["logits"])
    assert np.array_equal(ids, ref["ids"])
    assert np.array_equal(bf16_bits(det["weights"]), ref["weights"])
    # the single-call layer's own routing (one-launch router for decode batches)
    assert np.array_equal(fused_ids.cpu().numpy(), ref["ids"])
    assert np.array_equal(bf16_bits(fused_w), ref["weights"])

    n_tok = x.shape[0]
    gated = det["gated"].cpu().numpy().reshape(n_tok, k, -1)
    eo = det["expert_out"].cpu().numpy().reshape(n_tok, k, -1)
    assert_close(gated, ref["gated"], "SwiGLU output", precision)
    assert_close(eo, ref["expert_out"], "expert output", precision)

    out = bf16_bits(det["out"])
    # combine: bit-exact given the GPU's own expert outputs
    assert np.array_equal(out, oex.combine(eo, bf16_bits(det["weights"])))
    # fused single-call layer == step-by-step path, bit for bit
    assert np.array_equal(bf16_bits(fused), out)
    assert_final_close(out, ref, precision)
    return det, ref


def assert_final_close(out_bits, ref, precision="fp32"):
    """Final bf16 output vs the oracle's, with the combine's rounding slack."""
    w = bf16_to_f32(ref["weights"])
    slack = 2.0 ** -7 * np.sum(np.abs(w[:, :, None] * ref["expert_out"]), axis=1)
    got = bf16_to_f32(np.asarray(out_bits).reshape(ref["out"].shape)).astype(np.float64)
    want = bf16_to_f32(ref["out"]).astype(np.float64)
    err = np.abs(got - want)
    if precision == "bf16":
        slack = slack + 2.0 ** -8 * np.sum(np.abs(w[:, :, None]) * np.sqrt(np.mean(ref["expert_out"] ** 2, axis=-1,
                                                                               keepdims=True)), axis=1)
    assert (err <= ATOL + RTOL * np.abs(want) + slack).all(), f"final output worst error {err.max():.3e}"


@pytest.mark.parametrize("n_tok,k,n_exp", [(1, 4, 8), (1, 2, 8), (1, 3, 37), (1, 1, 4), (16, 4, 8), (5, 2, 3),
                                           (33, 4, 16), (97, 2, 37), (128, 4, 256)])
def test_small_layer_matches_oracle(gpu, n_tok, k, n_exp):
    host, dev_w, x = build(gpu, 50 + n_tok, 128, 64, n_exp, n_tok)
    check_layer(gpu, host, dev_w, x, k, "fp32")


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
@pytest.mark.parametrize("n_tok", [1, 3])
def test_gpt_oss_20b_shape_layer(gpu, precision, n_tok):
    """gpt-oss-20B shape: H = I = 2880, 32 experts, top-4; one decode token (the single-token layer of the
    20B-shape benchmark) and three."""
    host, dev_w, x = build(gpu, 0, 2880, 2880, 32, n_tok)
    check_layer(gpu, host, dev_w, x, 4, precision)


def test_gpt_oss_120b_shape_batch8(gpu):
    host, dev_w, x = build(gpu, 2, 2880, 2880, 128, 8)
    check_layer(gpu, host, dev_w, x, 4, "fp32")


@pytest.mark.parametrize("n_tok", [64, 45])
def test_gemv_layer_many_units_per_expert(gpu, n_tok):
    """Decode GEMVs with 4-6 gate_up and 8-12 down units per expert (20B shape, 8 experts): in the one-call
    layer every down workgroup waits for several gate_up workgroups of its expert."""
    host, dev_w, x = build(gpu, 5, 2880, 2880, 8, n_tok)
    check_layer(gpu, host, dev_w, x, 4, "fp32", path="gemv")


def test_many_tokens_one_expert(gpu):
    """Router bias forces every token onto the same 4 experts: > 4 tokens per expert tile pass."""
    n_exp = 8
    bias = np.full(n_exp, 0xC2C8, dtype=np.uint16)  # -100.0
    bias[[1, 3, 4, 6]] = 0x42C8  # +100.0
    host, dev_w, x = build(gpu, 77, 128, 64, n_exp, 21, bias_override=bias)
    det, ref = check_layer(gpu, host, dev_w, x, 4, "fp32")
    assert set(np.unique(ref["ids"])) == {1, 3, 4, 6}


def test_bias_only_combine(gpu):
    n_tok, k, n_exp, hidden = 9, 4, 16, 256
    from klcquant_amd import synth
    from oracle.router import topk
    dbias = synth.random_normal_bf16(5, n_exp * hidden, 0, 0.5).reshape(n_exp, hidden)
    logits = synth.random_normal_bf16(6, n_tok * n_exp).reshape(n_tok, n_exp)
    ids, vals = topk(logits, k)
    from oracle.router import softmax_weights
    w = softmax_weights(vals)
    got = ops.bias_combine(bf16_tensor(dbias, gpu), torch.from_numpy(ids.astype(np.int32)).to(gpu), bf16_tensor(w, gpu))
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(got), oex.bias_only(dbias, ids, w))


def test_pair_norms(gpu):
    host, dev_w, x = build(gpu, 9, 128, 64, 8, 6)
    layer = moe.MoELayer(dev_w, 4)
    det = layer.forward_detailed(bf16_tensor(x, gpu))
    norms = ops.pair_norms(det["gated"], det["expert_out"]).cpu().numpy()
    g = det["gated"].cpu().numpy().astype(np.float64)
    o = det["expert_out"].cpu().numpy().astype(np.float64)
    np.testing.assert_allclose(norms[:, 0], np.linalg.norm(g, axis=1), rtol=1e-6)
    np.testing.assert_allclose(norms[:, 1], np.linalg.norm(o, axis=1), rtol=1e-6)


@pytest.mark.parametrize("k", [4, 2])
def test_single_token_layer_with_residual(gpu, k):
    """One token takes the single-token kernels (gate_up by slot, down with the combine in one launch); with a
    residual its output is the step-by-step path's combine plus the residual, bit for bit."""
    host, dev_w, x = build(gpu, 91, 2880, 2880, 128, 1)
    layer = moe.MoELayer(dev_w, k)
    xt = bf16_tensor(x, gpu)
    res = bf16_tensor(moe.synthetic_hidden(92, 1, 2880), gpu)
    out = layer.forward(xt, residual=res)
    det = layer.forward_detailed(xt)
    want = ops.combine(det["expert_out"], det["weights"], 1, k, residual=res)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(out), bf16_bits(want))
