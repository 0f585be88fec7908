"""Every benchmark workload against the oracle at its own size (gpt-oss shapes).

* 128 x down_proj dequant, 2880 x 2880 each (2.12 GB of bf16 output), plus
  8 more matrices of the same stream so that the output runs past 2^31
  bytes: every matrix bit-exact (mxfp4_expert.py:357-379).
* 120B-shape decode layer (E = 128, top-4) at B = 1 and B = 64, the fused
  layer's GEMV path: routing bit-exact, expert outputs within
  1e-2 + 2e-2 |ref|, the final output with the combine's rounding slack
  (streamed_moe_router.py:257-329, 483-529).
* 120B-shape prefill of 2048 tokens with the Zipf(1.1) router bias: the
  grouped GEMM, whose hottest expert takes ~1848 pairs (29 GEMM units).
* 36-layer 120B-shape stack (RMSNorm -> MoE -> residual, 61 GB of resident
  experts) at B = 64: routing of all 36 layers equals the oracle router on
  the GPU's own normed inputs, every hidden state is finite, and layers 0,
  17 and 35 are compared in full on the GPU's own inputs.

The oracle builds only the experts the tokens select (synth.mxfp4_expert_slice)
and evaluates them on a few threads.
"""

from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor
from klcquant_amd import moe, ops, synth
from oracle import layer as olayer
from oracle import mxfp4 as omx
from oracle import router as orr
from oracle.numerics import bf16_to_f32, f32_to_bf16
from oracle.rmsnorm import residual_add, rms_norm
from test_gpu_experts import ATOL, RTOL, assert_close, assert_final_close

pytestmark = pytest.mark.gpu

H = I = 2880
E, K = 128, 4
WORKERS = 8


def host_router(workload, layer, n_exp=E, bias=None):
    seed = {n: synth.tensor_seed(workload, n, layer) for n in synth.TENSOR_IDS}
    return {
        "router_weight": synth.random_normal_bf16(seed["router_weight"], n_exp * H, 0.0, 0.02).reshape(n_exp, H),
        "router_bias": bias if bias is not None else synth.random_normal_bf16(seed["router_bias"], n_exp, 0.0, 0.01),
        "gate_up_bias": synth.random_normal_bf16(seed["gate_up_bias"], n_exp * 2 * I, 0.0, 0.01).reshape(n_exp, -1),
        "down_bias": synth.random_normal_bf16(seed["down_bias"], n_exp * H, 0.0, 0.01).reshape(n_exp, -1),
    }


def expert_fn(workload, layer):
    seed = {n: synth.tensor_seed(workload, n, layer) for n in synth.TENSOR_IDS}

    def fn(e):
        gub, gus = synth.mxfp4_expert_slice(seed["gate_up_blocks"], seed["gate_up_scales"], e, 2 * I, H)
        db, ds = synth.mxfp4_expert_slice(seed["down_blocks"], seed["down_scales"], e, H, I)
        return gub, gus, db, ds

    return fn


def oracle(workload, layer, x, host, precision="fp32"):
    return olayer.moe_layer_lazy(x, host["router_weight"], host["router_bias"], expert_fn(workload, layer),
                                 host["gate_up_bias"], host["down_bias"], k=K, precision=precision, workers=WORKERS)


def check_layer_full(gpu, dev_w, x, ref, path, precision="fp32"):
    """Fused layer (routing, output) and the step-by-step path (expert outputs) against the oracle."""
    layer = moe.MoELayer(dev_w, K, precision=precision, path=path)
    xt = bf16_tensor(x, gpu)
    ids = torch.empty((x.shape[0], K), dtype=torch.int32, device=gpu)
    wts = torch.empty((x.shape[0], K), dtype=torch.bfloat16, device=gpu)
    out = layer.forward(xt, ids=ids, weights=wts)
    det = layer.forward_detailed(xt)
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy(), ref["ids"])
    assert np.array_equal(bf16_bits(wts), ref["weights"])
    n = x.shape[0]
    assert_close(det["gated"].cpu().numpy().reshape(n, K, -1), ref["gated"], "SwiGLU output", precision)
    assert_close(det["expert_out"].cpu().numpy().reshape(n, K, -1), ref["expert_out"], "expert output", precision)
    assert np.array_equal(bf16_bits(out), bf16_bits(det["out"]))
    assert_final_close(bf16_bits(out), ref, precision)


@pytest.mark.timeout(300)
def test_dequant_128_down_proj_full_size(gpu):
    n, rows, groups = E + 8, H, I // 32  # the benchmark's 128 matrices, then 8 past 2^31 output bytes
    seed_b, seed_s = 1000 * 1 + 7, 1000 * 1 + 8  # the benchmark's dequant workload
    blocks = torch.empty((n, rows, groups, 16), dtype=torch.uint8, device=gpu)
    scales = torch.empty((n, rows, groups), dtype=torch.uint8, device=gpu)
    ops.synth_fill(blocks, seed_b, 0)
    ops.synth_fill(scales, seed_s, 1, 118, 124)
    out = ops.mxfp4_dequant(blocks, scales, torch.bfloat16)
    torch.cuda.synchronize()
    assert out.shape == (n, groups * 32, rows) and out.numel() * 2 > 2 ** 31 > E * rows * groups * 64
    del blocks, scales

    def check(m):
        b, s = synth.mxfp4_expert_slice(seed_b, seed_s, m, rows, groups * 32)
        want = f32_to_bf16(omx.dequant_values_f32(b, s))  # [out, in]; the kernel writes [in, out]
        got = out[m].view(torch.int16).cpu().numpy().view(np.uint16)
        return bool(np.array_equal(got.T, want))

    with ThreadPoolExecutor(max_workers=WORKERS) as pool:
        ok = list(pool.map(check, range(n)))
    assert all(ok), [m for m, good in enumerate(ok) if not good][:8]


@pytest.mark.timeout(300)
@pytest.mark.parametrize("n_tok", [1, 64])
def test_decode_layer_120b_full_size(gpu, n_tok):
    workload = 2  # the benchmark's decode workload, layer 0, input batch 0
    dev_w = moe.MoELayerWeights.synthetic(workload, 0, H, I, E, gpu)
    x = moe.synthetic_hidden(workload, n_tok, H)
    ref = oracle(workload, 0, x, host_router(workload, 0))
    check_layer_full(gpu, dev_w, x, ref, "gemv")


@pytest.mark.timeout(300)
@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_prefill_2048_zipf_full_size(gpu, precision):
    workload, n_tok = 3, 2048  # the benchmark's prefill workload
    host = host_router(workload, 0)
    x = moe.synthetic_hidden(workload, n_tok, H)
    bias, _ = synth.zipf_router_bias(x, host["router_weight"], K, 1.1, 1000 * workload + 11)
    host["router_bias"] = bias
    dev_w = moe.MoELayerWeights.synthetic(workload, 0, H, I, E, gpu, bias)
    ref = oracle(workload, 0, x, host, precision)
    counts = np.bincount(ref["ids"].ravel(), minlength=E)
    assert counts.max() >= 1500  # the hot expert spans many 64-token GEMM units
    check_layer_full(gpu, dev_w, x, ref, "auto", precision)


@pytest.mark.timeout(400)
def test_stack_36_layers_full_size(gpu):
    workload, n_layers, n_tok = 4, 36, 64  # the benchmark's stacked workload, first decode step
    stack = moe.MoEStack.synthetic(workload, n_layers, H, I, E, gpu)
    x = moe.synthetic_hidden(workload, n_tok, H)
    trace: list = []
    ids = [torch.empty((n_tok, K), dtype=torch.int32, device=gpu) for _ in range(n_layers)]
    out = stack(bf16_tensor(x, gpu), trace=trace, ids=ids)
    torch.cuda.synchronize()
    assert torch.equal(out, trace[-1])
    h_in = x
    for layer in range(n_layers):
        got_bits = bf16_bits(trace[layer])
        assert np.isfinite(bf16_to_f32(got_bits)).all(), f"layer {layer}: non-finite hidden state"
        host = host_router(workload, layer)
        normed = rms_norm(h_in, moe.synthetic_norm_weight(workload, layer, H))
        want_ids, _ = orr.topk(orr.router_logits(normed, host["router_weight"], host["router_bias"]), K)
        assert np.array_equal(ids[layer].cpu().numpy(), want_ids), f"layer {layer} routing"
        if layer in (0, 17, 35):
            ref = oracle(workload, layer, normed, host)
            want = bf16_to_f32(residual_add(h_in, ref["out"])).astype(np.float64)
            got = bf16_to_f32(got_bits).astype(np.float64)
            w = bf16_to_f32(ref["weights"])
            slack = 2.0 ** -7 * np.sum(np.abs(w[:, :, None] * ref["expert_out"]), axis=1) + 2.0 ** -8 * np.abs(want)
            err = np.abs(got - want)
            assert (err <= ATOL + RTOL * np.abs(want) + slack).all(), f"layer {layer}: worst error {err.max():.3e}"
        h_in = got_bits
