"""Long inputs: one call up to KLC_LAYER_MAX_TOKENS tokens, row chunks past it.

9,700 tokens at top-4 are 38,800 (token, slot) pairs, which one call takes
(the dispatch of 1024 pairs and more runs over one workgroup per expert and
stages no pair in LDS): routing must equal the oracle's exactly and the
outputs stay within the expert tolerance.  Past KLC_LAYER_MAX_TOKENS,
``MoELayer.forward`` splits the rows into chunks; every token depends on its
own row only (streamed_moe_router.py:257-329 routes one token per call), so
the split result must equal separate calls on any split of the rows, bit for
bit, with no seam at the chunk boundary.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor
from klcquant_amd import _native as nat
from klcquant_amd import moe, ops
from klcquant_amd.mxfp4_expert import ResidentExpertStore
from klcquant_amd.streamed_moe_router import StreamedMoERouter
from test_gpu_experts import assert_final_close, oracle_layer

pytestmark = pytest.mark.gpu

H, I, E, K = 256, 128, 16, 4
WORKLOAD = 71
N_TOK = 9700


@pytest.fixture(scope="module")
def setup(gpu):
    assert N_TOK * K > 38648 and N_TOK <= ops.max_tokens_per_call(K)
    host = moe.synthetic_host_layer(WORKLOAD, 0, H, I, E)
    dev_w = moe.MoELayerWeights.synthetic(WORKLOAD, 0, H, I, E, gpu)
    x = moe.synthetic_hidden(WORKLOAD, N_TOK, H)
    return host, dev_w, x, oracle_layer(host, x, K)


@pytest.mark.timeout(300)
@pytest.mark.parametrize("path", ["auto", "gemv"])
def test_layer_long_input(gpu, setup, path):
    host, dev_w, x, ref = setup
    layer = moe.MoELayer(dev_w, K, path=path)
    ids = torch.empty((N_TOK, K), dtype=torch.int32, device=gpu)
    wts = torch.empty((N_TOK, K), dtype=torch.bfloat16, device=gpu)
    out = layer.forward(bf16_tensor(x, gpu), ids=ids, weights=wts)
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy(), ref["ids"])
    assert np.array_equal(bf16_bits(wts), ref["weights"])
    assert_final_close(bf16_bits(out), ref)


@pytest.mark.timeout(300)
def test_route_long_input(gpu, setup):
    host, dev_w, x, ref = setup
    names = {"router.weight": "router_weight", "router.bias": "router_bias",
             "experts.gate_up_proj_bias": "gate_up_bias", "experts.down_proj_bias": "down_bias"}
    tensors = {f"model.layers.0.mlp.{k}": bf16_tensor(host[v], gpu) for k, v in names.items()}
    out, route = StreamedMoERouter(K).route(0, bf16_tensor(x, gpu), tensors, ResidentExpertStore({0: dev_w}),
                                            position=0)
    torch.cuda.synchronize()
    assert out.shape == (N_TOK, H)
    assert np.array_equal(np.array(route["experts"]), ref["ids"])
    assert len(route["expert_logs"]) == N_TOK
    assert_final_close(bf16_bits(out), ref)


@pytest.mark.timeout(300)
@pytest.mark.parametrize("path", ["auto", "gemv"])
def test_layer_splits_past_layer_limit(gpu, path):
    """66,000 tokens (past KLC_LAYER_MAX_TOKENS): forward() runs two chunks; the result equals two
    separate calls split elsewhere."""
    h, i, e, k, n = 64, 32, 8, 2, 66000
    assert n > nat.LAYER_MAX_TOKENS
    dev_w = moe.MoELayerWeights.synthetic(72, 0, h, i, e, gpu)
    layer = moe.MoELayer(dev_w, k, path=path)
    x = bf16_tensor(moe.synthetic_hidden(72, n, h), gpu)
    ids = torch.empty((n, k), dtype=torch.int32, device=gpu)
    out = layer.forward(x, ids=ids)
    cut = 33000
    ids_a = torch.empty((cut, k), dtype=torch.int32, device=gpu)
    ids_b = torch.empty((n - cut, k), dtype=torch.int32, device=gpu)
    out_a = layer.forward(x[:cut], ids=ids_a)
    out_b = layer.forward(x[cut:], ids=ids_b)
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy(), np.concatenate([ids_a.cpu().numpy(), ids_b.cpu().numpy()]))
    assert np.array_equal(bf16_bits(out), np.concatenate([bf16_bits(out_a), bf16_bits(out_b)]))


@pytest.mark.timeout(300)
def test_route_splits_past_layer_limit(gpu):
    """route() on a resident store past KLC_LAYER_MAX_TOKENS: one klc_moe_route call per row chunk and one
    read-back each; outputs and routing equal one layer forward over the whole input, bit for bit."""
    h, i, e, k, n = 64, 32, 8, 2, 66000
    dev_w = moe.MoELayerWeights.synthetic(73, 0, h, i, e, gpu)
    p = "model.layers.0.mlp"
    tensors = {f"{p}.router.weight": dev_w.router_weight, f"{p}.router.bias": dev_w.router_bias,
               f"{p}.experts.gate_up_proj_bias": dev_w.gate_up_bias, f"{p}.experts.down_proj_bias": dev_w.down_bias}
    x = bf16_tensor(moe.synthetic_hidden(73, n, h), gpu)
    ids = torch.empty((n, k), dtype=torch.int32, device=gpu)
    wts = torch.empty((n, k), dtype=torch.bfloat16, device=gpu)
    want = moe.MoELayer(dev_w, k).forward(x, ids=ids, weights=wts)
    out, route = StreamedMoERouter(k).route(0, x, tensors, ResidentExpertStore({0: dev_w}))
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(out), bf16_bits(want))
    assert route["experts"] == ids.cpu().tolist()
    assert route["weights"] == wts.float().cpu().tolist()
    assert len(route["expert_logs"]) == n and route["expert_logs"][-1][0]["expert"] == route["experts"][-1][0]


@pytest.mark.timeout(300)
@pytest.mark.parametrize("precision", ["bf16", "fp32"])
def test_gemm_down_planes_past_2gib(gpu, precision):
    """47,000 tokens at top-8 with a 2880-wide expert input: each of down's activation planes (pairs x 2880
    bf16) passes 2 GiB, past what the GEMM's 32-bit buffer offsets reach, so the down GEMM takes its
    64-bit-pointer form; the result equals two calls of half the rows (planes under 2 GiB), bit for bit."""
    h, i, e, k, n = 256, 2880, 16, 8, 47000
    assert n * k * i * 2 > 2**31 - 1 and (n // 2) * k * i * 2 < 2**31 - 1
    dev_w = moe.MoELayerWeights.synthetic(74, 0, h, i, e, gpu)
    layer = moe.MoELayer(dev_w, k, precision=precision, path="gemm")
    x = bf16_tensor(moe.synthetic_hidden(74, n, h), gpu)
    out = layer.forward(x)
    cut = n // 2
    out_a = layer.forward(x[:cut])
    out_b = layer.forward(x[cut:])
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(out), np.concatenate([bf16_bits(out_a), bf16_bits(out_b)]))


@pytest.mark.timeout(300)
@pytest.mark.parametrize("precision", ["bf16", "fp32"])
def test_gemm_gate_up_hidden_plane_past_2gib(gpu, precision):
    """380,000 tokens of a 2880-wide hidden state (2.19 GB of bf16, one call of the grouped gate_up GEMM at
    top-1, which has no token cap of its own): past the 32-bit buffer offsets, so gate_up takes its
    64-bit-pointer form; every (token, slot) row equals the row of two calls on half the tokens each (planes
    under 2 GiB, the buffer-offset form), bit for bit, in both down-input planes and the float32 SwiGLU
    output."""
    h, i, e, k, n = 2880, 64, 4, 1, 380_000
    assert n * h * 2 > 2**31 - 1 and (n // 2) * h * 2 < 2**31 - 1 and n * k <= nat.DISPATCH_MAX_PAIRS
    w = moe.MoELayerWeights.synthetic(75, 0, h, i, e, gpu)
    gen = torch.Generator(device=gpu).manual_seed(75)
    x = torch.randn((n, h), generator=gen, device=gpu).to(torch.bfloat16)
    ids = torch.randint(0, e, (n, k), generator=gen, device=gpu, dtype=torch.int32)

    def run(rows):
        disp = ops.dispatch(ids[rows].contiguous(), e)
        return ops.gate_up(w.gate_up_table, w.gate_up_bias, x[rows], k, disp, h, i, precision=precision,
                           want_raw=True, gemm=True)

    split, raw = run(slice(0, n))
    cut = n // 2
    split_a, raw_a = run(slice(0, cut))
    split_b, raw_b = run(slice(cut, n))
    torch.cuda.synchronize()
    assert torch.equal(split.view(torch.int16), torch.cat([split_a, split_b], dim=1).view(torch.int16))
    assert torch.equal(raw.view(torch.int32), torch.cat([raw_a, raw_b]).view(torch.int32))
    assert bool((split[0].view(torch.int16) != 0).any())
