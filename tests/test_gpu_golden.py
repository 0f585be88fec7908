"""GPU routing and combine against torch's own CPU results (tests/golden/).

The golden vectors are what the reference's torch CPU ops produced for 2048
seeded tokens of the 20B-shape (E = 32) and 120B-shape (E = 128) router
(streamed_moe_router.py:268-284, 497, 512-513; tests/golden/make_router_golden.py).
The GPU's logits are the correctly rounded bf16(f32(x . w) + b); torch's
F.linear accumulates in float32 and differs from that by one bf16 ulp in one
logit on a few tokens (listed in the fixture).  None of those logits is a
selected one or sits at the top-k boundary on these tokens, so the expert ids,
their order (ties included) and the bf16 weights must be torch's exactly on
all 2048 tokens.  The crafted boundary cases, where such a logit does decide
the routing, are in tests/test_gpu_router_boundary.py.
"""

from __future__ import annotations

import zlib
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor
from klcquant_amd import _native as nat
from klcquant_amd import moe, ops, synth
from oracle import router as orr

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
HIDDEN = 2880
K = 4


def load(name):
    g = np.load(GOLDEN / f"{name}.npz", allow_pickle=False)
    workload, n_exp = int(g["workload"]), int(g["n_experts"])
    x = moe.synthetic_hidden(workload, g["ids"].shape[0], HIDDEN)
    return g, workload, n_exp, x


def check_against_golden(name, g, logits_bits, ids, weights):
    diff_tokens = np.unique(g["logit_diffs"][:, 0])
    # the GPU's logits differ from torch's exactly at the fixture's recorded positions
    theirs = logits_bits.copy()
    d = g["logit_diffs"]
    theirs[d[:, 0], d[:, 1]] = d[:, 2].astype(np.uint16)
    crc = np.array([zlib.crc32(theirs[t].tobytes()) for t in range(theirs.shape[0])], dtype=np.uint32)
    assert np.array_equal(crc, g["logits_crc"])
    # every token, those with a differing F.linear logit included
    assert np.array_equal(ids, g["ids"].astype(ids.dtype))
    assert np.array_equal(weights, g["weights"])
    print(f"{name}: all {ids.shape[0]} tokens identical to torch ({len(diff_tokens)} with a differing F.linear "
          f"logit)", flush=True)


@pytest.mark.parametrize("name", ["router_e32", "router_e128"])
def test_router_kernels_match_torch_golden(gpu, name):
    """klc_moe_router_logits + klc_moe_topk_softmax over all 2048 tokens at once."""
    g, workload, n_exp, x = load(name)
    w = synth.random_normal_bf16(synth.tensor_seed(workload, "router_weight"), n_exp * HIDDEN, 0.0, 0.02)
    b = synth.random_normal_bf16(synth.tensor_seed(workload, "router_bias"), n_exp, 0.0, 0.01)
    logits = ops.router_logits(bf16_tensor(x, gpu), bf16_tensor(w.reshape(n_exp, HIDDEN), gpu), bf16_tensor(b, gpu))
    ids, _, weights = ops.topk_softmax(logits, K)
    torch.cuda.synchronize()
    check_against_golden(name, g, bf16_bits(logits), ids.cpu().numpy(), bf16_bits(weights))


@pytest.mark.parametrize("name", ["router_e32", "router_e128"])
def test_decode_layer_routing_matches_torch_golden(gpu, name):
    """The one-launch decode router inside klc_moe_layer, in 64-token batches."""
    g, workload, n_exp, x = load(name)
    layer = moe.MoELayer(moe.MoELayerWeights.synthetic(workload, 0, HIDDEN, HIDDEN, n_exp, gpu), K)
    w = synth.random_normal_bf16(synth.tensor_seed(workload, "router_weight"), n_exp * HIDDEN, 0.0, 0.02)
    b = synth.random_normal_bf16(synth.tensor_seed(workload, "router_bias"), n_exp, 0.0, 0.01)
    logits = orr.router_logits(x, w.reshape(n_exp, HIDDEN), b)  # equal to the GPU's (test_gpu_router)
    n = x.shape[0]
    ids = torch.empty((n, K), dtype=torch.int32, device=gpu)
    weights = torch.empty((n, K), dtype=torch.bfloat16, device=gpu)
    xt = bf16_tensor(x, gpu)
    for t0 in range(0, n, 64):
        layer.forward(xt[t0:t0 + 64], ids=ids[t0:t0 + 64], weights=weights[t0:t0 + 64])
    torch.cuda.synchronize()
    check_against_golden(name, g, logits, ids.cpu().numpy(), bf16_bits(weights))


@pytest.mark.parametrize("name", ["router_e32", "router_e128"])
def test_combine_matches_torch_bits(gpu, name):
    g = np.load(GOLDEN / f"{name}.npz", allow_pickle=False)
    n = g["combine_crc"].shape[0]
    outs = synth.random_normal_f32(int(g["combine_seed"]), n * K * HIDDEN, 0.0, 64.0).reshape(n * K, HIDDEN)
    out = ops.combine(torch.from_numpy(outs).to(gpu), bf16_tensor(g["weights"][:n], gpu), n, K)
    torch.cuda.synchronize()
    got = bf16_bits(out)
    crc = np.array([zlib.crc32(got[t].tobytes()) for t in range(n)], dtype=np.uint32)
    assert np.array_equal(crc, g["combine_crc"])


@pytest.mark.parametrize("n_exp,k", [(128, 4), (32, 4), (200, 4), (256, 4), (128, 1), (64, 20)])
@pytest.mark.parametrize("n_tok", [1, 16, 64, 128])
def test_decode_router_replays_torch_order_on_ties(gpu, n_tok, n_exp, k):
    """Router rows repeated across experts make many logits equal, so most tokens take the
    tie replay inside the one-launch decode router (one and several token tiles).  The expert
    counts cover each compiled form of the router: 32 / 128 / 200 experts with k = 4 (the
    kernels built for <= 64, 128 and 256 experts in torch's introselect regime) and the
    general kernel for k * 64 <= n (256 and 128 experts with k = 4 and 1) and k > 16 (20)."""
    hidden, inter = 256, 64
    weights = moe.MoELayerWeights.synthetic(5, 0, hidden, inter, n_exp, gpu)
    base = synth.random_normal_bf16(501, 3 * hidden, 0.0, 0.02).reshape(3, hidden)
    rw = base[synth.random_ints(502, n_exp, 0, 2)]
    rb = np.zeros(n_exp, np.uint16)
    weights.router_weight.copy_(bf16_tensor(rw, gpu))
    weights.router_bias.copy_(bf16_tensor(rb, gpu))
    x = synth.random_normal_bf16(503 + n_tok, n_tok * hidden).reshape(n_tok, hidden)
    xt = bf16_tensor(x, gpu)
    ids = torch.empty((n_tok, k), dtype=torch.int32, device=gpu)
    wts = torch.empty((n_tok, k), dtype=torch.bfloat16, device=gpu)
    if k <= K:
        # the layer's own launch: routing, then the dispatch of its experts
        moe.MoELayer(weights, k).forward(xt, ids=ids, weights=wts)
    else:
        # routing only (klc_moe_select: the same one-launch router, no dispatch)
        ws = torch.zeros(ops.workspace_bytes(n_tok, hidden, inter, n_exp, k), dtype=torch.uint8, device=gpu)
        nat.call("klc_moe_select", ops._ptr(xt), ops._ptr(weights.router_weight), ops._ptr(weights.router_bias),
                 n_tok, hidden, n_exp, k, ops._ptr(ws), ws.numel(), ops._ptr(ids), ops._ptr(wts), ops._stream(gpu))
    torch.cuda.synchronize()
    logits = orr.router_logits(x, rw, rb)
    want_ids, want_vals = orr.topk(logits, k)
    assert np.array_equal(ids.cpu().numpy(), want_ids)
    assert np.array_equal(bf16_bits(wts), orr.softmax_weights(want_vals))
    # nearly every token has equal values among its k + 1 largest logits
    srt = np.sort(synth.bf16_bits_to_f32(logits), axis=1)[:, ::-1]
    assert np.count_nonzero(np.any(srt[:, :k] == srt[:, 1:k + 1], axis=1)) >= n_tok // 2
