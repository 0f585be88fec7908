"""klc_moe_route_readback against klc_moe_route through the C-ABI: the same device outputs bit for bit,
and host copies of ids, weights and norms equal to the device record."""

from __future__ import annotations

import ctypes
import time

import numpy as np
import pytest
import torch

from conftest import bf16_tensor
from klcquant_amd import _native as nat
from klcquant_amd import moe, ops

pytestmark = pytest.mark.gpu


def run(w, x, k, readback, adjacent):
    """One klc_moe_route (readback False) or klc_moe_route_readback call; returns the device outputs
    (out, gated, ids, weight bits, norms words) and, for the readback, the host record and the selection
    as read when router_done fired."""
    dev = x.device
    n, hidden = x.shape
    pairs = n * k
    half = (pairs + 1) // 2
    ws = torch.zeros(ops.workspace_bytes(n, hidden, w.inter, w.n_experts, k), dtype=torch.uint8, device=dev)
    out = torch.empty_like(x)
    gated = torch.empty(pairs * w.inter, dtype=torch.float32, device=dev)
    words = pairs + half + 2 * pairs  # ids, bf16 weights, norms
    rec = torch.full((words + 32 + half,), -7, dtype=torch.int32, device=dev)
    ids_p = rec.data_ptr()
    # weights right after the ids or past the norms
    w_p = ids_p + 4 * pairs if adjacent else ids_p + 4 * (words + 32)
    assert (w_p - ids_p) // 4 + half <= rec.numel()
    norms_p = ids_p + 4 * (pairs + half)
    cur = torch.cuda.current_stream(dev)
    stream = ctypes.c_void_p(cur.cuda_stream)
    args = [x.data_ptr(), w.router_weight.data_ptr(), w.router_bias.data_ptr(), w.gate_up_table.data_ptr(),
            w.gate_up_bias.data_ptr(), w.down_table.data_ptr(), w.down_bias.data_ptr(), n, hidden, w.inter,
            w.n_experts, k, 7.0, nat.PRECISION_FP32, nat.PATH_AUTO, ws.data_ptr(), ws.numel(), out.data_ptr(),
            ids_p, w_p, gated.data_ptr()]
    host = sel = None
    if readback:
        host = torch.full((words + 1,), -9, dtype=torch.int32, pin_memory=True)
        hn = host.numpy()
        hn[words] = 0  # the tag word
        tag = 1000 + n
        nat.call("klc_moe_route_readback", *args, host.data_ptr(), tag, stream)
        deadline = time.perf_counter() + 5.0
        while hn[words] != tag and time.perf_counter() < deadline:
            pass
        sel = hn[:pairs + half].copy()  # read once the tag is there, before the layer's stream is waited for
        cur.synchronize()
        assert hn[words] == tag
        host = hn[:words].copy()
    else:
        nat.call("klc_moe_route", *args, norms_p, stream)
        cur.synchronize()
    raw = rec.cpu().numpy()
    w_off = (w_p - ids_p) // 4
    dev_out = (out.cpu(), gated.cpu(), raw[:pairs].copy(), raw[w_off:w_off + half].view(np.uint16)[:pairs].copy(),
               raw[pairs + half:words].copy())
    return dev_out, host, sel


@pytest.mark.parametrize("n_tok", [1, 5, 200])
@pytest.mark.parametrize("adjacent", [True, False])
def test_readback_equals_route(gpu, n_tok, adjacent):
    print(f"[route-readback] n_tok={n_tok} adjacent={adjacent}", flush=True)
    hidden, inter, n_exp, k = 2880, 2880, 128, 4
    w = moe.MoELayerWeights.synthetic(31, 0, hidden, inter, n_exp, gpu)
    x = bf16_tensor(moe.synthetic_hidden(31, n_tok, hidden, step=n_tok), gpu)
    want, _, _ = run(w, x, k, False, adjacent)
    got, host, sel = run(w, x, k, True, adjacent)
    assert torch.equal(want[0].view(torch.int16), got[0].view(torch.int16))
    assert torch.equal(want[1].view(torch.int32), got[1].view(torch.int32))
    assert np.array_equal(want[2], got[2]) and np.array_equal(want[3], got[3])
    pairs, half = n_tok * k, (n_tok * k + 1) // 2
    assert (got[2] >= 0).all() and (got[2] < n_exp).all()
    # the host record: the selection (complete when the tag arrived), then the norms of klc_moe_route
    assert np.array_equal(sel, host[:pairs + half])
    assert np.array_equal(host[:pairs], want[2])
    assert np.array_equal(host[pairs:pairs + half].view(np.uint16)[:pairs], want[3])
    assert np.array_equal(host[pairs + half:], want[4])


def test_readback_refuses_pageable_host_memory(gpu):
    hidden, inter, n_exp, k = 2880, 2880, 128, 4
    w = moe.MoELayerWeights.synthetic(31, 0, hidden, inter, n_exp, gpu)
    x = bf16_tensor(moe.synthetic_hidden(31, 1, hidden), gpu)
    ws = torch.zeros(ops.workspace_bytes(1, hidden, inter, n_exp, k), dtype=torch.uint8, device=gpu)
    out = torch.empty_like(x)
    gated = torch.empty(k * inter, dtype=torch.float32, device=gpu)
    rec = torch.zeros(64, dtype=torch.int32, device=gpu)
    pageable = np.zeros(64, np.int32)
    with pytest.raises(nat.KlcError, match="pinned host memory"):
        nat.call("klc_moe_route_readback", x.data_ptr(), w.router_weight.data_ptr(), w.router_bias.data_ptr(),
                 w.gate_up_table.data_ptr(), w.gate_up_bias.data_ptr(), w.down_table.data_ptr(),
                 w.down_bias.data_ptr(), 1, hidden, inter, n_exp, k, 7.0, nat.PRECISION_FP32, nat.PATH_AUTO,
                 ws.data_ptr(), ws.numel(), out.data_ptr(), rec.data_ptr(), rec.data_ptr() + 16, gated.data_ptr(),
                 pageable.ctypes.data, 1, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


@pytest.mark.parametrize("n_exp,k", [(128, 4), (128, 6), (16, 4)])
def test_route_single_token_tags(gpu, n_exp, k):
    """route() on a resident store, one token per call: the tag that releases the host's bookkeeping comes
    from the one-wave router (top-4) or from the tag kernel after the decode-batch router (top-6 is past the
    one-token expert kernels); garbage collections between calls change nothing, and every call's output
    and routing equal klc_moe_layer's."""
    import gc

    from klcquant_amd.mxfp4_expert import ResidentExpertStore
    from klcquant_amd.streamed_moe_router import StreamedMoERouter

    print(f"[route-tags] n_exp={n_exp} k={k}", flush=True)
    hidden, inter = (2880, 2880) if n_exp == 128 else (256, 128)
    w = moe.MoELayerWeights.synthetic(33, 0, hidden, inter, n_exp, gpu)
    p = "model.layers.0.mlp"
    tensors = {f"{p}.router.weight": w.router_weight, f"{p}.router.bias": w.router_bias,
               f"{p}.experts.gate_up_proj_bias": w.gate_up_bias, f"{p}.experts.down_proj_bias": w.down_bias}
    router = StreamedMoERouter(k)
    store = ResidentExpertStore({0: w})
    layer = moe.MoELayer(w, k)
    for step in range(4):
        x = bf16_tensor(moe.synthetic_hidden(33, 1, hidden, step=step), gpu)
        out, route = router.route(0, x[0], tensors, store, position=step)
        gc.collect()
        ids = torch.empty((1, k), dtype=torch.int32, device=gpu)
        want = layer.forward(x, ids=ids)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want[0].view(torch.int16))
        assert route["experts"] == ids[0].tolist()
        assert len(route["expert_logs"]) == k
    assert router._tag == 4
