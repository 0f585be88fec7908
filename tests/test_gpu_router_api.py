"""GPU parity of the reference-shaped API: ``StreamedMoERouter.route`` with a
resident and a streaming expert store, its fallbacks, and
``dequantize_mxfp4_matrix`` / ``Mxfp4ExpertStore.load_expert_matrix``.

Expected values come from the oracle on the same seeded inputs.  Selection
(experts, weights) and dequantized matrices are bit-exact; outputs use the
tolerances of test_gpu_experts (1e-2 + 2e-2 |ref| per expert output, plus the
bf16 combine slack); the per-expert norms in ``expert_logs`` follow from
those outputs to 2e-2 relative.
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor
from klcquant_amd import moe
from klcquant_amd.mxfp4_expert import Mxfp4ExpertStore, ResidentExpertStore, dequantize_mxfp4_matrix
from klcquant_amd.streamed_moe_router import RoutingLocalityConfig, StreamedMoERouter
from oracle import experts as oex
from oracle import mxfp4 as omx
from oracle.numerics import bf16_to_f32
from test_gpu_experts import assert_close, assert_final_close, oracle_layer

pytestmark = pytest.mark.gpu

H, I, E, K = 256, 128, 16, 4
WORKLOAD = 61


def layer_tensors(host, gpu, layer=0, drop=()):
    names = {"router.weight": "router_weight", "router.bias": "router_bias",
             "experts.gate_up_proj_bias": "gate_up_bias", "experts.down_proj_bias": "down_bias"}
    return {f"model.layers.{layer}.mlp.{k}": bf16_tensor(host[v], gpu) for k, v in names.items() if k not in drop}


@pytest.fixture(scope="module")
def setup(gpu):
    host = moe.synthetic_host_layer(WORKLOAD, 0, H, I, E)
    dev_w = moe.MoELayerWeights.synthetic(WORKLOAD, 0, H, I, E, gpu)
    return host, dev_w


def check_route(out, route, host, x, batched, precision="fp32"):
    ref = oracle_layer(host, x, K, precision)
    experts = route["experts"] if batched else [route["experts"]]
    weights = route["weights"] if batched else [route["weights"]]
    assert experts == ref["ids"].tolist()
    assert weights == bf16_to_f32(ref["weights"]).astype(np.float64).tolist()
    assert_final_close(bf16_bits(out), ref, precision)
    logs = route["expert_logs"] if batched else [route["expert_logs"]]
    for t, row in enumerate(logs):
        assert [entry["expert"] for entry in row] == experts[t]
        for j, entry in enumerate(row):
            assert entry["routing_weight"] == weights[t][j]
            np.testing.assert_allclose(entry["gate_up_norm"], np.linalg.norm(ref["gated"][t, j]), rtol=2e-2)
            np.testing.assert_allclose(entry["output_norm"], np.linalg.norm(ref["expert_out"][t, j]), rtol=2e-2)
    return ref


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_route_single_token_resident_store(gpu, setup, precision):
    host, dev_w = setup
    x = moe.synthetic_hidden(WORKLOAD, 1, H)
    router = StreamedMoERouter(K, 7.0, matmul_precision=precision)
    store = ResidentExpertStore({0: dev_w})
    out, route = router.route(0, bf16_tensor(x[0], gpu), layer_tensors(host, gpu), store, position=3)
    assert out.shape == (H,) and out.dtype == torch.bfloat16
    assert route["mode"] == "mxfp4_expert_matmul" and route["active_expert_cap"] == K
    assert route["raw_experts"] == route["experts"] and route["sticky_adjusted"] is False
    check_route(out, route, host, x, False, precision)
    st = router.stats.to_json()
    assert st["routed_tokens"] == 1 and st["route_events"][0]["position"] == 3
    assert store.cache.stats.hits == 2 * K
    json.dumps(store.to_json())


def test_route_batch_resident_store(gpu, setup):
    host, dev_w = setup
    x = moe.synthetic_hidden(WORKLOAD, 12, H, step=1)
    router = StreamedMoERouter(K)
    out, route = router.route(0, bf16_tensor(x, gpu), layer_tensors(host, gpu), ResidentExpertStore({0: dev_w}),
                              position=list(range(12)))
    assert out.shape == (12, H)
    check_route(out, route, host, x, True)
    assert router.stats.routed_tokens == 12


def write_checkpoint(path, host, layer=0):
    from safetensors.torch import save_file

    prefix = f"model.layers.{layer}.mlp.experts"
    tensors = {f"{prefix}.gate_up_proj_blocks": torch.from_numpy(host["gate_up_blocks"]),
               f"{prefix}.gate_up_proj_scales": torch.from_numpy(host["gate_up_scales"]),
               f"{prefix}.down_proj_blocks": torch.from_numpy(host["down_blocks"]),
               f"{prefix}.down_proj_scales": torch.from_numpy(host["down_scales"])}
    save_file(tensors, str(path / "model-00001.safetensors"))
    (path / "model.safetensors.index.json").write_text(
        json.dumps({"weight_map": {name: "model-00001.safetensors" for name in tensors}}))


def test_route_streaming_store_matches_resident(gpu, setup, tmp_path):
    host, dev_w = setup
    write_checkpoint(tmp_path, host)
    x = moe.synthetic_hidden(WORKLOAD, 1, H, step=2)
    tensors = layer_tensors(host, gpu)
    per_expert = (dev_w.gate_up.shape[1] + dev_w.down.shape[1])
    store = Mxfp4ExpertStore(tmp_path, tmp_path, gpu, dtype=torch.bfloat16, cache_bytes=E * per_expert)
    router = StreamedMoERouter(K)
    out, route = router.route(0, bf16_tensor(x[0], gpu), tensors, store)
    check_route(out, route, host, x, False)
    assert store.cache.stats.misses == 2 * K and store.cache.stats.hits == 0
    assert store.resident_experts(0) == set(route["experts"])
    out2, route2 = router.route(0, bf16_tensor(x[0], gpu), tensors, store, position=1)
    assert store.cache.stats.hits == 2 * K and store.cache.stats.misses == 2 * K
    assert torch.equal(out, out2) and route2["experts"] == route["experts"]
    delta = router.stats.cache_delta_events[-1]
    assert (delta["hits"], delta["misses"]) == (2 * K, 0)
    resident, _ = StreamedMoERouter(K).route(0, bf16_tensor(x[0], gpu), tensors, ResidentExpertStore({0: dev_w}))
    assert torch.equal(out, resident)
    json.dumps(store.to_json())


def test_store_load_expert_matrix_is_exact(gpu, setup, tmp_path):
    host, _ = setup
    write_checkpoint(tmp_path, host)
    store = Mxfp4ExpertStore(tmp_path, tmp_path, gpu, dtype=torch.bfloat16, cache_bytes=1 << 30)
    for e, proj in [(3, "gate_up_proj"), (11, "down_proj")]:
        got = store.load_expert_matrix(0, e, proj)
        want = omx.dequantize(host[f"{proj[:-5]}_blocks"][e], host[f"{proj[:-5]}_scales"][e], "bf16")
        assert np.array_equal(bf16_bits(got), want)
    store.pin_experts([(0, 5, "down_proj")])
    assert (0, 5, "down_proj") in store.cache.pinned


def test_store_split_shards_take_the_copy_then_pack_path(gpu, setup, tmp_path):
    """Blocks and scales in different shards: staged copies, then the pack."""
    from safetensors.torch import save_file

    host, _ = setup
    prefix = "model.layers.0.mlp.experts"
    blocks = {f"{prefix}.{p}_blocks": torch.from_numpy(host[f"{p[:-5]}_blocks"]) for p in ("gate_up_proj", "down_proj")}
    scales = {f"{prefix}.{p}_scales": torch.from_numpy(host[f"{p[:-5]}_scales"]) for p in ("gate_up_proj", "down_proj")}
    save_file(blocks, str(tmp_path / "model-00001.safetensors"))
    save_file(scales, str(tmp_path / "model-00002.safetensors"))
    wmap = {**{n: "model-00001.safetensors" for n in blocks}, **{n: "model-00002.safetensors" for n in scales}}
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wmap}))
    store = Mxfp4ExpertStore(tmp_path, tmp_path, gpu, dtype=torch.bfloat16, cache_bytes=1 << 30)
    for e, proj in [(4, "gate_up_proj"), (9, "down_proj")]:
        got = store.load_expert_matrix(0, e, proj)
        want = omx.dequantize(host[f"{proj[:-5]}_blocks"][e], host[f"{proj[:-5]}_scales"][e], "bf16")
        assert np.array_equal(bf16_bits(got), want)
    assert store.cache.stats.miss_loaded_bytes == sum(
        host[f"{p}_blocks"][0].nbytes + host[f"{p}_scales"][0].nbytes for p in ("gate_up", "down"))


def test_store_prefetch_then_consume(gpu, setup, tmp_path):
    host, _ = setup
    write_checkpoint(tmp_path, host)
    store = Mxfp4ExpertStore(tmp_path, tmp_path, gpu, cache_bytes=1 << 30, async_prefetch=True)
    store.prefetch_experts(0, [2, 7])
    got = store.load_expert_matrix(0, 7, "down_proj")
    assert got.dtype == torch.float16
    want = omx.dequantize(host["down_blocks"][7], host["down_scales"][7], "f16")
    assert np.array_equal(got.view(torch.int16).cpu().numpy().view(np.uint16), want.view(np.uint16))
    store.close()
    js = store.to_json()
    assert js["prefetch_submitted"] == 4 and js["prefetch_failed"] == 0


def test_store_quant_loader_branch(gpu, setup, tmp_path):
    """A quantized loader that owns the expert tensors (mxfp4_expert.py:516-522): the full tensor comes
    back as floats with a uint8 meta dtype, is rounded and clamped to bytes, copied and packed."""
    from types import SimpleNamespace

    host, _ = setup
    write_checkpoint(tmp_path, host)
    prefix = "model.layers.0.mlp.experts"

    class Loader:
        tensor_index = {f"{prefix}.{p}_{kind}": None for p in ("gate_up_proj", "down_proj")
                        for kind in ("blocks", "scales")}
        calls = []

        def load_tensor(self, name, dtype=None):
            self.calls.append(name)
            arr = host[name.split(".")[-1].replace("_proj", "")]
            return torch.from_numpy(arr).to(torch.float32) + 0.25, SimpleNamespace(dtype="torch.uint8")

    loader = Loader()
    store = Mxfp4ExpertStore(tmp_path, tmp_path, gpu, dtype=torch.bfloat16, cache_bytes=1 << 30, quant_loader=loader)
    for e, proj in [(6, "gate_up_proj"), (13, "down_proj")]:
        got = store.load_expert_matrix(0, e, proj)
        want = omx.dequantize(host[f"{proj[:-5]}_blocks"][e], host[f"{proj[:-5]}_scales"][e], "bf16")
        assert np.array_equal(bf16_bits(got), want)
    assert loader.calls == [f"{prefix}.gate_up_proj_blocks", f"{prefix}.gate_up_proj_scales",
                            f"{prefix}.down_proj_blocks", f"{prefix}.down_proj_scales"]


def test_async_prefetch_with_evictions_matches_resident(gpu, setup, tmp_path):
    """Background loaders bring the next tokens' experts in while the compute stream runs, and a cache of
    three experts evicts constantly: every route() output must equal the resident store's bit for bit."""
    host, dev_w = setup
    write_checkpoint(tmp_path, host)
    tensors = layer_tensors(host, gpu)
    per_expert = dev_w.gate_up.shape[1] + dev_w.down.shape[1]
    store = Mxfp4ExpertStore(tmp_path, tmp_path, gpu, dtype=torch.bfloat16, cache_bytes=3 * per_expert,
                             async_prefetch=True, max_prefetch_workers=2)
    resident = ResidentExpertStore({0: dev_w})
    x = moe.synthetic_hidden(WORKLOAD, 12, H, step=5)
    ref_router, router = StreamedMoERouter(K), StreamedMoERouter(K)
    want = [ref_router.route(0, bf16_tensor(x[t], gpu), tensors, resident, position=t) for t in range(12)]
    for t in range(12):
        if t + 1 < 12:
            store.prefetch_experts(0, want[t + 1][1]["experts"])
        out, route = router.route(0, bf16_tensor(x[t], gpu), tensors, store, position=t)
        assert route["experts"] == want[t][1]["experts"]
        assert torch.equal(out, want[t][0]), t
    store.close()
    js = store.to_json()
    assert js["evictions"] > 0 and js["prefetch_failed"] == 0


def test_dequantize_matrix_default_fp16(gpu):
    from klcquant_amd import synth

    blocks, scales = synth.mxfp4_expert_tensors(3, 4, 1, 64, 96, scale_lo=100, scale_hi=140)
    got = dequantize_mxfp4_matrix(torch.from_numpy(blocks[0]).to(gpu), torch.from_numpy(scales[0]).to(gpu))
    assert got.dtype == torch.float16 and got.shape == (96, 64)
    want = omx.dequantize(blocks[0], scales[0], "f16")
    assert np.array_equal(got.view(torch.int16).cpu().numpy().view(np.uint16), want.view(np.uint16))
    with pytest.raises(ValueError, match="shape mismatch"):
        dequantize_mxfp4_matrix(torch.from_numpy(blocks[0]).to(gpu), torch.from_numpy(scales[0][:, :2]).to(gpu))


def test_route_fallback_modes(gpu, setup):
    host, dev_w = setup
    x = moe.synthetic_hidden(WORKLOAD, 3, H, step=3)
    ref = oracle_layer(host, x, K)
    xt = bf16_tensor(x, gpu)
    out, route = StreamedMoERouter(K).route(0, xt, layer_tensors(host, gpu), execute_experts=False)
    assert route["mode"] == "bias_only_moe" and route["experts"] == ref["ids"].tolist()
    assert np.array_equal(bf16_bits(out), oex.bias_only(host["down_bias"], ref["ids"], ref["weights"]))
    out, route = StreamedMoERouter(K).route(0, xt, layer_tensors(host, gpu, drop=("experts.down_proj_bias",)))
    assert route["mode"] == "router_only" and not out.any()
    out, route = StreamedMoERouter(K).route(0, xt, layer_tensors(host, gpu, drop=("experts.gate_up_proj_bias",)),
                                            ResidentExpertStore({0: dev_w}))
    assert route["mode"] == "mxfp4_missing_bias" and not out.any() and route["experts"] == ref["ids"].tolist()
    with pytest.raises(KeyError):
        StreamedMoERouter(K).route(1, xt, layer_tensors(host, gpu))


def test_locality_without_bonus_equals_plain_routing(gpu, setup):
    host, dev_w = setup
    x = moe.synthetic_hidden(WORKLOAD, 4, H, step=4)
    store = ResidentExpertStore({0: dev_w})
    plain_out, plain = StreamedMoERouter(K).route(0, bf16_tensor(x, gpu), layer_tensors(host, gpu), store)
    cfg = RoutingLocalityConfig(enabled=True, predictive_prefetch=True)
    router = StreamedMoERouter(K, locality_config=cfg)
    out, route = router.route(0, bf16_tensor(x, gpu), layer_tensors(host, gpu), store)
    assert route["experts"] == plain["experts"] and route["weights"] == plain["weights"]
    assert torch.equal(out, plain_out)
    # predictions for later rows come from the earlier rows' experts
    assert route["predicted_experts"][0] == [] and len(route["predicted_experts"][1]) == K


def test_locality_sticky_bonus_changes_selection(gpu, setup):
    """A large sticky bonus on an expert inside the candidate margin moves it into the top-k;
    the weights are the softmax of the adjusted scores (klc_moe_softmax_weights)."""
    host, dev_w = setup
    x = moe.synthetic_hidden(WORKLOAD, 1, H, step=5)
    ref = oracle_layer(host, x, E)  # all experts, descending
    order = ref["ids"][0].tolist()
    vals = bf16_to_f32(ref["logits"][0])
    # the best expert outside the top-k that is within 0.5 of the k-th logit
    cand = [e for e in order[K:] if vals[e] >= np.float32(vals[order[K - 1]]) - np.float32(0.5)]
    assert cand, "seeded input has no candidate within the margin"
    e = cand[0]
    router = StreamedMoERouter(K, locality_config=RoutingLocalityConfig(enabled=True, sticky_strength=1.0))
    router.sticky_scores[0] = {e: 5.0}
    out, route = router.route(0, bf16_tensor(x[0], gpu), layer_tensors(host, gpu), ResidentExpertStore({0: dev_w}))
    assert route["experts"][0] == e and route["sticky_adjusted"]
    assert route["raw_experts"] == order[:K]
    adjusted = [float(np.float32(vals[e]) + np.float32(5.0))] + [float(vals[j]) for j in order[:K - 1]]
    from oracle.router import softmax_weights
    assert route["weights"] == bf16_to_f32(softmax_weights(np.array([adjusted], np.float32)))[0].tolist()
    assert route["experts"][1:] == order[:K - 1]


def test_route_batch_gemm_streaming_matches_resident(gpu, setup, tmp_path):
    """40 tokens at E = 16 take the grouped GEMM (n_tokens * k >= 8 * n_experts) in both stores: the resident
    store's one-call path (klc_moe_route) and the streaming store's separate kernels give the same bits,
    the same routing and the same expert_logs."""
    host, dev_w = setup
    write_checkpoint(tmp_path, host)
    tensors = layer_tensors(host, gpu)
    per_expert = dev_w.gate_up.shape[1] + dev_w.down.shape[1]
    store = Mxfp4ExpertStore(tmp_path, tmp_path, gpu, dtype=torch.bfloat16, cache_bytes=E * per_expert)
    x = moe.synthetic_hidden(WORKLOAD, 40, H, step=6)
    assert moe.MoELayer(dev_w, K).layer_path(40) == "gemm"
    out_s, route_s = StreamedMoERouter(K).route(0, bf16_tensor(x, gpu), tensors, store, position=list(range(40)))
    out_r, route_r = StreamedMoERouter(K).route(0, bf16_tensor(x, gpu), tensors, ResidentExpertStore({0: dev_w}),
                                                position=list(range(40)))
    assert torch.equal(out_s, out_r)
    for key in ("experts", "weights", "raw_experts", "expert_logs", "mode", "active_expert_cap"):
        assert route_s[key] == route_r[key], key
    check_route(out_r, route_r, host, x, True)


def layer_tensor_dict(w, layer=0):
    p = f"model.layers.{layer}.mlp"
    return {f"{p}.router.weight": w.router_weight, f"{p}.router.bias": w.router_bias,
            f"{p}.experts.gate_up_proj_bias": w.gate_up_bias, f"{p}.experts.down_proj_bias": w.down_bias}


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_route_120b_matches_layer(gpu, precision):
    """gpt-oss-120B shape: route() on a resident store gives klc_moe_layer's bits and routing at decode batches
    (1, 8, 64, GEMV) and a prefill chunk (300 tokens, GEMM), one router serving every size in turn."""
    w = moe.MoELayerWeights.synthetic(75, 0, 2880, 2880, 128, gpu)
    layer = moe.MoELayer(w, 4, precision=precision)
    router = StreamedMoERouter(4, matmul_precision=precision)
    store = ResidentExpertStore({0: w})
    tensors = layer_tensor_dict(w)
    for step, n_tok in enumerate((8, 64, 1, 300, 8)):
        print(f"[route-120b] {precision} B={n_tok}", flush=True)
        xt = bf16_tensor(moe.synthetic_hidden(75, n_tok, 2880, step=step), gpu)
        ids = torch.empty((n_tok, 4), dtype=torch.int32, device=gpu)
        wts = torch.empty((n_tok, 4), dtype=torch.bfloat16, device=gpu)
        want = layer.forward(xt, ids=ids, weights=wts)
        out, route = router.route(0, xt, tensors, store, position=list(range(n_tok)))
        assert torch.equal(out, want), f"B={n_tok}"
        assert route["experts"] == ids.cpu().tolist()
        assert route["weights"] == wts.float().cpu().tolist()
        norms = np.array([[e["gate_up_norm"], e["output_norm"]] for row in route["expert_logs"] for e in row])
        assert norms.shape == (n_tok * 4, 2) and np.isfinite(norms).all() and (norms > 0).all()
    assert router.stats.routed_tokens == 8 + 64 + 1 + 300 + 8
    assert store.cache.stats.hits == 2 * 4 * router.stats.routed_tokens


@pytest.mark.parametrize("n_tok", [1, 37, 200])
def test_select_then_experts_equal_the_layer(gpu, n_tok):
    """klc_moe_select (one launch up to 128 tokens, logits + top-k above) and klc_moe_experts on its
    selection give klc_moe_layer's ids, weights and output bits, at the 20B expert count (E = 32)."""
    from klcquant_amd import _native as nat
    from klcquant_amd import ops

    h, i, e, k = 512, 256, 32, 4
    w = moe.MoELayerWeights.synthetic(76, 0, h, i, e, gpu)
    xt = bf16_tensor(moe.synthetic_hidden(76, n_tok, h), gpu)
    ids_l = torch.empty((n_tok, k), dtype=torch.int32, device=gpu)
    wts_l = torch.empty((n_tok, k), dtype=torch.bfloat16, device=gpu)
    want = moe.MoELayer(w, k).forward(xt, ids=ids_l, weights=wts_l)
    ws = torch.zeros(ops.workspace_bytes(n_tok, h, i, e, k), dtype=torch.uint8, device=gpu)
    ids = torch.empty_like(ids_l)
    wts = torch.empty_like(wts_l)
    stream = ops._stream(gpu)
    nat.call("klc_moe_select", ops._ptr(xt), ops._ptr(w.router_weight), ops._ptr(w.router_bias), n_tok, h, e, k,
             ops._ptr(ws), ws.numel(), ops._ptr(ids), ops._ptr(wts), stream)
    out = torch.empty_like(want)
    gated = torch.empty((n_tok * k, i), dtype=torch.float32, device=gpu)
    norms = torch.empty((n_tok * k, 2), dtype=torch.float32, device=gpu)
    nat.call("klc_moe_experts", ops._ptr(xt), ops._ptr(ids), ops._ptr(wts), ops._ptr(w.gate_up_table),
             ops._ptr(w.gate_up_bias), ops._ptr(w.down_table), ops._ptr(w.down_bias), n_tok, h, i, e, k, 7.0,
             nat.PRECISION_FP32, nat.PATH_AUTO, ops._ptr(ws), ws.numel(), ops._ptr(out), ops._ptr(gated),
             ops._ptr(norms), stream)
    torch.cuda.synchronize()
    assert torch.equal(ids, ids_l) and torch.equal(wts.view(torch.int16), wts_l.view(torch.int16))
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    assert torch.isfinite(norms).all() and (norms > 0).all()
