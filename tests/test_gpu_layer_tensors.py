"""LayerTensorLoader against the executor's safe_open chain (streamed_transformer_executor.py:318-370).

Two layers' dense tensors are spread over two shards with bf16, float32 and
float16 entries; every tensor must come out byte-identical to ``safe_open``
-> ``.to(dtype)`` -> ``pin_memory().to(device)``, with the reference's
cache counts and transfer accounting.
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from klcquant_amd.layer_tensors import LayerTensorLoader, layer_tensor_names

pytestmark = pytest.mark.gpu

H, NQ, NKV, D, E, I = 256, 8, 2, 32, 16, 128


def shapes() -> dict[str, tuple[int, ...]]:
    return {
        "input_layernorm.weight": (H,), "self_attn.o_proj.bias": (H,), "self_attn.o_proj.weight": (H, NQ * D),
        "self_attn.q_proj.bias": (NQ * D,), "self_attn.k_proj.bias": (NKV * D,), "self_attn.v_proj.bias": (NKV * D,),
        "self_attn.q_proj.weight": (NQ * D, H), "self_attn.k_proj.weight": (NKV * D, H),
        "self_attn.v_proj.weight": (NKV * D, H), "self_attn.sinks": (NQ,), "mlp.router.bias": (E,),
        "mlp.router.weight": (E, H), "mlp.experts.gate_up_proj_bias": (E, 2 * I),
        "mlp.experts.down_proj_bias": (E, H), "post_attention_layernorm.weight": (H,),
    }


@pytest.fixture(scope="module")
def checkpoint(tmp_path_factory):
    from safetensors.torch import save_file

    root = tmp_path_factory.mktemp("ckpt")
    rng = np.random.default_rng(5)
    dtypes = [torch.bfloat16, torch.float32, torch.float16]
    files = {0: {}, 1: {}}
    weight_map = {}
    for layer in (0, 1):
        for j, (suffix, shape) in enumerate(shapes().items()):
            name = f"model.layers.{layer}.{suffix}"
            t = torch.from_numpy(rng.standard_normal(shape).astype(np.float32) * 3.0).to(dtypes[(j + layer) % 3])
            shard = (j + layer) % 2
            files[shard][name] = t
            weight_map[name] = f"model-{shard:05d}.safetensors"
    files[1]["model.layers.0.mlp.experts.gate_up_proj_blocks"] = torch.zeros((E, 2 * I, H // 32, 16), dtype=torch.uint8)
    weight_map["model.layers.0.mlp.experts.gate_up_proj_blocks"] = "model-00001.safetensors"
    for shard, tensors in files.items():
        save_file(tensors, str(root / f"model-{shard:05d}.safetensors"))
    (root / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))
    return root, weight_map


def reference_chain(root, weight_map, layer, device, dtype, skip=()):
    from safetensors import safe_open

    by_shard: dict[str, list[str]] = {}
    for name in layer_tensor_names(layer):
        if name in skip:
            continue
        by_shard.setdefault(weight_map[name], []).append(name)
    out, events = {}, []
    for shard, names in by_shard.items():
        with safe_open(str(root / shard), framework="pt", device="cpu") as handle:
            for name in names:
                t = handle.get_tensor(name)
                if t.is_floating_point():
                    t = t.to(dtype)
                out[name] = t.pin_memory().to(device, non_blocking=True)
                events.append({"kind": "original_tensor", "layer": layer, "name": name,
                               "bytes": t.numel() * t.element_size()})
    torch.cuda.synchronize()
    return out, events


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_layer_tensors_match_safe_open_chain(gpu, checkpoint, dtype):
    root, weight_map = checkpoint
    hits = []
    loader = LayerTensorLoader(root, gpu, dtype=dtype, on_hit=lambda: hits.append(1))
    want_events = []
    for layer in (0, 1):
        got = loader.load(layer)
        torch.cuda.synchronize()
        want, events = reference_chain(root, weight_map, layer, gpu, dtype)
        want_events += events
        assert list(got) == list(want)
        for name in want:
            assert got[name].dtype == want[name].dtype and got[name].shape == want[name].shape, name
            assert got[name].device == want[name].device
            assert torch.equal(got[name].view(torch.uint8), want[name].view(torch.uint8)), name
    assert loader.transfer_events == want_events
    assert loader.transfer_bytes == sum(e["bytes"] for e in want_events)
    assert loader.layer_tensor_cache_misses == 2 and loader.layer_tensor_cache_hits == 0
    again = loader.load(1)
    assert loader.layer_tensor_cache_hits == 1 and hits == [1]
    assert all(again[n] is loader.layer_tensor_cache[1][n] for n in again) and again is not loader.layer_tensor_cache[1]
    assert loader.layer_tensor_cache_bytes == loader.transfer_bytes
    assert len(loader.transfer_events) == len(want_events)  # a hit transfers nothing


def test_layer_tensors_skip_and_unpinned(gpu, checkpoint):
    root, weight_map = checkpoint
    skip = {"model.layers.0.self_attn.q_proj.weight", "model.layers.0.mlp.router.weight"}
    loader = LayerTensorLoader(root, gpu, skip=skip, pin_layer_tensors=False)
    got = loader.load(0)
    want, events = reference_chain(root, weight_map, 0, gpu, torch.bfloat16, skip)
    assert list(got) == list(want) and not skip & set(got)
    assert all(torch.equal(got[n], want[n]) for n in want)
    assert loader.transfer_events == events
    assert loader.layer_tensor_cache == {} and loader.layer_tensor_cache_bytes == 0
    loader.load(0)
    assert loader.layer_tensor_cache_misses == 2 and loader.layer_tensor_cache_hits == 0
    pred = LayerTensorLoader(root, gpu, skip=lambda n: n.endswith(".bias"))
    assert not any(n.endswith(".bias") for n in pred.load(1))
