"""Host-side checks of the layer-tensor loader (no GPU needed)."""

from __future__ import annotations

import pytest

from klcquant_amd.layer_tensors import LAYER_TENSOR_SUFFIXES, LayerTensorLoader, layer_tensor_names


def test_layer_tensor_names():
    names = layer_tensor_names(7)
    assert len(names) == len(set(names)) == 15
    assert names[0] == "model.layers.7.input_layernorm.weight"
    assert names[-1] == "model.layers.7.post_attention_layernorm.weight"
    assert "model.layers.7.self_attn.sinks" in names and "model.layers.7.mlp.router.weight" in names
    assert not any(s.endswith(("_blocks", "_scales")) for s in LAYER_TENSOR_SUFFIXES)


def test_loader_refuses_host_device(tmp_path):
    with pytest.raises(ValueError, match="GPU"):
        LayerTensorLoader(tmp_path, "cpu")
