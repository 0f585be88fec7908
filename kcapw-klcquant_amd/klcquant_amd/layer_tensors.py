"""A layer's dense tensors read from the shards straight into HBM.

Drop-in for ``StreamedTransformerExecutor._load_executable_layer_tensors``
(streamed_transformer_executor.py:318-370).  The reference opens each shard
with ``safe_open`` on every miss, reads every tensor into host memory,
converts floating-point tensors to the executor's dtype on the host, and
copies each through ``pin_memory().to(device)`` before a device-wide
synchronize.  Here the shards stay open (their headers parsed once), all of
a shard's tensors for the layer go through one staged copy
(``SafetensorShard.copy_rows_batch``: pread into a pinned ring, DMA to HBM,
one wait at the end), and the dtype conversion runs on the device.  The
cache and the accounting keep the reference's fields: ``layer_tensor_cache``
with its hit and miss counts and bytes, ``transfer_bytes`` and
``transfer_events`` entries ``{"kind": "original_tensor", "layer", "name",
"bytes"}`` (the bytes of the converted tensor).
"""

from __future__ import annotations

from pathlib import Path
from typing import Callable, Iterable

import torch

from .mxfp4_expert import SafetensorIndex

#: The names the executor loads per layer, in the reference's order
#: (streamed_transformer_executor.py:325-341).
LAYER_TENSOR_SUFFIXES = (
    "input_layernorm.weight",
    "self_attn.o_proj.bias",
    "self_attn.o_proj.weight",
    "self_attn.q_proj.bias",
    "self_attn.k_proj.bias",
    "self_attn.v_proj.bias",
    "self_attn.q_proj.weight",
    "self_attn.k_proj.weight",
    "self_attn.v_proj.weight",
    "self_attn.sinks",
    "mlp.router.bias",
    "mlp.router.weight",
    "mlp.experts.gate_up_proj_bias",
    "mlp.experts.down_proj_bias",
    "post_attention_layernorm.weight",
)


def layer_tensor_names(layer_idx: int) -> list[str]:
    prefix = f"model.layers.{layer_idx}"
    return [f"{prefix}.{suffix}" for suffix in LAYER_TENSOR_SUFFIXES]


class LayerTensorLoader:
    """Loads and (with ``pin_layer_tensors``) caches each layer's dense tensors on ``device``.

    ``skip``: names served elsewhere (the reference skips the quantized
    overrides' names, streamed_transformer_executor.py:344-345), as a
    collection or a predicate.  ``on_hit`` is called on every cache hit (the
    reference counts it in its scheduler, :320).
    """

    def __init__(self, model_dir: str | Path, device: torch.device | str, dtype: torch.dtype = torch.bfloat16,
                 support_dir: str | Path | None = None, pin_layer_tensors: bool = True,
                 skip: Iterable[str] | Callable[[str], bool] | None = None,
                 on_hit: Callable[[], None] | None = None) -> None:
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError(f"LayerTensorLoader copies to a GPU, got device {self.device}")
        self.dtype = dtype
        self.index = SafetensorIndex(model_dir, support_dir if support_dir is not None else model_dir)
        self.pin_layer_tensors = bool(pin_layer_tensors)
        if skip is None:
            self._skip = lambda name: False
        elif callable(skip):
            self._skip = skip
        else:
            names = frozenset(skip)
            self._skip = names.__contains__
        self._on_hit = on_hit
        self.layer_tensor_cache: dict[int, dict[str, torch.Tensor]] = {}
        self.layer_tensor_cache_hits = 0
        self.layer_tensor_cache_misses = 0
        self.layer_tensor_cache_bytes = 0
        self.transfer_bytes = 0
        self.transfer_events: list[dict] = []

    def load(self, layer_idx: int) -> dict[str, torch.Tensor]:
        """``{name: device tensor}`` of the layer (a new dict each call, as the reference returns)."""
        cached = self.layer_tensor_cache.get(layer_idx)
        if cached is not None:
            self.layer_tensor_cache_hits += 1
            if self._on_hit is not None:
                self._on_hit()
            return dict(cached)
        self.layer_tensor_cache_misses += 1
        by_file: dict[str, list[str]] = {}
        for name in layer_tensor_names(layer_idx):
            if self._skip(name):
                continue
            file = self.index.weight_map.get(name)
            if file:
                by_file.setdefault(file, []).append(name)
        stream = torch.cuda.current_stream(self.device)
        tensors: dict[str, torch.Tensor] = {}
        for names in by_file.values():
            shard = self.index.shard(names[0])
            requests = []
            for name in names:
                _, shape, _, _ = shard.info(name)
                if not shape:
                    raise ValueError(f"{shard.path}: layer tensor '{name}' is a scalar")
                requests.append((name, 0, shape[0]))
            for name, raw in zip(names, shard.copy_rows_batch(requests, self.device, stream)):
                tensor = raw.to(self.dtype) if raw.is_floating_point() else raw
                tensors[name] = tensor
                nbytes = tensor.numel() * tensor.element_size()
                self.transfer_bytes += nbytes
                self.transfer_events.append({"kind": "original_tensor", "layer": layer_idx, "name": name,
                                             "bytes": nbytes})
        if self.pin_layer_tensors:
            self.layer_tensor_cache[layer_idx] = tensors
            self.layer_tensor_cache_bytes += sum(t.numel() * t.element_size() for t in tensors.values())
            return dict(tensors)
        return tensors

    __call__ = load

    def clear(self) -> None:
        self.layer_tensor_cache.clear()
        self.layer_tensor_cache_bytes = 0
