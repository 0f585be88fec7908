"""Decode attention with a device-resident KV cache.

Same surface as the reference's streamed_attention.py (AttentionConfig,
rms_norm, yarn_attention_scaling, yarn_inv_freq, rope_cos_sin, apply_rope,
StreamedAttention) and kv_cache_manager.py (KVCacheManager's methods, here
``DeviceKVCache``).  What differs underneath:

* the cache is a preallocated ring per layer in HBM ([cap, n_kv, head_dim] of
  the cache type); ``append`` writes one slot and ``get`` only builds the
  stacked view the reference API returns;
* ``StreamedAttention.forward`` with a ``DeviceKVCache`` runs RoPE + append in
  one kernel (klc_rope_append) and the scores / softmax with sinks / value
  sum over the window in klc_attn_decode; the q/k/v/o projections stay
  torch's ``F.linear`` (plain library GEMVs), so they are the reference's.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch

from . import _native

_KV_DTYPES = {"fp16": (torch.float16, 1), "bf16": (torch.bfloat16, 0)}  # KLC_DTYPE_F16 = 1, KLC_DTYPE_BF16 = 0


@dataclass
class AttentionConfig:
    """streamed_attention.py:11-24."""
    hidden_size: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    rope_theta: float = 150000.0
    rope_factor: float = 1.0
    rope_beta_fast: float = 32.0
    rope_beta_slow: float = 1.0
    rope_original_max_position_embeddings: int = 4096
    rope_truncate: bool = False
    sliding_window: int | None = None
    rms_norm_eps: float = 1e-5


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """streamed_attention.py:27-28 (for 2-D bfloat16 rows, ops.rms_norm runs it on the GPU)."""
    scale = torch.rsqrt(torch.mean(x.float() * x.float(), dim=-1, keepdim=True) + eps).to(x.dtype)
    return x * scale * weight


def yarn_attention_scaling(config: AttentionConfig) -> float:
    """streamed_attention.py:30-36."""
    f = float(config.rope_factor)
    return 1.0 if f <= 1.0 else 0.1 * math.log(f) + 1.0


def yarn_inv_freq(config: AttentionConfig, device: torch.device) -> torch.Tensor:
    """float32 [head_dim / 2] YaRN inverse frequencies (streamed_attention.py:39-78),
    computed with the same float32 torch ops on ``device``."""
    d, base = int(config.head_dim), float(config.rope_theta)

    def corr(rot: float) -> float:
        return d * math.log(config.rope_original_max_position_embeddings / (rot * 2 * math.pi)) / (2 * math.log(base))

    lo, hi = corr(float(config.rope_beta_fast)), corr(float(config.rope_beta_slow))
    if config.rope_truncate:
        lo, hi = math.floor(lo), math.ceil(hi)
    lo, hi = max(lo, 0.0), min(hi, float(d - 1))
    if lo == hi:
        hi += 0.001
    ramp = torch.clamp((torch.arange(d // 2, dtype=torch.float32, device=device) - lo) / (hi - lo), 0, 1)
    pos = base ** (torch.arange(0, d, 2, dtype=torch.float32, device=device) / d)
    extrap_share = 1 - ramp
    return (1.0 / (float(config.rope_factor) * pos)) * (1 - extrap_share) + (1.0 / pos) * extrap_share


def rope_cos_sin(config: AttentionConfig, position: int, device: torch.device,
                 dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    """streamed_attention.py:81-85: cos/sin of the position times the YaRN scaling, in ``dtype``."""
    ang = yarn_inv_freq(config, device).float() * float(position)
    s = yarn_attention_scaling(config)
    return (torch.cos(ang) * s).to(dtype), (torch.sin(ang) * s).to(dtype)


def apply_rope(q: torch.Tensor, k: torch.Tensor, position: int, config: AttentionConfig):
    """streamed_attention.py:88-98 in torch (the kernel path fuses it)."""
    cos, sin = rope_cos_sin(config, position, q.device, q.dtype)

    def rot(x: torch.Tensor) -> torch.Tensor:
        a, b = torch.chunk(x, 2, dim=-1)
        return torch.cat((a * cos - b * sin, b * cos + a * sin), dim=-1)

    return rot(q), rot(k)


class DeviceKVCache:
    """KVCacheManager (kv_cache_manager.py:18-113) for the "fp16" and "bf16"
    precisions, kept as one ring per layer in device memory.

    ``offload_to_cpu`` is accepted (the executor passes its
    ``offload_kv_cache`` setting, streamed_transformer_executor.py) but the
    ring stays in HBM: the attention kernels read it in place, and a gpt-oss
    cache of 4,096 tokens is about 8 MB per layer of the 288 GB.  ``get``
    returns tensors on the compute device either way, as the reference's does.
    """

    def __init__(self, device: torch.device, offload_to_cpu: bool = False, max_tokens: int | None = None,
                 precision: str = "fp16", capacity: int = 4096) -> None:
        if precision not in _KV_DTYPES:
            raise ValueError(f"unsupported KV cache precision for the device cache: {precision}")
        self.offload_to_cpu = bool(offload_to_cpu)  # recorded; the ring stays on the device
        self.device = torch.device(device)
        self.compute_device = self.device
        self.max_tokens = max_tokens
        self.precision = precision
        self.dtype, self.kv_code = _KV_DTYPES[precision]
        self._initial = int(max_tokens) if max_tokens else int(capacity)
        self.layers: dict[int, dict] = {}  # layer -> {k, v, cap, total}
        self.corruption_events: list[dict] = []

    # ---- ring bookkeeping ---------------------------------------------------------
    def _ring(self, layer_idx: int, n_kv: int, head_dim: int) -> dict:
        r = self.layers.get(layer_idx)
        if r is None:
            cap = self._initial
            r = {"k": torch.empty((cap, n_kv, head_dim), dtype=self.dtype, device=self.device),
                 "v": torch.empty((cap, n_kv, head_dim), dtype=self.dtype, device=self.device), "cap": cap, "total": 0}
            self.layers[layer_idx] = r
        elif not self.max_tokens and r["total"] >= r["cap"]:
            # unbounded cache: grow, keeping the tokens in order from slot 0
            k, v = self._ordered(r)
            cap = 2 * r["cap"]
            r["k"] = torch.empty((cap, n_kv, head_dim), dtype=self.dtype, device=self.device)
            r["v"] = torch.empty((cap, n_kv, head_dim), dtype=self.dtype, device=self.device)
            r["k"][: k.shape[0]] = k
            r["v"][: v.shape[0]] = v
            r["cap"] = cap
            r["total"] = k.shape[0]
        return r

    @staticmethod
    def _span(r: dict, window: int | None) -> tuple[int, int]:
        held = min(r["total"], r["cap"])
        count = min(held, window) if window else held
        first = (r["total"] - count) % r["cap"]
        return first, count

    def _ordered(self, r: dict, window: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        first, count = self._span(r, window)
        idx = (torch.arange(count, device=self.device) + first) % r["cap"]
        return r["k"][idx], r["v"][idx]

    def next_slot(self, layer_idx: int, n_kv: int, head_dim: int) -> tuple[dict, int]:
        r = self._ring(layer_idx, n_kv, head_dim)
        return r, r["total"] % r["cap"]

    # ---- KVCacheManager API -----------------------------------------------------------
    def append(self, layer_idx: int, key: torch.Tensor, value: torch.Tensor) -> None:
        r, slot = self.next_slot(layer_idx, key.shape[0], key.shape[1])
        r["k"][slot] = key.detach().to(self.dtype)
        r["v"][slot] = value.detach().to(self.dtype)
        r["total"] += 1

    def get(self, layer_idx: int, window: int | None = None):
        r = self.layers.get(layer_idx)
        if r is None or r["total"] == 0:
            return None, None
        return self._ordered(r, window)

    def stats(self):
        from types import SimpleNamespace

        tokens = max((min(r["total"], r["cap"]) for r in self.layers.values()), default=0)
        resident = sum(2 * min(r["total"], r["cap"]) * r["k"][0].numel() * r["k"].element_size()
                       for r in self.layers.values())
        return SimpleNamespace(tokens=tokens, resident_bytes=resident, device=str(self.device))

    def extended_stats(self) -> dict:
        s = self.stats()
        return {"tokens": s.tokens, "resident_bytes": s.resident_bytes, "resident_mb": round(s.resident_bytes / 2**20, 6),
                "device": s.device, "precision": self.precision, "corruption_events": [],
                "cache_corruption_likelihood": 0.0}

    def snapshot(self) -> dict:
        out = {}
        for layer, r in self.layers.items():
            k, v = self._ordered(r)
            out[layer] = ([t.clone() for t in k], [t.clone() for t in v])
        return out

    def restore(self, snapshot: dict) -> None:
        self.layers = {}
        for layer, (keys, values) in snapshot.items():
            for key, value in zip(keys, values):
                self.append(layer, key, value)

    def clear(self) -> None:
        self.layers.clear()


class StreamedAttention:
    """StreamedAttention (streamed_attention.py:101-152)."""

    def __init__(self, config: AttentionConfig) -> None:
        self.config = config
        self._tables: dict = {}
        self._workspace: torch.Tensor | None = None

    def _cos_sin(self, position: int, device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
        key = (int(position), str(device))
        t = self._tables.get(key)
        if t is None:
            t = rope_cos_sin(self.config, position, device, torch.bfloat16)
            if len(self._tables) > 4096:
                self._tables.clear()
            self._tables[key] = t
        return t

    def forward(self, layer_idx: int, hidden: torch.Tensor, tensors: dict, position: int, kv_cache,
                sliding_window: int | None = None):
        cfg = self.config
        prefix = f"model.layers.{layer_idx}.self_attn"
        lin = torch.nn.functional.linear
        q = lin(hidden, tensors[f"{prefix}.q_proj.weight"], tensors[f"{prefix}.q_proj.bias"]).view(cfg.num_heads, cfg.head_dim)
        k = lin(hidden, tensors[f"{prefix}.k_proj.weight"], tensors[f"{prefix}.k_proj.bias"]).view(cfg.num_kv_heads, cfg.head_dim)
        v = lin(hidden, tensors[f"{prefix}.v_proj.weight"], tensors[f"{prefix}.v_proj.bias"]).view(cfg.num_kv_heads, cfg.head_dim)
        if not isinstance(kv_cache, DeviceKVCache) or q.dtype != torch.bfloat16 or q.device.type != "cuda":
            raise ValueError("StreamedAttention runs on a DeviceKVCache with bfloat16 activations on the GPU")
        window = sliding_window if sliding_window is not None else cfg.sliding_window
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        q_rot, k_rot = torch.empty_like(q), torch.empty_like(k)
        cos, sin = self._cos_sin(position, q.device)
        ring, slot = kv_cache.next_slot(layer_idx, cfg.num_kv_heads, cfg.head_dim)
        stream = ctypes.c_void_p(torch.cuda.current_stream(q.device).cuda_stream)
        P = ctypes.c_void_p
        _native.call("klc_rope_append", P(q.data_ptr()), P(k.data_ptr()), P(v.data_ptr()), P(cos.data_ptr()),
                     P(sin.data_ptr()), P(q_rot.data_ptr()), P(k_rot.data_ptr()), P(ring["k"].data_ptr()),
                     P(ring["v"].data_ptr()), slot, ring["cap"], cfg.num_heads, cfg.num_kv_heads, cfg.head_dim,
                     kv_cache.kv_code, stream)
        ring["total"] += 1
        first, count = kv_cache._span(ring, window)
        need = _native.call("klc_attn_workspace_bytes", cfg.num_heads, cfg.head_dim, count)
        if self._workspace is None or self._workspace.numel() < need or self._workspace.device != q.device:
            self._workspace = torch.empty(max(need, 1 << 20), dtype=torch.uint8, device=q.device)
        sinks = tensors.get(f"{prefix}.sinks")
        if sinks is not None:
            sinks = sinks.to(torch.bfloat16).contiguous()
        context = torch.empty((cfg.num_heads, cfg.head_dim), dtype=torch.bfloat16, device=q.device)
        _native.call("klc_attn_decode", P(q_rot.data_ptr()), P(ring["k"].data_ptr()), P(ring["v"].data_ptr()),
                     P(0 if sinks is None else sinks.data_ptr()), ring["cap"], first, count, cfg.num_heads,
                     cfg.num_kv_heads, cfg.head_dim, kv_cache.kv_code, P(self._workspace.data_ptr()),
                     self._workspace.numel(), P(context.data_ptr()), stream)
        o_weight = tensors[f"{prefix}.o_proj.weight"]
        out = lin(context.reshape(-1).to(o_weight.dtype), o_weight, tensors[f"{prefix}.o_proj.bias"])
        qf, kf, qp, kp = q_rot.float(), k_rot.float(), q.float(), k.float()
        diagnostics = {
            "rope_position": int(position),
            "rope_attention_scaling": float(yarn_attention_scaling(cfg)),
            "sliding_window": sliding_window,
            "q_pre_rope_norm": float(torch.linalg.vector_norm(qp).item()),
            "k_pre_rope_norm": float(torch.linalg.vector_norm(kp).item()),
            "q_post_rope_norm": float(torch.linalg.vector_norm(qf).item()),
            "k_post_rope_norm": float(torch.linalg.vector_norm(kf).item()),
            "q_rope_delta_norm": float(torch.linalg.vector_norm(qf - qp).item()),
            "k_rope_delta_norm": float(torch.linalg.vector_norm(kf - kp).item()),
            "q_post_rope_nonfinite_count": int((~torch.isfinite(q_rot)).sum().item()),
            "k_post_rope_nonfinite_count": int((~torch.isfinite(k_rot)).sum().item()),
        }
        return out, diagnostics
