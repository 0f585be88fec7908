"""MXFP4 expert weights: dequant and an HBM-resident expert store.

Same public surface as the reference's ``mxfp4_expert.py`` (FP4_VALUES,
ExpertCacheStats, ExpertWeightCache, dequantize_mxfp4_matrix,
Mxfp4ExpertStore), so callers such as the streamed executor construct and use
it unchanged.  What differs underneath:

* ``dequantize_mxfp4_matrix`` runs the gfx950 dequant kernel
  (klc_mxfp4_dequant); it is bit-exact with the reference's torch.ldexp
  arithmetic (mxfp4_expert.py:357-379) and takes GPU tensors only.
* the store caches experts **packed** (MXFP4 codes + E8M0 scales in the
  row-tile layout the expert kernels stream), 13.2 MB per gpt-oss expert
  instead of 49.8 MB dequantized, so the same ``cache_bytes`` budget holds
  3.76x more experts.  ``load_expert_matrix`` dequantizes from the packed copy
  on demand; the router's fused kernels read the packed copy directly.
* a miss reads the expert's slice from the checkpoint shard straight into the
  packed layout in HBM (klc_st_load_mxfp4_packed: pread into pinned staging,
  copy, pack, chunk by chunk on a side stream); there is no device-wide
  synchronisation.
"""

from __future__ import annotations

import json
import time
from collections import Counter
from concurrent.futures import Future, ThreadPoolExecutor
from dataclasses import dataclass
from pathlib import Path
from threading import RLock

import torch

from . import ops
from .safetensors_shard import SafetensorShard

# E2M1 code -> value (bit 3 is the sign); the same table as mxfp4_expert.py:17-34.
FP4_VALUES = [
    +0.0, +0.5, +1.0, +1.5, +2.0, +3.0, +4.0, +6.0,
    -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0,
]

PROJECTIONS = ("gate_up_proj", "down_proj")


@dataclass
class ExpertCacheStats:
    """Counters of the expert cache (field names of mxfp4_expert.py:37-65)."""

    hits: int = 0
    misses: int = 0
    evictions: int = 0
    loaded_bytes: int = 0
    dequantized_bytes: int = 0  # bytes put into the cache (packed bytes here)
    hit_bytes: int = 0
    miss_loaded_bytes: int = 0
    pinned_hits: int = 0
    lifetime_accesses: int = 0
    materializations: int = 0
    materialization_time_s: float = 0.0
    transfer_time_s: float = 0.0
    dequant_time_s: float = 0.0  # time of the on-device pack step of a miss
    blocked_on_prefetch_s: float = 0.0
    futures_waited: int = 0
    prefetch_submitted: int = 0
    prefetch_completed: int = 0
    prefetch_failed: int = 0
    prefetch_used: int = 0
    prefetch_skipped_resident: int = 0
    prefetch_skipped_pending: int = 0
    protected_eviction_skips: int = 0

    @property
    def hit_rate(self) -> float:
        total = self.hits + self.misses
        return self.hits / total if total else 0.0


Key = tuple[int, int, str]


def _nbytes(t: torch.Tensor) -> int:
    return t.numel() * t.element_size()


class ExpertWeightCache:
    """Byte-bounded cache of expert matrices keyed ``(layer, expert, proj)``.

    Eviction follows mxfp4_expert.py:183-245: among unpinned entries (and, with
    layer-aware quotas, the most over-quota layer's entries first), prefer those
    whose protection window has passed, then evict the lowest
    ``(future_score, frequency, last_access)``.  ``max_bytes <= 0`` disables
    insertion.  Thread safe.
    """

    def __init__(self, max_bytes: int, layer_count: int = 0, layer_aware: bool = False,
                 adaptive_layer_quota: bool = False, adaptive_layer_quota_strength: float = 1.5) -> None:
        self.max_bytes = max_bytes
        self.layer_count = max(int(layer_count), 0)
        self.layer_aware = layer_aware
        self.adaptive_layer_quota = adaptive_layer_quota
        self.adaptive_layer_quota_strength = max(float(adaptive_layer_quota_strength), 0.0)
        self.current_bytes = 0
        self.items: dict[Key, torch.Tensor] = {}
        self.item_bytes: dict[Key, int] = {}
        self.layer_bytes: Counter[int] = Counter()
        self.frequency: dict[Key, int] = {}
        self.last_access: dict[Key, int] = {}
        self.birth_access: dict[Key, int] = {}
        self.future_score: dict[Key, float] = {}
        self.protected_until: dict[Key, int] = {}
        self.prefetched: set[Key] = set()
        self.evicted_lifetimes: list[int] = []
        self.eviction_reasons: Counter[str] = Counter()
        self.layer_hits: Counter[int] = Counter()
        self.layer_misses: Counter[int] = Counter()
        self.layer_evictions: Counter[int] = Counter()
        self.layer_hit_bytes: Counter[int] = Counter()
        self.layer_loaded_bytes: Counter[int] = Counter()
        self.pinned: set[Key] = set()
        self.access_index = 0
        self.stats = ExpertCacheStats()
        self.lock = RLock()

    def get(self, key: Key) -> torch.Tensor | None:
        with self.lock:
            self.access_index += 1
            self.stats.lifetime_accesses += 1
            value = self.items.get(key)
            if value is None:
                self.stats.misses += 1
                self.layer_misses[key[0]] += 1
                return None
            size = _nbytes(value)
            self.stats.hits += 1
            self.stats.hit_bytes += size
            self.layer_hits[key[0]] += 1
            self.layer_hit_bytes[key[0]] += size
            self.frequency[key] = self.frequency.get(key, 0) + 1
            self.last_access[key] = self.access_index
            self.future_score[key] = self.future_score.get(key, 0.0) * 0.80
            if key in self.pinned:
                self.stats.pinned_hits += 1
            if key in self.prefetched:
                self.prefetched.discard(key)
                self.stats.prefetch_used += 1
            return value

    def put(self, key: Key, value: torch.Tensor, pin: bool = False, prefetched: bool = False) -> None:
        size = _nbytes(value)
        if self.max_bytes <= 0:
            return
        with self.lock:
            if key in self.items:
                old = self.item_bytes.get(key, _nbytes(self.items[key]))
                self.current_bytes -= old
                self.layer_bytes[key[0]] -= old
            else:
                self.birth_access[key] = self.access_index
            self.items[key] = value
            self.item_bytes[key] = size
            self.access_index += 1
            self.frequency[key] = self.frequency.get(key, 0) + 1
            self.last_access[key] = self.access_index
            if prefetched:
                self.prefetched.add(key)
            if pin:
                self.pinned.add(key)
            self.current_bytes += size
            self.layer_bytes[key[0]] += size
            self.stats.dequantized_bytes += size
            self._evict_to_budget()

    def pin(self, key: Key) -> None:
        with self.lock:
            if key in self.items:
                self.pinned.add(key)

    def contains(self, key: Key) -> bool:
        with self.lock:
            return key in self.items

    def resident_experts(self, layer_idx: int) -> set[int]:
        with self.lock:
            return {expert for layer, expert, _ in self.items if layer == layer_idx}

    def set_future_scores(self, keys: list[Key], scores: dict[Key, float] | None = None,
                          protect_window: int = 64) -> None:
        with self.lock:
            for key in list(self.future_score):
                decayed = self.future_score[key] * 0.85
                if decayed < 1e-4:
                    del self.future_score[key]
                else:
                    self.future_score[key] = decayed
            horizon = self.access_index + max(int(protect_window), 1)
            for key in keys:
                score = float(scores.get(key, 1.0)) if scores else 1.0
                self.future_score[key] = max(self.future_score.get(key, 0.0), score)
                self.protected_until[key] = max(self.protected_until.get(key, 0), horizon)

    def _evict_to_budget(self) -> None:
        while self.current_bytes > self.max_bytes and self.items:
            candidates, reason = self._eviction_candidates()
            if not candidates:
                break
            free = [k for k in candidates if self.protected_until.get(k, 0) <= self.access_index]
            if free:
                candidates = free
            else:
                self.stats.protected_eviction_skips += 1
            victim = min(candidates, key=lambda k: (self.future_score.get(k, 0.0), self.frequency.get(k, 0),
                                                     self.last_access.get(k, 0)))
            old = self.items.pop(victim)
            size = self.item_bytes.pop(victim, _nbytes(old))
            born = self.birth_access.pop(victim, self.access_index)
            self.evicted_lifetimes.append(max(self.access_index - born, 0))
            for table in (self.frequency, self.last_access, self.future_score, self.protected_until):
                table.pop(victim, None)
            self.prefetched.discard(victim)
            self.current_bytes -= size
            self.layer_bytes[victim[0]] -= size
            if self.layer_bytes[victim[0]] <= 0:
                self.layer_bytes.pop(victim[0], None)
            self.eviction_reasons[reason] += 1
            self.layer_evictions[victim[0]] += 1
            self.stats.evictions += 1

    def _eviction_candidates(self) -> tuple[list[Key], str]:
        candidates = [k for k in self.items if k not in self.pinned]
        if not candidates or not self.layer_aware or self.layer_count <= 0:
            return candidates, "global_pressure"
        base = self.max_bytes / max(self.layer_count, 1)
        over = [layer for layer, size in self.layer_bytes.items()
                if size > self._layer_quota(layer, base)
                and any(k[0] == layer and k not in self.pinned for k in self.items)]
        if not over:
            return candidates, "global_pressure"
        worst = max(over, key=lambda layer: self.layer_bytes[layer] / max(self._layer_quota(layer, base), 1.0))
        in_layer = [k for k in candidates if k[0] == worst]
        reason = "adaptive_layer_quota_pressure" if self.adaptive_layer_quota else "layer_quota_pressure"
        return in_layer or candidates, reason

    def _layer_quota(self, layer: int, base_quota: float) -> float:
        if not self.adaptive_layer_quota:
            return base_quota
        hits = self.layer_hits.get(layer, 0)
        total = hits + self.layer_misses.get(layer, 0)
        if total < 32:
            return base_quota
        weight = 0.5 + self.adaptive_layer_quota_strength * (hits / max(total, 1))
        return base_quota * max(weight, 0.25)

    def to_json(self) -> dict:
        """Telemetry with the keys of mxfp4_expert.py:310-354."""
        with self.lock:
            st = self.stats
            hot = sorted(
                ({"layer": k[0], "expert": k[1], "proj": k[2], "frequency": self.frequency.get(k, 0),
                  "future_score": round(self.future_score.get(k, 0.0), 6),
                  "age_accesses": self.access_index - self.birth_access.get(k, self.access_index),
                  "pinned": k in self.pinned, "prefetched": k in self.prefetched} for k in self.items),
                key=lambda row: (row["future_score"], row["frequency"], row["pinned"]), reverse=True)
            life = sorted(self.evicted_lifetimes)

            def pct(q):
                return life[int(q * (len(life) - 1))] if life else None

            mats = max(st.materializations, 1)
            finished = st.prefetch_completed + st.prefetch_failed
            residency = [{"layer": int(layer), "resident_mb": round(size / 2**20, 6),
                          "resident_items": sum(1 for k in self.items if k[0] == layer),
                          "resident_experts": len({k[1] for k in self.items if k[0] == layer})}
                         for layer, size in sorted(self.layer_bytes.items())]
            layers = sorted(set(self.layer_hits) | set(self.layer_misses) | set(self.layer_evictions)
                            | set(self.layer_loaded_bytes) | set(self.layer_hit_bytes))
            activity = []
            for layer in layers:
                h, m = int(self.layer_hits.get(layer, 0)), int(self.layer_misses.get(layer, 0))
                activity.append({"layer": int(layer), "hits": h, "misses": m, "hit_rate": h / max(h + m, 1),
                                 "evictions": int(self.layer_evictions.get(layer, 0)),
                                 "loaded_mb": round(int(self.layer_loaded_bytes.get(layer, 0)) / 2**20, 6),
                                 "hit_mb": round(int(self.layer_hit_bytes.get(layer, 0)) / 2**20, 6)})
            return {
                "hits": st.hits, "misses": st.misses, "hit_rate": st.hit_rate, "pinned_hits": st.pinned_hits,
                "evictions": st.evictions, "resident_bytes": self.current_bytes,
                "resident_mb": round(self.current_bytes / 2**20, 6), "resident_items": len(self.items),
                "pinned_items": len(self.pinned), "loaded_bytes": st.loaded_bytes,
                "loaded_mb": round(st.loaded_bytes / 2**20, 6), "dequantized_bytes": st.dequantized_bytes,
                "dequantized_mb": round(st.dequantized_bytes / 2**20, 6), "hit_bytes": st.hit_bytes,
                "hit_mb": round(st.hit_bytes / 2**20, 6), "miss_loaded_bytes": st.miss_loaded_bytes,
                "miss_loaded_mb": round(st.miss_loaded_bytes / 2**20, 6),
                "effective_useful_bandwidth": st.hit_bytes / max(st.loaded_bytes, 1),
                "materializations": st.materializations,
                "materialization_time_s": round(st.materialization_time_s, 6),
                "avg_materialization_time_ms": round(1000.0 * st.materialization_time_s / mats, 6),
                "transfer_time_s": round(st.transfer_time_s, 6), "dequant_time_s": round(st.dequant_time_s, 6),
                "avg_dequant_time_ms": round(1000.0 * st.dequant_time_s / mats, 6),
                "blocked_on_prefetch_s": round(st.blocked_on_prefetch_s, 6), "futures_waited": st.futures_waited,
                "prefetch_submitted": st.prefetch_submitted, "prefetch_completed": st.prefetch_completed,
                "prefetch_failed": st.prefetch_failed, "prefetch_used": st.prefetch_used,
                "prefetch_use_rate": st.prefetch_used / max(finished, 1),
                "prefetch_skipped_resident": st.prefetch_skipped_resident,
                "prefetch_skipped_pending": st.prefetch_skipped_pending,
                "protected_eviction_skips": st.protected_eviction_skips,
                "evicted_lifetime": {"count": len(life), "mean_accesses": sum(life) / len(life) if life else None,
                                     "p50_accesses": pct(0.50), "p90_accesses": pct(0.90)},
                "layer_aware": self.layer_aware, "adaptive_layer_quota": self.adaptive_layer_quota,
                "layer_count": self.layer_count,
                "layer_quota_mb": round((self.max_bytes / max(self.layer_count, 1)) / 2**20, 6)
                if self.layer_count else None,
                "layer_residency": residency, "layer_activity": activity,
                "eviction_reasons": dict(self.eviction_reasons), "hot_items": hot[:50],
            }


def dequantize_mxfp4_matrix(blocks: torch.Tensor, scales: torch.Tensor,
                            dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """Dequantize one MXFP4 expert matrix on the GPU.

    ``blocks [out, G, 16]`` (two E2M1 codes per byte, low nibble first) and
    ``scales [out, G]`` (E8M0) -> ``[in = 32 G, out]`` in ``dtype``
    (bfloat16, float16 or float32), bit-exact with mxfp4_expert.py:357-379.
    Leading batch dimensions are allowed.  Raises ValueError on a block/scale
    shape mismatch and on tensors that are not on a GPU.
    """
    return ops.mxfp4_dequant(blocks, scales, dtype)


class SafetensorIndex:
    """The ``model.safetensors.index.json`` weight map (streamed_loader.py:43-50)."""

    def __init__(self, model_dir: str | Path, support_dir: str | Path) -> None:
        self.model_dir = Path(model_dir)
        self.support_dir = Path(support_dir)
        self.index_path = self.support_dir / "model.safetensors.index.json"
        with self.index_path.open("r", encoding="utf-8") as f:
            self.index = json.load(f)
        self.weight_map: dict[str, str] = self.index["weight_map"]
        self._shards: dict[str, SafetensorShard] = {}
        self._shards_lock = RLock()

    def shard(self, name: str) -> SafetensorShard:
        """The open shard holding tensor ``name`` (opened once, then shared)."""
        file = self.weight_map[name]
        with self._shards_lock:
            shard = self._shards.get(file)
            if shard is None:
                shard = SafetensorShard(self.model_dir / file)
                self._shards[file] = shard
            return shard


class Mxfp4ExpertStore:
    """Expert store with the constructor and methods of mxfp4_expert.py:382-531.

    Cached values are packed matrices (uint8, row-tile layout).  Misses are
    read from the checkpoint (``model.layers.{L}.mlp.experts.{proj}_{blocks,scales}``
    sliced at the expert), copied to the device on a side stream and packed
    there; the compute stream waits on an event, never on the device.
    """

    def __init__(self, model_dir: str | Path, support_dir: str | Path, device: torch.device,
                 dtype: torch.dtype = torch.float16, cache_bytes: int = 0, quant_loader=None,
                 async_prefetch: bool = False, max_prefetch_workers: int = 1, layer_count: int = 0,
                 layer_aware_cache: bool = False, adaptive_layer_quota: bool = False,
                 adaptive_layer_quota_strength: float = 1.5, default_protect_window: int = 64) -> None:
        self.index = SafetensorIndex(model_dir, support_dir)
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError(f"Mxfp4ExpertStore keeps experts in GPU memory; got device {self.device}")
        self.dtype = dtype
        self.cache = ExpertWeightCache(cache_bytes, layer_count=layer_count, layer_aware=layer_aware_cache,
                                       adaptive_layer_quota=adaptive_layer_quota,
                                       adaptive_layer_quota_strength=adaptive_layer_quota_strength)
        self.quant_loader = quant_loader
        self.async_prefetch = async_prefetch
        self.default_protect_window = max(int(default_protect_window), 1)
        self.executor = (ThreadPoolExecutor(max_workers=max_prefetch_workers)
                         if async_prefetch and max_prefetch_workers > 0 else None)
        self.pending: dict[Key, Future] = {}
        self.pending_lock = RLock()
        self._shapes: dict[Key, tuple[int, int]] = {}
        self._side = torch.cuda.Stream(self.device)
        # side-stream events of packs enqueued without a host wait, per key,
        # until one is seen complete
        self._ready: dict[Key, torch.cuda.Event] = {}
        self._ready_lock = RLock()

    # ---- reference API ---------------------------------------------------------

    def load_expert_matrix(self, layer_idx: int, expert_idx: int, proj: str) -> torch.Tensor:
        """Dequantized ``[in, out]`` matrix in the store's dtype (mxfp4_expert.py:416-422)."""
        key = (layer_idx, expert_idx, proj)
        packed = self.packed_expert(layer_idx, expert_idx, proj)
        rows, groups = self._shapes[key]
        return ops.mxfp4_dequant_packed(packed, rows, groups, self.dtype)

    def protect_experts(self, layer_idx: int, expert_ids: list[int], protect_window: int | None = None) -> None:
        self.cache.set_future_scores(self._matrix_keys(layer_idx, expert_ids),
                                     protect_window=protect_window or self.default_protect_window)

    def prefetch_experts(self, layer_idx: int, expert_ids: list[int], protect_window: int | None = None) -> None:
        if not expert_ids:
            return
        keys = self._matrix_keys(layer_idx, expert_ids)
        self.cache.set_future_scores(keys, protect_window=protect_window or self.default_protect_window)
        if self.executor is None:
            return
        with self.pending_lock:
            for key in keys:
                if self.cache.contains(key):
                    self.cache.stats.prefetch_skipped_resident += 1
                elif key in self.pending:
                    self.cache.stats.prefetch_skipped_pending += 1
                else:
                    self.pending[key] = self.executor.submit(self._prefetch_worker, key)
                    self.cache.stats.prefetch_submitted += 1

    def resident_experts(self, layer_idx: int) -> set[int]:
        return self.cache.resident_experts(layer_idx)

    def pin_experts(self, keys: list[Key]) -> None:
        for layer_idx, expert_idx, proj in keys:
            self.packed_expert(layer_idx, expert_idx, proj)
            self.cache.pin((layer_idx, expert_idx, proj))

    def to_json(self) -> dict:
        payload = self.cache.to_json()
        with self.pending_lock:
            payload["pending_prefetches"] = len(self.pending)
        return payload

    # ---- packed access (the fused router path) ---------------------------------

    def packed_expert(self, layer_idx: int, expert_idx: int, proj: str) -> torch.Tensor:
        """Packed matrix of one expert projection, usable on the current stream.

        Counts one cache access, like ``load_expert_matrix`` in the reference.
        """
        key = (int(layer_idx), int(expert_idx), proj)
        self._consume_pending_if_needed(key)
        cached = self.cache.get(key)
        if cached is None:
            cached = self._materialize_expert_matrix(key, prefetched=False)
        if self._ready:
            self._order_after_load(key)
        return cached

    def _order_after_load(self, key: Key) -> None:
        """Makes the current stream wait (on the device) for the pack of
        ``key`` if it may still be running on the side stream."""
        with self._ready_lock:
            ev = self._ready.get(key)
            if ev is None:
                return
            if ev.query():
                del self._ready[key]
                return
        torch.cuda.current_stream(self.device).wait_event(ev)

    def matrix_shape(self, layer_idx: int, expert_idx: int, proj: str) -> tuple[int, int]:
        """``(rows, groups)`` of a materialized projection."""
        return self._shapes[(int(layer_idx), int(expert_idx), proj)]

    # ---- internals ----------------------------------------------------------------

    @staticmethod
    def _matrix_keys(layer_idx: int, expert_ids: list[int]) -> list[Key]:
        return [(int(layer_idx), int(e), "gate_up_proj") for e in expert_ids] + \
               [(int(layer_idx), int(e), "down_proj") for e in expert_ids]

    def _consume_pending_if_needed(self, key: Key) -> None:
        with self.pending_lock:
            future = self.pending.pop(key, None)
        if future is None:
            return
        start = time.perf_counter()
        self.cache.stats.futures_waited += 1
        try:
            future.result()
        finally:
            self.cache.stats.blocked_on_prefetch_s += time.perf_counter() - start

    def _prefetch_worker(self, key: Key) -> None:
        try:
            if not self.cache.contains(key):
                self._materialize_expert_matrix(key, prefetched=True)
            self.cache.stats.prefetch_completed += 1
        except Exception:
            self.cache.stats.prefetch_failed += 1
            raise
        finally:
            with self.pending_lock:
                self.pending.pop(key, None)

    def _materialize_expert_matrix(self, key: Key, prefetched: bool) -> torch.Tensor:
        """Checkpoint shard -> pinned staging -> device (side stream) -> packed layout.

        Blocks and scales in one shard (the checkpoint's layout) take the fused
        path: klc_st_load_mxfp4_packed reads and packs chunk by chunk on the
        side stream without waiting for the compute stream, and returns once
        the last pack is enqueued; ``packed_expert`` then makes the caller's
        stream wait for an event after that pack, so no host wait is needed
        and the next miss's reads overlap these packs.  Otherwise
        (a quantized loader, or the two tensors in different shards) the slices
        are copied first and packed after the side stream has waited for the
        compute stream, into a tensor allocated on the compute stream.  Only
        the side stream is synchronised.
        """
        layer_idx, expert_idx, proj = key
        start = time.perf_counter()
        base = f"model.layers.{layer_idx}.mlp.experts.{proj}"
        names = (f"{base}_blocks", f"{base}_scales")
        compute = torch.cuda.current_stream(self.device)
        if not self._from_quant_loader(names[0]) and self.index.shard(names[0]) is self.index.shard(names[1]):
            # shard -> pinned staging -> packed, chunk by chunk on the side
            # stream; the packed tensor is allocated on the compute stream
            # and marked as used by the side stream, so its memory is reused
            # only after both the packs and the compute work that reads it
            packed, rows, groups = self.index.shard(names[0]).load_mxfp4_packed(
                names[0], names[1], expert_idx, self.device, self._side, wait=False)
            ready = torch.cuda.Event()
            ready.record(self._side)
            with self._ready_lock:
                self._ready[key] = ready
            loaded = rows * groups * 17
            self.cache.stats.transfer_time_s += time.perf_counter() - start
        else:
            if self._from_quant_loader(names[0]):
                blocks, scales = (self._load_expert_tensor(n, expert_idx) for n in names)
                self._check_pair(blocks.shape, scales.shape)
                with torch.cuda.stream(self._side):
                    b_dev = blocks.to(torch.uint8).contiguous().pin_memory().to(self.device, non_blocking=True)
                    s_dev = scales.to(torch.uint8).contiguous().pin_memory().to(self.device, non_blocking=True)
            else:
                # blocks and scales in different shards: staged copies, then the pack
                b_dev, s_dev = self._copy_expert_tensors(names, expert_idx)
                self._check_pair(b_dev.shape, s_dev.shape)
            copied = torch.cuda.Event()
            copied.record(self._side)
            loaded = _nbytes(b_dev) + _nbytes(s_dev)
            rows, groups = int(b_dev.shape[0]), int(b_dev.shape[1])
            packed = torch.empty(ops.packed_bytes(rows, groups), dtype=torch.uint8, device=self.device)
            self._side.wait_stream(compute)
            with torch.cuda.stream(self._side):
                ops.mxfp4_pack(b_dev, s_dev, out=packed)
                done = torch.cuda.Event()
                done.record(self._side)
            copied.synchronize()
            self.cache.stats.transfer_time_s += time.perf_counter() - start
            pack_start = time.perf_counter()
            done.synchronize()
            self.cache.stats.dequant_time_s += time.perf_counter() - pack_start
        self.cache.stats.loaded_bytes += loaded
        self.cache.stats.miss_loaded_bytes += loaded
        self.cache.layer_loaded_bytes[layer_idx] += loaded
        self.cache.stats.materialization_time_s += time.perf_counter() - start
        self.cache.stats.materializations += 1
        self._shapes[key] = (rows, groups)
        self.cache.put(key, packed, prefetched=prefetched)
        return packed

    @staticmethod
    def _check_pair(bshape, sshape) -> None:
        if len(bshape) != 3 or tuple(bshape[:-1]) != tuple(sshape):
            raise ValueError(f"MXFP4 block/scale shape mismatch: blocks.shape={tuple(bshape)} "
                             f"scales.shape={tuple(sshape)}")

    def _from_quant_loader(self, name: str) -> bool:
        loader = self.quant_loader
        return loader is not None and name in getattr(loader, "tensor_index", {})

    def _copy_expert_tensors(self, names: tuple[str, ...], expert_idx: int) -> list[torch.Tensor]:
        """The expert's slices of ``names`` (U8), from their shards to the
        device, one staged copy per shard."""
        by_shard: dict[int, tuple[SafetensorShard, list[int]]] = {}
        for i, name in enumerate(names):
            shard = self.index.shard(name)
            dtype = shard.info(name)[0]
            if dtype != "U8":
                raise ValueError(f"{name}: MXFP4 blocks and scales are U8 in the checkpoint, found {dtype}")
            by_shard.setdefault(id(shard), (shard, []))[1].append(i)
        out: list[torch.Tensor | None] = [None] * len(names)
        for shard, idx in by_shard.values():
            got = shard.copy_rows_batch([(names[i], expert_idx, 1) for i in idx], self.device, self._side)
            for i, t in zip(idx, got):
                out[i] = t[0]
        return out

    def _load_expert_tensor(self, name: str, expert_idx: int) -> torch.Tensor:
        """The expert's slice as a host tensor (the quantized-loader path, or the shard reader)."""
        if self._from_quant_loader(name):
            full, meta = self.quant_loader.load_tensor(name, dtype=self.dtype)
            selected = full[expert_idx].detach().cpu()
            if getattr(meta, "dtype", None) == "torch.uint8":
                return torch.clamp(torch.round(selected.float()), 0, 255).to(torch.uint8)
            return selected
        return self.index.shard(name).read_rows(name, expert_idx, 1)[0]


class ResidentExpertStore:
    """Every expert of the given layers packed in HBM: no streaming, no eviction.

    The MI355X deployment form of the expert store: 128 gpt-oss-120b experts
    of one layer take 1.69 GB packed, all 36 layers 60.9 GB of the 288 GB.
    It offers the store methods the router and the executor call
    (mxfp4_expert.py:416-452,509-531); protection and prefetch are no-ops, and
    ``cache`` only counts accesses so the router's cache telemetry stays
    meaningful.  The router runs a layer held here with no host
    synchronisation before its last kernel.
    """

    def __init__(self, layers: dict, dtype: torch.dtype = torch.bfloat16) -> None:
        self.layers = dict(layers)
        self.dtype = dtype
        self.cache = ExpertWeightCache(0)

    def layer(self, layer_idx: int):
        try:
            return self.layers[int(layer_idx)]
        except KeyError:
            raise KeyError(f"layer {layer_idx} is not resident") from None

    def record_access(self, layer_idx: int, n_matrices: int) -> None:
        """Counts ``n_matrices`` expert-matrix reads of a resident layer as hits."""
        with self.cache.lock:
            self.cache.stats.hits += n_matrices
            self.cache.stats.lifetime_accesses += n_matrices
            self.cache.layer_hits[int(layer_idx)] += n_matrices

    def load_expert_matrix(self, layer_idx: int, expert_idx: int, proj: str) -> torch.Tensor:
        w = self.layer(layer_idx)
        if proj == "gate_up_proj":
            packed, rows, groups = w.gate_up[expert_idx], 2 * w.inter, w.hidden // 32
        elif proj == "down_proj":
            packed, rows, groups = w.down[expert_idx], w.hidden, w.inter // 32
        else:
            raise KeyError(f"unknown projection {proj!r}")
        self.record_access(layer_idx, 1)
        return ops.mxfp4_dequant_packed(packed, rows, groups, self.dtype)

    def protect_experts(self, layer_idx: int, expert_ids: list[int], protect_window: int | None = None) -> None:
        return None

    def prefetch_experts(self, layer_idx: int, expert_ids: list[int], protect_window: int | None = None) -> None:
        return None

    def resident_experts(self, layer_idx: int) -> set[int]:
        w = self.layers.get(int(layer_idx))
        return set(range(w.n_experts)) if w is not None else set()

    def pin_experts(self, keys: list[Key]) -> None:
        for layer_idx, _, _ in keys:
            self.layer(layer_idx)

    def resident_bytes(self) -> int:
        return sum(int(w.gate_up.numel() + w.down.numel()) for w in self.layers.values())

    def to_json(self) -> dict:
        payload = self.cache.to_json()
        nbytes = self.resident_bytes()
        payload.update({"resident_bytes": nbytes, "resident_mb": round(nbytes / 2**20, 6),
                        "resident_items": 2 * sum(w.n_experts for w in self.layers.values()),
                        "resident_layers": sorted(self.layers), "pending_prefetches": 0})
        return payload
