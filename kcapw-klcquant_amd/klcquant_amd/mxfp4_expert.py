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
import queue
import threading
import time
from collections import Counter, OrderedDict, deque
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


@dataclass
class _Entry:
    """One cached packed matrix and what the eviction policy knows about it."""

    value: torch.Tensor
    nbytes: int
    born: int  # clock value at insertion
    uses: int = 0  # lookups that found it
    hold_until: int = 0  # clock value up to which a protect/prefetch hint holds it
    pinned: bool = False
    prefetched: bool = False  # brought in by a prefetch and not looked up since


class ExpertWeightCache:
    """Byte-budgeted cache of packed expert matrices, keyed ``(layer, expert, proj)``.

    The reference's cache holds dequantized matrices (mxfp4_expert.py:68-354);
    this one holds the packed MXFP4 form the expert kernels stream, 3.76x
    smaller, with its own policy:

    * **Recency order.**  Entries sit in least-recently-used order; a lookup
      that finds an entry moves it to the back.  The clock advances by one per
      lookup and per insertion.
    * **Holds.**  ``hold(keys, window)`` (the store's protect / prefetch hints,
      also reachable as ``set_future_scores``) protects those matrices for the
      next ``window`` clock ticks, whether or not they are resident yet.
    * **Eviction.**  While the resident bytes exceed ``max_bytes``, the victim
      is the least recently used entry that is neither pinned nor held; if
      every unpinned candidate is held, the least recently used held one goes
      (counted in ``protected_eviction_skips``).  Pinned entries never go.
    * **Layer quotas** (``layer_aware`` with ``layer_count > 0``): each layer's
      quota is ``max_bytes / layer_count``; while some layer is over its quota,
      victims come from the layer with the largest bytes-to-quota ratio first.
      With ``adaptive_layer_quota``, a layer with at least 32 lookups gets the
      quota scaled by ``max(0.25, 1 + strength * (its hit rate - the mean hit
      rate of such layers))``: layers that reuse their experts keep more.
    * ``max_bytes <= 0`` stores nothing.

    Counters and telemetry keep the reference's names (``ExpertCacheStats``,
    ``to_json`` keys), since the router and the executor's runtime stats read
    them.  Thread safe (one re-entrant lock).
    """

    HOLD_ADAPT_MIN_LOOKUPS = 32

    def __init__(self, max_bytes: int, layer_count: int = 0, layer_aware: bool = False,
                 adaptive_layer_quota: bool = False, adaptive_layer_quota_strength: float = 1.5) -> None:
        self.max_bytes = int(max_bytes)
        self.layer_count = max(int(layer_count), 0)
        self.layer_aware = bool(layer_aware)
        self.adaptive_layer_quota = bool(adaptive_layer_quota)
        self.adaptive_layer_quota_strength = max(float(adaptive_layer_quota_strength), 0.0)
        self.stats = ExpertCacheStats()
        self.lock = RLock()
        self.clock = 0
        self.current_bytes = 0
        self._entries: OrderedDict[Key, _Entry] = OrderedDict()
        self._held: dict[Key, int] = {}  # holds of keys that are not resident (yet)
        self._layer_bytes: Counter[int] = Counter()
        self._lookups: Counter[int] = Counter()  # per layer
        self._found: Counter[int] = Counter()  # per layer
        self._layer_found_bytes: Counter[int] = Counter()
        self._layer_evicted: Counter[int] = Counter()
        self.layer_loaded_bytes: Counter[int] = Counter()  # the store books miss traffic here
        self._lifetimes: list[int] = []
        self._reasons: Counter[str] = Counter()
        self.eviction_log: deque[Key] = deque(maxlen=4096)  # the most recent victims, oldest first

    # ---- lookups and insertions -------------------------------------------------------

    def get(self, key: Key) -> torch.Tensor | None:
        with self.lock:
            self.clock += 1
            self.stats.lifetime_accesses += 1
            layer = key[0]
            self._lookups[layer] += 1
            entry = self._entries.get(key)
            if entry is None:
                self.stats.misses += 1
                return None
            self._entries.move_to_end(key)
            entry.uses += 1
            self._found[layer] += 1
            self._layer_found_bytes[layer] += entry.nbytes
            self.stats.hits += 1
            self.stats.hit_bytes += entry.nbytes
            self.stats.pinned_hits += entry.pinned
            if entry.prefetched:
                entry.prefetched = False
                self.stats.prefetch_used += 1
            return entry.value

    def put(self, key: Key, value: torch.Tensor, pin: bool = False, prefetched: bool = False) -> None:
        if self.max_bytes <= 0:
            return
        nbytes = _nbytes(value)
        with self.lock:
            self.clock += 1
            old = self._entries.pop(key, None)
            if old is not None:
                self._account(key, -old.nbytes)
            entry = _Entry(value, nbytes, born=self.clock, pinned=pin or (old is not None and old.pinned),
                           prefetched=prefetched, hold_until=self._held.pop(key, 0))
            if old is not None:
                entry.hold_until = max(entry.hold_until, old.hold_until)
            self._entries[key] = entry
            self._account(key, nbytes)
            self.stats.dequantized_bytes += nbytes
            self._shrink_to_budget()

    def count_hits(self, layer: int, n: int) -> None:
        """Books ``n`` lookups served outside the cache (always-resident matrices) as hits."""
        with self.lock:
            self.clock += n
            self.stats.lifetime_accesses += n
            self.stats.hits += n
            self._lookups[layer] += n
            self._found[layer] += n

    def pin(self, key: Key) -> None:
        with self.lock:
            entry = self._entries.get(key)
            if entry is not None:
                entry.pinned = True

    @property
    def pinned(self) -> set[Key]:
        with self.lock:
            return {k for k, e in self._entries.items() if e.pinned}

    def contains(self, key: Key) -> bool:
        with self.lock:
            return key in self._entries

    def resident_experts(self, layer_idx: int) -> set[int]:
        with self.lock:
            return {expert for layer, expert, _ in self._entries if layer == layer_idx}

    def hold(self, keys, window: int = 64) -> None:
        """Protects ``keys`` from eviction for the next ``window`` clock ticks."""
        with self.lock:
            until = self.clock + max(int(window), 1)
            for key in keys:
                entry = self._entries.get(key)
                if entry is not None:
                    entry.hold_until = max(entry.hold_until, until)
                else:
                    self._held[key] = max(self._held.get(key, 0), until)
            # forget holds of keys that never arrived once they have run out
            if len(self._held) > 4096:
                self._held = {k: t for k, t in self._held.items() if t > self.clock}

    def set_future_scores(self, keys, scores=None, protect_window: int = 64) -> None:
        """The reference's name for a hint (mxfp4_expert.py:166-181): a hold of ``protect_window``."""
        self.hold(keys, protect_window)

    # ---- eviction -----------------------------------------------------------------------

    def _account(self, key: Key, delta: int) -> None:
        self.current_bytes += delta
        self._layer_bytes[key[0]] += delta
        if self._layer_bytes[key[0]] <= 0:
            del self._layer_bytes[key[0]]

    def layer_quota(self, layer: int) -> float:
        """Bytes layer ``layer`` may hold before its entries are evicted first."""
        base = self.max_bytes / max(self.layer_count, 1)
        if not self.adaptive_layer_quota:
            return base
        rates = {l: self._found[l] / n for l, n in self._lookups.items() if n >= self.HOLD_ADAPT_MIN_LOOKUPS}
        if layer not in rates:
            return base
        mean = sum(rates.values()) / len(rates)
        return base * max(0.25, 1.0 + self.adaptive_layer_quota_strength * (rates[layer] - mean))

    def _pressured_layer(self) -> int | None:
        if not (self.layer_aware and self.layer_count > 0):
            return None
        worst, worst_ratio = None, 1.0
        for layer, nbytes in self._layer_bytes.items():
            ratio = nbytes / max(self.layer_quota(layer), 1.0)
            if ratio > worst_ratio and any(k[0] == layer and not e.pinned for k, e in self._entries.items()):
                worst, worst_ratio = layer, ratio
        return worst

    def _oldest_evictable(self, layer: int | None) -> Key | None:
        """Least recently used unpinned entry (of ``layer``, if given), preferring unheld ones."""
        first_held = None
        for key, entry in self._entries.items():  # least recently used first
            if entry.pinned or (layer is not None and key[0] != layer):
                continue
            if entry.hold_until <= self.clock:
                return key
            if first_held is None:
                first_held = key
        if first_held is not None:
            self.stats.protected_eviction_skips += 1
        return first_held

    def _pick_victim(self) -> tuple[Key | None, str]:
        layer = self._pressured_layer()
        if layer is not None:
            victim = self._oldest_evictable(layer)
            if victim is not None:
                return victim, ("adaptive_layer_quota_pressure" if self.adaptive_layer_quota
                                else "layer_quota_pressure")
        return self._oldest_evictable(None), "global_pressure"

    def _shrink_to_budget(self) -> None:
        while self.current_bytes > self.max_bytes:
            victim, reason = self._pick_victim()
            if victim is None:
                return  # everything left is pinned
            entry = self._entries.pop(victim)
            self._account(victim, -entry.nbytes)
            self._lifetimes.append(self.clock - entry.born)
            self._reasons[reason] += 1
            self._layer_evicted[victim[0]] += 1
            self.stats.evictions += 1
            self.eviction_log.append(victim)

    @property
    def eviction_reasons(self) -> Counter[str]:
        return self._reasons

    # ---- telemetry (keys of mxfp4_expert.py:310-354) --------------------------------------

    def to_json(self) -> dict:
        with self.lock:
            st = self.stats
            mib = 2 ** 20
            per_item = [{"layer": k[0], "expert": k[1], "proj": k[2], "frequency": e.uses,
                         "future_score": float(max(e.hold_until - self.clock, 0)),
                         "age_accesses": self.clock - e.born, "pinned": e.pinned, "prefetched": e.prefetched}
                        for k, e in self._entries.items()]
            per_item.sort(key=lambda r: (r["future_score"], r["frequency"], r["pinned"]), reverse=True)
            life = sorted(self._lifetimes)
            n_mat = max(st.materializations, 1)
            finished = st.prefetch_completed + st.prefetch_failed
            by_layer: dict[int, list[Key]] = {}
            for k in self._entries:
                by_layer.setdefault(k[0], []).append(k)
            residency = [{"layer": int(l), "resident_mb": round(self._layer_bytes[l] / mib, 6),
                          "resident_items": len(keys), "resident_experts": len({k[1] for k in keys})}
                         for l, keys in sorted(by_layer.items())]
            activity = [{"layer": int(l), "hits": int(self._found[l]), "misses": int(self._lookups[l] - self._found[l]),
                         "hit_rate": self._found[l] / max(self._lookups[l], 1),
                         "evictions": int(self._layer_evicted[l]),
                         "loaded_mb": round(self.layer_loaded_bytes[l] / mib, 6),
                         "hit_mb": round(self._layer_found_bytes[l] / mib, 6)}
                        for l in sorted(set(self._lookups) | set(self._layer_evicted) | set(self.layer_loaded_bytes))]
            return {
                "hits": st.hits, "misses": st.misses, "hit_rate": st.hit_rate, "pinned_hits": st.pinned_hits,
                "evictions": st.evictions, "resident_bytes": self.current_bytes,
                "resident_mb": round(self.current_bytes / mib, 6), "resident_items": len(self._entries),
                "pinned_items": sum(e.pinned for e in self._entries.values()), "loaded_bytes": st.loaded_bytes,
                "loaded_mb": round(st.loaded_bytes / mib, 6), "dequantized_bytes": st.dequantized_bytes,
                "dequantized_mb": round(st.dequantized_bytes / mib, 6), "hit_bytes": st.hit_bytes,
                "hit_mb": round(st.hit_bytes / mib, 6), "miss_loaded_bytes": st.miss_loaded_bytes,
                "miss_loaded_mb": round(st.miss_loaded_bytes / mib, 6),
                "effective_useful_bandwidth": st.hit_bytes / max(st.loaded_bytes, 1),
                "materializations": st.materializations,
                "materialization_time_s": round(st.materialization_time_s, 6),
                "avg_materialization_time_ms": round(1e3 * st.materialization_time_s / n_mat, 6),
                "transfer_time_s": round(st.transfer_time_s, 6), "dequant_time_s": round(st.dequant_time_s, 6),
                "avg_dequant_time_ms": round(1e3 * st.dequant_time_s / n_mat, 6),
                "blocked_on_prefetch_s": round(st.blocked_on_prefetch_s, 6), "futures_waited": st.futures_waited,
                "prefetch_submitted": st.prefetch_submitted, "prefetch_completed": st.prefetch_completed,
                "prefetch_failed": st.prefetch_failed, "prefetch_used": st.prefetch_used,
                "prefetch_use_rate": st.prefetch_used / max(finished, 1),
                "prefetch_skipped_resident": st.prefetch_skipped_resident,
                "prefetch_skipped_pending": st.prefetch_skipped_pending,
                "protected_eviction_skips": st.protected_eviction_skips,
                "evicted_lifetime": {"count": len(life), "mean_accesses": sum(life) / len(life) if life else None,
                                     "p50_accesses": life[(len(life) - 1) // 2] if life else None,
                                     "p90_accesses": life[int(0.9 * (len(life) - 1))] if life else None},
                "layer_aware": self.layer_aware, "adaptive_layer_quota": self.adaptive_layer_quota,
                "layer_count": self.layer_count,
                "layer_quota_mb": round(self.max_bytes / max(self.layer_count, 1) / mib, 6) if self.layer_count else None,
                "layer_residency": residency, "layer_activity": activity,
                "eviction_reasons": dict(self._reasons), "hot_items": per_item[:50],
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


class _Inflight:
    """A miss being brought in by a background loader: done when ``event`` is set."""

    __slots__ = ("event", "error")

    def __init__(self) -> None:
        self.event = threading.Event()
        self.error: BaseException | None = None


class Mxfp4ExpertStore:
    """Expert store with the constructor and methods of mxfp4_expert.py:382-531.

    Cached values are packed matrices (uint8, row-tile layout).  A miss reads
    the expert's slice of ``model.layers.{L}.mlp.experts.{proj}_{blocks,scales}``
    from the checkpoint shard into pinned staging and packs it into HBM on a
    side stream; the stream that then uses the matrix waits on an event, never
    on the device.

    Prefetch (``async_prefetch=True``): ``max_prefetch_workers`` daemon loader
    threads take keys from one queue and bring them in; a key is "in flight"
    from its submission until its loader finishes.  A lookup of an in-flight
    key waits (host) for its loader and re-raises the loader's exception, as
    the reference does when it consumes a failed prefetch (mxfp4_expert.py:454-462).
    Packed tensors are allocated on the side stream and recorded on every
    stream they are handed to, so the caching allocator reuses their memory
    only after the work that reads them.
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
        self._side = torch.cuda.Stream(self.device)
        self._shapes: dict[Key, tuple[int, int]] = {}
        # side-stream events of packs not yet seen complete, per key
        self._ready: dict[Key, torch.cuda.Event] = {}
        self._ready_lock = RLock()
        self._inflight: dict[Key, _Inflight] = {}
        self._inflight_lock = RLock()
        self._queue: queue.SimpleQueue | None = None
        self._loaders: list[threading.Thread] = []
        if async_prefetch and max_prefetch_workers > 0:
            self._queue = queue.SimpleQueue()
            for i in range(int(max_prefetch_workers)):
                t = threading.Thread(target=self._loader_loop, name=f"expert-loader-{i}", daemon=True)
                t.start()
                self._loaders.append(t)

    # ---- reference API ---------------------------------------------------------

    def load_expert_matrix(self, layer_idx: int, expert_idx: int, proj: str) -> torch.Tensor:
        """Dequantized ``[in, out]`` matrix in the store's dtype (mxfp4_expert.py:416-422)."""
        key = (layer_idx, expert_idx, proj)
        packed = self.packed_expert(layer_idx, expert_idx, proj)
        rows, groups = self._shapes[key]
        return ops.mxfp4_dequant_packed(packed, rows, groups, self.dtype)

    def protect_experts(self, layer_idx: int, expert_ids: list[int], protect_window: int | None = None) -> None:
        self.cache.hold(self._matrix_keys(layer_idx, expert_ids), protect_window or self.default_protect_window)

    def prefetch_experts(self, layer_idx: int, expert_ids: list[int], protect_window: int | None = None) -> None:
        if not expert_ids:
            return
        keys = self._matrix_keys(layer_idx, expert_ids)
        self.cache.hold(keys, protect_window or self.default_protect_window)
        if self._queue is None:
            return
        st = self.cache.stats
        for key in keys:
            if self.cache.contains(key):
                st.prefetch_skipped_resident += 1
                continue
            with self._inflight_lock:
                if key in self._inflight:
                    st.prefetch_skipped_pending += 1
                    continue
                self._inflight[key] = _Inflight()
            st.prefetch_submitted += 1
            self._queue.put(key)

    def resident_experts(self, layer_idx: int) -> set[int]:
        return self.cache.resident_experts(layer_idx)

    def pin_experts(self, keys: list[Key]) -> None:
        for layer_idx, expert_idx, proj in keys:
            self.packed_expert(layer_idx, expert_idx, proj)
            self.cache.pin((layer_idx, expert_idx, proj))

    def to_json(self) -> dict:
        payload = self.cache.to_json()
        with self._inflight_lock:
            payload["pending_prefetches"] = len(self._inflight)
        return payload

    def close(self) -> None:
        """Stops the loader threads after the keys already queued (idempotent)."""
        if self._queue is None:
            return
        for _ in self._loaders:
            self._queue.put(None)
        for t in self._loaders:
            t.join()
        self._loaders, self._queue = [], None

    # ---- packed access (the fused router path) ---------------------------------

    def packed_expert(self, layer_idx: int, expert_idx: int, proj: str) -> torch.Tensor:
        """Packed matrix of one expert projection, usable on the current stream.

        Counts one cache lookup, like ``load_expert_matrix`` in the reference.
        """
        key = (int(layer_idx), int(expert_idx), proj)
        self._wait_inflight(key)
        packed = self.cache.get(key)
        if packed is None:
            packed = self._materialize_expert_matrix(key, prefetched=False)
        stream = torch.cuda.current_stream(self.device)
        self._order_after_load(key, stream)
        if stream != self._side:
            packed.record_stream(stream)
        return packed

    def matrix_shape(self, layer_idx: int, expert_idx: int, proj: str) -> tuple[int, int]:
        """``(rows, groups)`` of a materialized projection."""
        return self._shapes[(int(layer_idx), int(expert_idx), proj)]

    # ---- internals ----------------------------------------------------------------

    @staticmethod
    def _matrix_keys(layer_idx: int, expert_ids: list[int]) -> list[Key]:
        # the order the router uses them: every gate_up, then every down
        return [(int(layer_idx), int(e), proj) for proj in PROJECTIONS for e in expert_ids]

    def _order_after_load(self, key: Key, stream: torch.cuda.Stream) -> None:
        """``stream`` waits (on the device) for the pack of ``key`` if it may still run."""
        with self._ready_lock:
            ev = self._ready.get(key)
            if ev is None:
                return
            if ev.query():
                del self._ready[key]
                return
        stream.wait_event(ev)

    def _wait_inflight(self, key: Key) -> None:
        with self._inflight_lock:
            job = self._inflight.get(key)
        if job is None:
            return
        start = time.perf_counter()
        self.cache.stats.futures_waited += 1
        job.event.wait()
        self.cache.stats.blocked_on_prefetch_s += time.perf_counter() - start
        if job.error is not None:
            raise job.error

    def _loader_loop(self) -> None:
        while True:
            key = self._queue.get() if self._queue is not None else None
            if key is None:
                return
            with self._inflight_lock:
                job = self._inflight.get(key)
            try:
                if not self.cache.contains(key):
                    self._materialize_expert_matrix(key, prefetched=True)
                self.cache.stats.prefetch_completed += 1
            except BaseException as exc:  # handed to whoever looks the key up
                self.cache.stats.prefetch_failed += 1
                if job is not None:
                    job.error = exc
            finally:
                with self._inflight_lock:
                    self._inflight.pop(key, None)
                if job is not None:
                    job.event.set()

    def _materialize_expert_matrix(self, key: Key, prefetched: bool) -> torch.Tensor:
        """Checkpoint shard -> pinned staging -> packed layout in HBM, on the side stream.

        Blocks and scales in one shard (the checkpoint's layout) take the fused
        path: klc_st_load_mxfp4_packed reads and packs chunk by chunk and
        returns once the last pack is enqueued; an event after that pack is
        what a consuming stream waits on (``_order_after_load``), so the next
        miss's reads overlap these packs.  Otherwise (a quantized loader, or
        the two tensors in different shards) the slices are copied to the
        device and packed, and the side stream is synchronised.  The packed
        tensor is always allocated on the side stream.
        """
        layer_idx, expert_idx, proj = key
        start = time.perf_counter()
        base = f"model.layers.{layer_idx}.mlp.experts.{proj}"
        names = (f"{base}_blocks", f"{base}_scales")
        st = self.cache.stats
        if not self._from_quant_loader(names[0]) and self.index.shard(names[0]) is self.index.shard(names[1]):
            packed, rows, groups = self.index.shard(names[0]).load_mxfp4_packed(
                names[0], names[1], expert_idx, self.device, self._side, wait=False)
            ready = torch.cuda.Event()
            ready.record(self._side)
            with self._ready_lock:
                self._ready[key] = ready
            loaded = rows * groups * 17
            st.transfer_time_s += time.perf_counter() - start
        else:
            if self._from_quant_loader(names[0]):
                blocks, scales = (self._load_expert_tensor(n, expert_idx) for n in names)
                self._check_pair(blocks.shape, scales.shape)
                with torch.cuda.stream(self._side):
                    b_dev = blocks.to(torch.uint8).contiguous().pin_memory().to(self.device, non_blocking=True)
                    s_dev = scales.to(torch.uint8).contiguous().pin_memory().to(self.device, non_blocking=True)
            else:
                b_dev, s_dev = self._copy_expert_tensors(names, expert_idx)
                self._check_pair(b_dev.shape, s_dev.shape)
            loaded = _nbytes(b_dev) + _nbytes(s_dev)
            rows, groups = int(b_dev.shape[0]), int(b_dev.shape[1])
            with torch.cuda.stream(self._side):
                copied = torch.cuda.Event()
                copied.record(self._side)
                packed = torch.empty(ops.packed_bytes(rows, groups), dtype=torch.uint8, device=self.device)
                ops.mxfp4_pack(b_dev, s_dev, out=packed)
                done = torch.cuda.Event()
                done.record(self._side)
            copied.synchronize()
            st.transfer_time_s += time.perf_counter() - start
            pack_start = time.perf_counter()
            done.synchronize()
            st.dequant_time_s += time.perf_counter() - pack_start
        st.loaded_bytes += loaded
        st.miss_loaded_bytes += loaded
        self.cache.layer_loaded_bytes[layer_idx] += loaded
        st.materialization_time_s += time.perf_counter() - start
        st.materializations += 1
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
        self.cache.count_hits(int(layer_idx), int(n_matrices))

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
