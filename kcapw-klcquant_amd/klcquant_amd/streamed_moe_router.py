"""MoE routing and expert execution with the reference router's interface.

``StreamedMoERouter.route`` keeps the signature, return value and telemetry of
streamed_moe_router.py:257-329: logits -> top-k -> softmax weights -> experts
(gate_up, clamped SwiGLU, down) -> weighted bf16 combine, plus RouterStats
bookkeeping.  Every numeric step runs on the GPU through the C ABI
(klc_moe_router_logits, klc_moe_topk_softmax, klc_moe_dispatch,
klc_moe_gate_up, klc_moe_down, klc_moe_combine): experts are read packed
(MXFP4 codes + E8M0 scales) and dequantized inside the GEMV, never
materialised.

Differences a caller can see:

* ``hidden`` may also be ``[B, H]`` (a batch of tokens routed independently);
  the route dict then holds one list per token.  ``position`` may be a list of
  per-row positions.
* none in the selection: equal logits come out in torch's CPU ``topk`` order
  (the GPU replays libstdc++'s nth_element + sort on rows with ties).  The
  logits themselves are correctly rounded, where torch's float32 F.linear
  differs by one bf16 ulp on about 1 token in 60 at E = 128.
* all tensors must be bf16 (the dtype the executor feeds,
  streamed_transformer_executor.py:354-355) and on the GPU.

The host reads the selected experts and weights back once per call, because
the route dict holds them as Python lists.  With a ``ResidentExpertStore`` that
read is the last thing the call does; with a streaming ``Mxfp4ExpertStore`` the
host needs the experts first to bring misses into HBM.
"""

from __future__ import annotations

import ctypes
import functools
import math
import time
from collections import Counter, deque
from dataclasses import dataclass, field
from typing import NamedTuple

import numpy as np
import torch

from . import _native as nat
from . import ops
from .mxfp4_expert import Mxfp4ExpertStore, ResidentExpertStore


class _ResidentPlan(NamedTuple):
    """A resident layer's checked tensors (router weight, router bias, gate_up bias, down bias, the store's
    layer weights), their pointers (the four tensors, then the gate_up and down pointer tables), device and
    sizes."""
    objects: tuple
    ptrs: tuple
    dev: torch.device
    dev_index: int
    n_exp: int
    hidden: int
    inter: int


@functools.lru_cache(maxsize=256)
def _workspace_bytes(n_tok: int, hidden: int, inter: int, n_exp: int, k: int) -> int:
    return ops.workspace_bytes(n_tok, hidden, inter, n_exp, k)


@dataclass
class RoutingLocalityConfig:
    """Routing-locality knobs (fields and defaults of streamed_moe_router.py:12-35)."""

    enabled: bool = False
    sticky_strength: float = 0.0
    sticky_decay: float = 0.92
    semantic_guard: bool = False
    sticky_candidate_margin: float = 0.50
    max_sticky_bonus: float = 0.25
    min_raw_overlap: int = 2
    max_hot_experts_per_layer: int = 0
    active_experts_per_token_cap: int = 0
    exploration_margin: float = 0.25
    cache_aware_strength: float = 0.0
    predictive_prefetch: bool = False
    prediction_window: int = 16
    workload_window: int = 64
    dynamic_active_expert_cap: bool = False
    min_active_experts_per_token: int = 1
    max_active_experts_per_token: int = 0
    cap_eviction_pressure_threshold: float = 0.50
    cap_hit_rate_expand_threshold: float = 0.65
    thrash_evictions_per_activation: float = 0.35
    thrash_reuse_density: float = 0.15
    thrash_active_growth: float = 0.25


def _percentile_summary(values: list[int]) -> dict:
    if not values:
        return {"count": 0, "mean": None, "p50": None, "p90": None, "max": None}
    v = sorted(values)
    n = len(v)
    return {"count": n, "mean": sum(v) / n, "p50": v[int(0.50 * (n - 1))], "p90": v[int(0.90 * (n - 1))],
            "max": v[-1]}


def _entropy(probabilities) -> float:
    return -sum(p * math.log(max(p, 1e-12)) for p in probabilities)


@dataclass
class RouterStats:
    """Routing telemetry; ``to_json`` has the keys of streamed_moe_router.py:54-102."""

    expert_hits: Counter = field(default_factory=Counter)
    routed_tokens: int = 0
    route_events: list[dict] = field(default_factory=list)
    last_seen_position: dict[tuple[int, int], int] = field(default_factory=dict)
    reuse_distances: list[int] = field(default_factory=list)
    active_by_position: dict[int, set[tuple[int, int]]] = field(default_factory=dict)
    route_entropies: list[float] = field(default_factory=list)
    cache_delta_events: list[dict] = field(default_factory=list)
    cap_events: list[dict] = field(default_factory=list)
    guarded_adjustments: int = 0
    blocked_adjustments: int = 0
    raw_overlap_total: int = 0
    route_count: int = 0

    def record_route(self, layer_idx: int, position: int, experts: list[int], weights: list[float],
                     raw_experts: list[int], adjusted: bool, predicted_experts: list[int] | None = None,
                     resident_experts: list[int] | None = None, active_cap: int | None = None,
                     blocked_adjustment: bool = False) -> None:
        """One token's routing decision (streamed_moe_router.py:104-155)."""
        layer_idx, position = int(layer_idx), int(position)
        experts = [int(e) for e in experts]
        raw = [int(e) for e in raw_experts]
        self.routed_tokens += 1
        self.route_count += 1
        entropy = 0
        for w in weights:  # _entropy's sum, term by term in the same order
            w = float(w)
            entropy += w * math.log(max(w, 1e-12))
        entropy = -entropy
        self.route_entropies.append(entropy)
        overlap = len(set(experts) & set(raw))
        self.raw_overlap_total += overlap
        self.guarded_adjustments += int(bool(adjusted))
        self.blocked_adjustments += int(bool(blocked_adjustment))
        active = self.active_by_position.setdefault(position, set())
        distances = []
        for e in experts:
            key = (layer_idx, e)
            self.expert_hits[key] += 1
            active.add(key)
            seen = self.last_seen_position.get(key)
            if seen is not None:
                distances.append(position - seen)
            self.last_seen_position[key] = position
        self.reuse_distances.extend(distances)
        self.route_events.append({
            "position": position, "layer": layer_idx, "experts": experts, "raw_experts": raw,
            "predicted_experts": [int(e) for e in (predicted_experts or [])],
            "resident_experts": [int(e) for e in (resident_experts or [])],
            "weights": [float(w) for w in weights], "route_entropy": entropy, "reuse_distances": distances,
            "sticky_adjusted": adjusted, "blocked_locality_adjustment": blocked_adjustment,
            "raw_route_overlap": overlap, "active_expert_cap": active_cap,
        })

    def record_cache_delta(self, layer_idx: int, position: int, experts: list[int], before: dict, after: dict) -> None:
        delta = {name: int(after.get(name, 0)) - int(before.get(name, 0)) for name in ("hits", "misses", "evictions")}
        self.cache_delta_events.append({"position": int(position), "layer": int(layer_idx),
                                        "experts": [int(e) for e in experts], **delta})

    def record_cache_deltas(self, layer_idx: int, positions: list[int], experts_rows: list[list[int]], before: dict,
                            after: dict) -> None:
        """record_cache_delta for each row of a batch: the first row carries the traffic between the two
        snapshots, the later rows (snapshot ``after`` on both sides) none."""
        layer_idx = int(layer_idx)
        first = {name: int(after.get(name, 0)) - int(before.get(name, 0)) for name in ("hits", "misses", "evictions")}
        later = {name: int(after.get(name, 0)) - int(after.get(name, 0)) for name in ("hits", "misses", "evictions")}
        self.cache_delta_events.extend(
            {"position": int(p), "layer": layer_idx, "experts": [int(e) for e in row], **(later if r else first)}
            for r, (p, row) in enumerate(zip(positions, experts_rows)))

    def record_cap_event(self, layer_idx: int, position: int, old_cap: int, new_cap: int, reason: str, hits: int,
                         misses: int, evictions: int) -> None:
        if old_cap != new_cap:
            self.cap_events.append({"position": int(position), "layer": int(layer_idx), "old_cap": int(old_cap),
                                    "new_cap": int(new_cap), "reason": reason, "hits": int(hits),
                                    "misses": int(misses), "evictions": int(evictions)})

    def _hit_eviction_correlation(self) -> dict:
        n = len(self.cache_delta_events)
        if n == 0:
            return {"sample_count": 0, "correlation": None}
        h = [float(ev.get("hits", 0)) for ev in self.cache_delta_events]
        e = [float(ev.get("evictions", 0)) for ev in self.cache_delta_events]
        mh, me = sum(h) / n, sum(e) / n
        cov = sum((a - mh) * (b - me) for a, b in zip(h, e))
        denom = math.sqrt(sum((a - mh) ** 2 for a in h) * sum((b - me) ** 2 for b in e))
        return {"sample_count": n, "correlation": cov / denom if denom > 0 else None}

    def _prediction_accuracy(self) -> dict:
        rows = [ev for ev in self.route_events if ev.get("predicted_experts")]
        if not rows:
            return {"sample_count": 0, "mean_precision": None, "mean_recall": None, "exact_match_rate": None}
        precision = recall = exact = 0.0
        for ev in rows:
            actual, predicted = set(ev.get("experts", [])), set(ev.get("predicted_experts", []))
            hit = len(actual & predicted)
            precision += hit / max(len(predicted), 1)
            recall += hit / max(len(actual), 1)
            exact += float(actual == predicted)
        n = len(rows)
        return {"sample_count": n, "mean_precision": precision / n, "mean_recall": recall / n,
                "exact_match_rate": exact / n}

    def to_json(self) -> dict:
        activations = sum(self.expert_hits.values())
        unique = len(self.expert_hits)
        evictions = sum(int(ev.get("evictions", 0)) for ev in self.cache_delta_events)
        active_rows = [{"position": int(p), "active_expert_count": len(s)}
                       for p, s in sorted(self.active_by_position.items())]
        growth = 0.0
        if len(active_rows) >= 2:
            first = active_rows[0]["active_expert_count"]
            growth = (active_rows[-1]["active_expert_count"] - first) / max(first, 1)
        reuse_density = len(self.reuse_distances) / max(activations, 1)
        per_activation = evictions / max(activations, 1)
        per_1k = 1000.0 * evictions / max(self.routed_tokens, 1)
        thrash = per_activation >= 0.35 and (reuse_density <= 0.15 or growth >= 0.25 or per_1k >= 1000.0
                                             or unique >= max(activations * 0.50, 1))
        distribution = _entropy(c / activations for c in self.expert_hits.values()) if activations else 0.0
        return {
            "routed_tokens": self.routed_tokens,
            "expert_activation_frequency": {str(k): v for k, v in self.expert_hits.most_common()},
            "locality": {
                "total_expert_activations": activations,
                "unique_expert_activations": unique,
                "reuse_density": reuse_density,
                "reuse_distance": _percentile_summary(self.reuse_distances),
                "routing_entropy_mean": sum(self.route_entropies) / max(len(self.route_entropies), 1),
                "routing_entropy_distribution": distribution,
                "active_expert_set_size_over_time": active_rows,
                "active_expert_set_growth": growth,
                "cache_evictions_observed": evictions,
                "evictions_per_activation": per_activation,
                "evictions_per_1k_routed_tokens": per_1k,
                "expert_thrash_mode": thrash,
                "cache_hit_eviction_correlation": self._hit_eviction_correlation(),
                "prediction_accuracy": self._prediction_accuracy(),
                "dynamic_cap_events": self.cap_events[:500],
                "guarded_adjustments": int(self.guarded_adjustments),
                "blocked_adjustments": int(self.blocked_adjustments),
                "mean_raw_route_overlap": self.raw_overlap_total / max(self.route_count, 1),
            },
            "route_events": self.route_events[:500],
            "cache_delta_events": self.cache_delta_events[:500],
        }


class _WorkloadScores:
    """One layer's workload scores (streamed_moe_router.py:413-424) with the per-call decay applied
    lazily.

    The reference multiplies every score by ``decay`` on every routed token
    and drops a score once it falls below 1e-4, then adds the token's
    weights.  Here an entry holds its value as of the last call that touched
    it (``[value, tick]``); the decays of the calls since are applied when it
    is touched again or read, one multiplication at a time with the same
    deletion test after each, so every value, every deletion and the dict
    order (a deleted and re-added expert moves to the end) come out as the
    eager loop's.  A change of ``decay`` first settles every entry with the
    old factor.
    """

    __slots__ = ("entries", "tick", "decay")

    def __init__(self) -> None:
        self.entries: dict[int, list] = {}  # expert -> [value, tick of its last update]
        self.tick = 0
        self.decay: float | None = None

    @staticmethod
    def _decayed(value: float, n: int, decay: float):
        """``value`` after n decays, or None once a step leaves it below 1e-4.

        With 0 <= decay < 1 a rounded product never exceeds its positive
        factor, so a positive value only shrinks: it went below 1e-4 at some
        step exactly when it ends below.  A value <= 0 is below after the
        first step and stays there; NaN and +inf never are.  So one test
        after the n multiplications decides as the per-step test does.
        """
        if n <= 0:
            return value
        for _ in range(n):
            value *= decay
        return None if value < 1e-4 else value

    def settle(self) -> None:
        """Applies every pending decay (deleting the scores that fall below 1e-4)."""
        if self.decay is None:
            return
        for e, ent in list(self.entries.items()):
            if ent[1] != self.tick:
                v = self._decayed(ent[0], self.tick - ent[1], self.decay)
                if v is None:
                    del self.entries[e]
                else:
                    ent[0], ent[1] = v, self.tick

    def update(self, experts, weights, decay: float) -> None:
        if decay != self.decay:
            self.settle()
            self.decay = decay
        self.tick += 1
        tick, entries = self.tick, self.entries
        for e, w in zip(experts, weights):
            e = int(e)
            ent = entries.get(e)
            if ent is not None:
                v = self._decayed(ent[0], tick - ent[1], decay)
                if v is not None:
                    ent[0], ent[1] = v + float(w), tick
                    continue
                del entries[e]  # fell below 1e-4 before this call's add: re-added at the end
            entries[e] = [0.0 + float(w), tick]

    def as_dict(self) -> dict[int, float]:
        self.settle()
        return {e: ent[0] for e, ent in self.entries.items()}

    @classmethod
    def from_dict(cls, scores: dict) -> "_WorkloadScores":
        st = cls()
        st.entries = {int(e): [float(v), 0] for e, v in scores.items()}
        return st


def _topk_order(values: np.ndarray, k: int) -> list[int]:
    """``torch.topk(values, k).indices`` of float32 host values (streamed_moe_router.py:271-273).

    The routing-locality path selects on the host, row by row, as the
    reference does; torch's own CPU top-k gives its order of equal values.
    """
    t = torch.from_numpy(np.ascontiguousarray(values, dtype=np.float32))
    return [int(i) for i in torch.topk(t, int(k)).indices.tolist()]


class StreamedMoERouter:
    """Router + expert executor (streamed_moe_router.py:236-529) on the gfx950 kernels."""

    def __init__(self, experts_per_token: int = 4, swiglu_limit: float = 7.0,
                 locality_config: RoutingLocalityConfig | None = None, matmul_precision: str = "fp32") -> None:
        if matmul_precision not in ops.PRECISIONS:
            raise ValueError(f"unknown matmul precision {matmul_precision!r} (expected 'fp32' or 'bf16')")
        self.experts_per_token = experts_per_token
        self.swiglu_limit = swiglu_limit
        self.alpha = 1.702  # fixed in the SwiGLU kernel
        self.stats = RouterStats()
        self.locality_config = locality_config or RoutingLocalityConfig()
        self.matmul_precision = matmul_precision
        self.sticky_scores: dict[int, dict[int, float]] = {}
        self._workload: dict[int, _WorkloadScores] = {}
        self.recent_history: dict[int, deque[int]] = {}
        self.dynamic_caps: dict[int, int] = {}
        # scratch of the resident-store path per (device, stream): workspace, float32 SwiGLU rows,
        # routing record on the device and its pinned host copy
        self._route_scratch: dict[tuple, tuple[torch.Tensor, ...]] = {}
        self._tag = 0  # klc_moe_route_readback's tag of the last call (1 .. 2^31 - 1, then again from 1)
        self._plans: dict[int, _ResidentPlan] = {}
        self._layer_names: dict[int, tuple[str, str, str, str]] = {}
        self._scratch_fit: dict[tuple, tuple[torch.Tensor, ...]] = {}
        # a streaming store's expert pointers per (device, layer, experts): device table and host mirror
        self._ptr_tables: dict[tuple, tuple[torch.Tensor, list]] = {}

    # ---- the routed layer -------------------------------------------------------------

    def route(self, layer_idx: int, hidden: torch.Tensor, tensors: dict[str, torch.Tensor],
              expert_store: Mxfp4ExpertStore | ResidentExpertStore | None = None, execute_experts: bool = True,
              position: int | list[int] = 0, predicted_experts: list[int] | None = None,
              resident_experts: set[int] | None = None) -> tuple[torch.Tensor, dict]:
        names = self._layer_names.get(layer_idx)
        if names is None:
            prefix = f"model.layers.{layer_idx}.mlp"
            names = self._layer_names[layer_idx] = (f"{prefix}.router.weight", f"{prefix}.router.bias",
                                                    f"{prefix}.experts.gate_up_proj_bias",
                                                    f"{prefix}.experts.down_proj_bias")
        router_w = tensors[names[0]]
        router_b = tensors[names[1]]
        if hidden.dim() not in (1, 2):
            raise ValueError(f"hidden must be [H] or [B, H], got shape {tuple(hidden.shape)}")
        batched = hidden.dim() == 2
        n_tok = hidden.shape[0] if batched else 1
        positions = [int(position)] * n_tok if isinstance(position, int) else [int(p) for p in position]
        if len(positions) != n_tok:
            raise ValueError(f"{len(positions)} positions for {n_tok} tokens")
        resident = sorted(int(e) for e in (resident_experts or ()))
        gu_bias = tensors.get(names[2])
        d_bias = tensors.get(names[3])
        run_experts = execute_experts and expert_store is not None
        if (run_experts and not self.locality_config.enabled and isinstance(expert_store, ResidentExpertStore)
                and gu_bias is not None and d_bias is not None):
            # the whole layer and its expert_logs in one library call
            k = self._effective_expert_count(layer_idx, int(router_w.shape[0]))
            before = self._cache_snapshot(expert_store)
            output, host, norms = self._route_resident(layer_idx, hidden.contiguous(), n_tok, router_w, router_b,
                                                       gu_bias, d_bias, expert_store, k)
            return self._finish_route(layer_idx, k, batched, positions, predicted_experts, resident, host, output,
                                      "mxfp4_expert_matmul", True, norms, expert_store, before, False)
        x = (hidden if batched else hidden.reshape(1, -1)).contiguous()
        k = self._effective_expert_count(layer_idx, int(router_w.shape[0]))
        recorded = self.locality_config.enabled  # the locality path records each row while it selects
        if not recorded:
            # one launch (up to 128 tokens) and one read-back: a streaming store needs the experts on the
            # host to bring misses into HBM before the expert kernels run
            ids, weights, host = self._select_on_device(x, router_w, router_b, k)
        else:
            logits = ops.router_logits(x, router_w, router_b)
            ids, weights, host = self._select_on_host(layer_idx, logits, k, resident_experts or set(), positions)

        norms = None
        before = None
        if run_experts:
            before = self._cache_snapshot(expert_store)
            for row in host[0]:
                expert_store.protect_experts(layer_idx, row)
            if gu_bias is None or d_bias is None:
                output, mode = torch.zeros_like(hidden), "mxfp4_missing_bias"
            else:
                output, norms = self._execute_experts(layer_idx, x, ids, weights, gu_bias, d_bias, expert_store,
                                                      host)
                output, mode = output.reshape(hidden.shape), "mxfp4_expert_matmul"
        elif d_bias is None:
            output, mode = torch.zeros_like(hidden), "router_only"
        else:
            chunk = ops.max_tokens_per_call(k)
            output = torch.cat([ops.bias_combine(d_bias, ids[t0:t0 + chunk], weights[t0:t0 + chunk])
                                for t0 in range(0, n_tok, chunk)])
            output, mode = output.reshape(hidden.shape), "bias_only_moe"

        return self._finish_route(layer_idx, k, batched, positions, predicted_experts, resident, host, output,
                                  mode, run_experts, norms, expert_store, before, recorded)

    def _finish_route(self, layer_idx, k, batched, positions, predicted_experts, resident, host, output, mode,
                      run_experts, norms, expert_store, before, recorded):
        """RouterStats bookkeeping and the route dict (streamed_moe_router.py:296-329)."""
        n_tok = len(positions)
        if not recorded:
            for r in range(n_tok):  # locality disabled: the selection is the raw top-k
                predicted = [int(e) for e in (predicted_experts if predicted_experts is not None
                                              else self.predict_experts(layer_idx, k))]
                host[4].append(predicted)
                self.stats.record_route(layer_idx, positions[r], host[0][r], host[1][r], host[2][r], False,
                                        predicted_experts=predicted, resident_experts=resident, active_cap=k,
                                        blocked_adjustment=False)
                self._update_workload_scores(layer_idx, host[0][r], host[1][r])
        experts_rows, weight_rows, raw_rows, _, predicted_rows = host
        adjusted_rows = [experts_rows[r] != raw_rows[r] for r in range(n_tok)]

        def per_token(rows):
            return rows if batched else rows[0]

        if not run_experts:
            if mode == "router_only":
                return output, {"experts": per_token(experts_rows), "weights": per_token(weight_rows), "mode": mode}
            return output, {"experts": per_token(experts_rows), "raw_experts": per_token(raw_rows),
                            "weights": per_token(weight_rows), "mode": mode,
                            "sticky_adjusted": per_token(adjusted_rows)}

        after = self._cache_snapshot(expert_store)
        self.stats.record_cache_deltas(layer_idx, positions, experts_rows, before, after)  # booked on the first row
        self._adapt_active_cap(layer_idx, positions[-1], before, after)
        route = {"experts": per_token(experts_rows), "weights": per_token(weight_rows), "mode": mode}
        if norms is not None:
            logs = [[{"expert": int(e), "routing_weight": float(w), "gate_up_norm": 0.0, "output_norm": 0.0}
                     for e, w in zip(experts_rows[r], weight_rows[r])] for r in range(n_tok)]
            if callable(norms):  # the norms arrive with the expert kernels, after everything above
                norms = norms()
            for r in range(n_tok):
                for j, entry in enumerate(logs[r]):
                    entry["gate_up_norm"], entry["output_norm"] = (float(v) for v in norms[r * k + j])
            route["expert_logs"] = per_token(logs)
        route.update({"raw_experts": per_token(raw_rows), "predicted_experts": per_token(predicted_rows),
                      "resident_experts": resident, "sticky_adjusted": per_token(adjusted_rows),
                      "active_expert_cap": k})
        return output, route

    # ---- device work ---------------------------------------------------------------------

    # Workspaces up to this size stay with the router between calls; larger
    # ones (long prefills) are allocated per call.
    _KEEP_SCRATCH_BYTES = 256 << 20

    def _scratch(self, dev, stream, n_tok, hidden, inter, n_exp, k):
        """Workspace (zero-filled when made), float32 SwiGLU buffer and routing record (device and
        pinned host) for one klc_moe_route call.

        ``stream`` is the raw stream handle (an int).  One set serves every
        batch size and layer on a stream: the call lays the workspace out for
        its own sizes, any larger buffer will do, and calls on one stream run
        in order; the host reads a record before the next call on the stream
        is made.
        """
        fit_key = (dev, stream, n_tok, hidden, inter, n_exp, k)
        held = self._scratch_fit.get(fit_key)
        if held is not None:
            return held
        # record: ids, bf16 weights, norms and klc_moe_route_readback's tag word
        need = (_workspace_bytes(n_tok, hidden, inter, n_exp, k), n_tok * k * inter, 4 * n_tok * k + 4)
        key = (dev, stream)
        held = self._route_scratch.get(key)
        if held is not None and all(t.numel() >= n for t, n in zip(held, need)):
            if len(self._scratch_fit) < 64:
                self._scratch_fit[fit_key] = held
            return held
        size = [max(n, held[i].numel() if held else 0) for i, n in enumerate(need)]
        made = (torch.zeros(size[0], dtype=torch.uint8, device=dev),
                torch.empty(size[1], dtype=torch.float32, device=dev),
                torch.empty(size[2], dtype=torch.int32, device=dev),
                torch.empty(size[2], dtype=torch.int32, pin_memory=True))
        if need[0] + 4 * need[1] <= self._KEEP_SCRATCH_BYTES:
            self._route_scratch[key] = made
            # sizes that fitted the old set now map to the new one
            self._scratch_fit = {f: t for f, t in self._scratch_fit.items() if f[:2] != key}
        return made

    # A selection that has not reached the host record after this long (with
    # the GPU still busy) is waited for by a synchronisation of the stream.
    _TAG_WAIT_S = 2.0

    def _wait_tag(self, record: np.ndarray, index: int, tag: int, dev) -> None:
        """Spins until the GPU has written ``tag`` into ``record[index]`` (klc_moe_route_readback).  Past
        ``_TAG_WAIT_S`` it synchronises the layer's stream instead, which raises if the device failed."""
        spins = 0
        deadline = None
        while record[index] != tag:
            spins += 1
            if spins & 1023 == 0:
                now = time.perf_counter()
                if deadline is None:
                    deadline = now + self._TAG_WAIT_S
                elif now > deadline:
                    torch.cuda.current_stream(dev).synchronize()
                    if record[index] != tag:
                        raise RuntimeError("route(): the layer finished without its selection in the host record")
                    return

    def _resident_plan(self, layer_idx, router_w, router_b, gu_bias, d_bias, store) -> _ResidentPlan:
        """The checked device, sizes and pointers of a resident layer.  Kept while the router and bias
        tensors and the store's layer are the same objects over the same storage; checked again
        otherwise."""
        w = store.layer(layer_idx)
        ptrs = (router_w.data_ptr(), router_b.data_ptr(), gu_bias.data_ptr(), d_bias.data_ptr(),
                w.gate_up_table.data_ptr(), w.down_table.data_ptr())
        plan = self._plans.get(layer_idx)
        if plan is not None and plan.ptrs == ptrs:
            held = plan.objects
            if held[0] is router_w and held[1] is router_b and held[2] is gu_bias and held[3] is d_bias and held[4] is w:
                return plan
        ops._check_gpu("router weight", router_w, torch.bfloat16, 2)
        ops._check_gpu("router bias", router_b, torch.bfloat16, 1)
        ops._check_gpu("gate_up bias", gu_bias, torch.bfloat16, 2)
        ops._check_gpu("down bias", d_bias, torch.bfloat16, 2)
        dev = ops._same_device(router_w, router_b, gu_bias, d_bias, w.gate_up_table)
        n_exp, inter, hidden = w.n_experts, w.inter, w.hidden
        if tuple(router_w.shape) != (n_exp, hidden) or tuple(router_b.shape) != (n_exp,):
            raise ValueError(f"router shapes mismatch: weight {tuple(router_w.shape)}, bias {tuple(router_b.shape)}, "
                             f"{n_exp} resident experts of hidden size {hidden}")
        if tuple(gu_bias.shape) != (n_exp, 2 * inter) or tuple(d_bias.shape) != (n_exp, hidden):
            raise ValueError(f"expert biases {tuple(gu_bias.shape)} / {tuple(d_bias.shape)} do not match "
                             f"E={n_exp} H={hidden} I={inter}")
        plan = _ResidentPlan((router_w, router_b, gu_bias, d_bias, w), ptrs, dev, dev.index, n_exp, hidden, inter)
        self._plans[layer_idx] = plan
        return plan

    def _route_resident(self, layer_idx, x, n_tok, router_w, router_b, gu_bias, d_bias, store, k):
        """route() for a layer resident in HBM; ``x`` is the contiguous hidden ``[H]`` or ``[B, H]``.

        Up to ``ops.max_tokens_per_call(k)`` tokens: one klc_moe_route_readback
        call, in which the kernel that selects the experts also writes the
        selection (ids, bf16 weights) into the pinned host record, followed by
        the call's tag, and the norms kernel writes the expert_logs norms
        there; the host spins on the tag only, so the caller's bookkeeping
        overlaps the expert kernels, and the norms are returned as a callable
        that waits for the layer's stream.  Longer inputs: klc_moe_route per
        chunk, each followed by one device->host copy of its record (ids,
        bf16 weights and norms in one int32 buffer).

        Returns the bf16 output (``x``'s shape), the host row lists of
        :meth:`_select_on_device` and the per-pair ``[gate_up_norm, output_norm]`` (or the callable
        that returns them).
        """
        plan = self._resident_plan(layer_idx, router_w, router_b, gu_bias, d_bias, store)
        if not isinstance(x, torch.Tensor):
            raise TypeError(f"hidden must be a torch.Tensor, got {type(x).__name__}")
        if x.dtype is not torch.bfloat16:
            raise TypeError(f"hidden must be torch.bfloat16, got {x.dtype}")
        if x.device != plan.dev:
            raise ValueError(f"hidden is on {x.device}, the layer on {plan.dev}")
        hidden, inter, n_exp = plan.hidden, plan.inter, plan.n_exp
        if x.shape[-1] != hidden:
            raise ValueError(f"hidden size {x.shape[-1]} does not match the layer's {hidden}")
        if n_tok == 0:
            raise ValueError("route() needs at least one token")
        store.record_access(layer_idx, 2 * n_tok * k)
        out = torch.empty_like(x)
        stream = torch._C._cuda_getCurrentRawStream(plan.dev_index)
        w_ptrs = plan.ptrs
        prec = ops.PRECISIONS[self.matmul_precision]
        chunk = ops.max_tokens_per_call(k)
        if n_tok <= chunk:
            pairs = n_tok * k
            half = (pairs + 1) // 2
            ws, gated, rec, rec_host = self._scratch(plan.dev, stream, n_tok, hidden, inter, n_exp, k)
            r = rec_host.numpy()
            tag_at = 3 * pairs + half
            r[tag_at] = 0  # the previous call on this stream has finished (its norms were waited for)
            self._tag = tag = self._tag % 0x7FFFFFFF + 1
            rec_p = rec.data_ptr()
            rc = self._route_readback_fn(x.data_ptr(), w_ptrs[0], w_ptrs[1], w_ptrs[4], w_ptrs[2], w_ptrs[5],
                                         w_ptrs[3], n_tok, hidden, inter, n_exp, k, self.swiglu_limit, prec,
                                         nat.PATH_AUTO, ws.data_ptr(), ws.numel(), out.data_ptr(), rec_p,
                                         rec_p + 4 * pairs, gated.data_ptr(), rec_host.data_ptr(), tag, stream)
            if rc < 0:
                raise nat.KlcError("klc_moe_route_readback", int(rc), nat.last_error())
            self._wait_tag(r, tag_at, tag, plan.dev)
            experts = r[:pairs].reshape(n_tok, k).tolist()
            bits = r[pairs:pairs + half].view(np.uint16)[:pairs].astype(np.uint32) << 16
            weights = bits.view(np.float32).reshape(n_tok, k).tolist()

            def norms():
                torch.cuda.current_stream(plan.dev).synchronize()
                return r[pairs + half:pairs + half + 2 * pairs].view(np.float32).reshape(pairs, 2).tolist()

            return out, (experts, weights, [list(row) for row in experts], [False] * n_tok, []), norms
        experts, weights, norms = [], [], []
        for t0 in range(0, n_tok, chunk):
            t1 = min(n_tok, t0 + chunk)
            pairs = (t1 - t0) * k
            half = (pairs + 1) // 2
            ws, gated, rec, rec_host = self._scratch(plan.dev, stream, t1 - t0, hidden, inter, n_exp, k)
            n_rec = pairs + half + 2 * pairs
            row0 = 2 * hidden * t0  # byte offset of row t0 of the bf16 input and output
            rec_p = rec.data_ptr()  # ids, then the bf16 weights, then the norms (int32 words)
            nat.call("klc_moe_route", x.data_ptr() + row0, w_ptrs[0], w_ptrs[1], w_ptrs[4], w_ptrs[2], w_ptrs[5],
                     w_ptrs[3], t1 - t0, hidden, inter, n_exp, k, self.swiglu_limit, prec, nat.PATH_AUTO,
                     ws.data_ptr(), ws.numel(), out.data_ptr() + row0, rec_p, rec_p + 4 * pairs, gated.data_ptr(),
                     rec_p + 4 * (pairs + half), stream)
            rec_host[:n_rec].copy_(rec[:n_rec], non_blocking=True)
            torch.cuda.current_stream(plan.dev).synchronize()
            r = rec_host[:n_rec].numpy()
            experts += r[:pairs].reshape(t1 - t0, k).tolist()
            bits = r[pairs:pairs + half].view(np.uint16)[:pairs].astype(np.uint32) << 16
            weights += bits.view(np.float32).reshape(t1 - t0, k).tolist()
            norms += r[pairs + half:].view(np.float32).reshape(pairs, 2).tolist()
        return out, (experts, weights, [list(row) for row in experts], [False] * n_tok, []), norms

    @functools.cached_property
    def _route_readback_fn(self):
        return getattr(nat.load(), "klc_moe_route_readback")

    def _select_on_device(self, x, router_w, router_b, k):
        """Top-k selection and softmax weights on the GPU (klc_moe_select, streamed_moe_router.py:268-284)
        with one device->host read of ids and weights per chunk of rows.

        Returns the device ids / weights and ``(experts, weights, raw_experts, blocked, predicted)`` host
        row lists; without routing locality the raw experts are the selection and the predictions are
        filled in by the caller.
        """
        ops._check_gpu("hidden", x, torch.bfloat16, 2)
        ops._check_gpu("router weight", router_w, torch.bfloat16, 2)
        ops._check_gpu("router bias", router_b, torch.bfloat16, 1)
        dev = ops._same_device(x, router_w, router_b)
        n_tok, hidden = x.shape
        n_exp = router_w.shape[0]
        if router_w.shape[1] != hidden or router_b.shape[0] != n_exp:
            raise ValueError(f"router shapes mismatch: x {tuple(x.shape)}, weight {tuple(router_w.shape)}, "
                             f"bias {tuple(router_b.shape)}")
        ids = torch.empty((n_tok, k), dtype=torch.int32, device=dev)
        weights = torch.empty((n_tok, k), dtype=torch.bfloat16, device=dev)
        stream = ops._stream(dev)
        chunk = ops.max_tokens_per_call(k)
        experts, w_rows = [], []
        for t0 in range(0, n_tok, chunk):
            t1 = min(n_tok, t0 + chunk)
            pairs = (t1 - t0) * k
            ws, _, _, rec_host = self._scratch(dev, stream.value, t1 - t0, hidden, 32, n_exp, k)
            nat.call("klc_moe_select", x.data_ptr() + 2 * hidden * t0, router_w.data_ptr(), router_b.data_ptr(),
                     t1 - t0, hidden, n_exp, k, ws.data_ptr(), ws.numel(), ids.data_ptr() + 4 * t0 * k,
                     weights.data_ptr() + 2 * t0 * k, stream)
            half = (pairs + 1) // 2
            rec_host[:pairs].copy_(ids[t0:t1].view(-1), non_blocking=True)
            rec_host[pairs:pairs + half].view(torch.int16)[:pairs].copy_(weights[t0:t1].view(-1).view(torch.int16),
                                                                         non_blocking=True)
            torch.cuda.current_stream(dev).synchronize()
            r = rec_host[:pairs + half].numpy()
            experts += r[:pairs].reshape(t1 - t0, k).tolist()
            bits = r[pairs:pairs + half].view(np.uint16)[:pairs].astype(np.uint32) << 16
            w_rows += bits.view(np.float32).reshape(t1 - t0, k).tolist()
        return ids, weights, (experts, w_rows, [list(row) for row in experts], [False] * n_tok, [])

    def _execute_experts(self, layer_idx, x, ids, weights, gu_bias, d_bias, store, host):
        """gate_up + SwiGLU + down + combine and the expert_logs norms for every (token, slot) pair of a
        selection already made (ids / weights on the device): one klc_moe_experts call per chunk of at
        most ``ops.max_tokens_per_call(k)`` rows, the expert kernels klc_moe_layer picks (so every store
        gives the same bits), then one read-back of the norms.  Returns the bf16 output and the per-pair
        ``[gate_up_norm, output_norm]`` host list."""
        n_tok, k = ids.shape
        if isinstance(store, ResidentExpertStore):
            w = store.layer(layer_idx)
            hidden, inter, n_exp = w.hidden, w.inter, w.n_experts
            gu_table, d_table = w.gate_up_table.data_ptr(), w.down_table.data_ptr()
            store.record_access(layer_idx, 2 * n_tok * k)
            keep = None
        else:
            hidden = x.shape[1]
            inter = gu_bias.shape[1] // 2
            n_exp = gu_bias.shape[0]
            # [gate_up pointers, down pointers] of the layer's experts, uploaded only when a selected
            # expert's packed matrices moved (a miss, an eviction); entries of experts not selected may be
            # stale and are never read (the kernels visit the selected experts only)
            key = (x.device, layer_idx, n_exp)
            if key not in self._ptr_tables:
                self._ptr_tables[key] = (torch.zeros((2, n_exp), dtype=torch.int64, device=x.device),
                                         [[0] * n_exp, [0] * n_exp])
            table, mirror = self._ptr_tables[key]
            dirty = False
            # one (gate_up, down) pair per distinct expert of the call: with a cache too small to hold
            # them (cache_bytes = 0, the reference's default) every lookup returns a fresh copy, and a
            # batched call must not keep one per (token, slot); the call holds at most one layer's experts
            keep = {}
            for row in host[0]:
                for e in row:  # the reference's access order: gate_up then down, slot by slot
                    gu = store.packed_expert(layer_idx, e, "gate_up_proj")
                    dn = store.packed_expert(layer_idx, e, "down_proj")
                    if store.matrix_shape(layer_idx, e, "gate_up_proj") != (2 * inter, hidden // 32) or \
                            store.matrix_shape(layer_idx, e, "down_proj") != (hidden, inter // 32):
                        raise ValueError(f"expert {e} of layer {layer_idx} does not match hidden={hidden} "
                                         f"inter={inter}")
                    if e in keep:
                        continue  # the pointer table already holds this call's copy (the same bits)
                    keep[e] = (gu, dn)
                    if mirror[0][e] != gu.data_ptr() or mirror[1][e] != dn.data_ptr():
                        mirror[0][e], mirror[1][e] = gu.data_ptr(), dn.data_ptr()
                        dirty = True
            if dirty:  # ordered on the stream before the kernels that read it (the last ones have finished)
                table.copy_(torch.tensor(mirror, dtype=torch.int64))
            gu_table = table.data_ptr()
            d_table = gu_table + 8 * n_exp
        if tuple(gu_bias.shape) != (n_exp, 2 * inter) or tuple(d_bias.shape) != (n_exp, hidden):
            raise ValueError(f"expert biases {tuple(gu_bias.shape)} / {tuple(d_bias.shape)} do not match "
                             f"E={n_exp} H={hidden} I={inter}")
        ops._check_gpu("expert ids", ids, torch.int32, 2)
        ops._check_gpu("routing weights", weights, torch.bfloat16, 2)
        dev = ops._same_device(x, ids, weights, gu_bias, d_bias)
        out = torch.empty((n_tok, hidden), dtype=torch.bfloat16, device=dev)
        stream = ops._stream(dev)
        chunk = ops.max_tokens_per_call(k)  # longer inputs: consecutive calls on row chunks
        norms = []
        for t0 in range(0, n_tok, chunk):
            t1 = min(n_tok, t0 + chunk)
            pairs = (t1 - t0) * k
            ws, gated, rec, rec_host = self._scratch(dev, stream.value, t1 - t0, hidden, inter, n_exp, k)
            row0 = 2 * hidden * t0
            nat.call("klc_moe_experts", x.data_ptr() + row0, ids.data_ptr() + 4 * t0 * k,
                     weights.data_ptr() + 2 * t0 * k, gu_table, gu_bias.data_ptr(), d_table, d_bias.data_ptr(),
                     t1 - t0, hidden, inter, n_exp, k, self.swiglu_limit, ops.PRECISIONS[self.matmul_precision],
                     nat.PATH_AUTO, ws.data_ptr(), ws.numel(), out.data_ptr() + row0, gated.data_ptr(),
                     rec.data_ptr(), stream)
            rec_host[:2 * pairs].copy_(rec[:2 * pairs], non_blocking=True)
            torch.cuda.current_stream(dev).synchronize()
            norms += rec_host[:2 * pairs].numpy().view(np.float32).reshape(pairs, 2).tolist()
        del keep  # the packed matrices and pointer table outlive the kernels that read them (synchronised)
        return out, norms

    # ---- routing locality (host control logic, streamed_moe_router.py:331-476) ------------

    def _select_on_host(self, layer_idx, logits, k, resident_set, positions):
        """Locality-adjusted selection, row by row, in the order the reference routes tokens.

        The sticky scores a row leaves behind steer the next row, so each row's
        bf16 weights are computed (klc_moe_softmax_weights) and read back before
        the next row is selected.
        """
        rows = logits.float().cpu().numpy()
        n_tok = rows.shape[0]
        ids = torch.empty((n_tok, k), dtype=torch.int32, device=logits.device)
        weights = torch.empty((n_tok, k), dtype=torch.bfloat16, device=logits.device)
        experts_rows, weight_rows, raw_rows, blocked_rows, predicted_rows = [], [], [], [], []
        for r in range(n_tok):
            row = rows[r].astype(np.float32)
            raw = _topk_order(row, k)
            adjusted_logits = self._apply_locality_bias(layer_idx, row, resident_set)
            experts, values, blocked = self._guarded_expert_selection(row, adjusted_logits, raw,
                                                                      _topk_order(adjusted_logits, k), k)
            vals = torch.tensor([values], dtype=torch.float32).to(logits.device)
            w_row = ops.softmax_weights(vals)
            ids[r] = torch.tensor(experts, dtype=torch.int32).to(logits.device)
            weights[r] = w_row[0]
            w_list = w_row.float().cpu()[0].tolist()
            predicted = [int(e) for e in self.predict_experts(layer_idx, k)]
            predicted_rows.append(predicted)
            experts_rows.append(experts)
            weight_rows.append(w_list)
            raw_rows.append(raw)
            blocked_rows.append(blocked)
            self.stats.record_route(layer_idx, positions[r], experts, w_list, raw, experts != raw,
                                    predicted_experts=predicted, resident_experts=sorted(resident_set),
                                    active_cap=k, blocked_adjustment=blocked)
            self._update_sticky_scores(layer_idx, experts, w_list)
            self._update_workload_scores(layer_idx, experts, w_list)
        return ids, weights, (experts_rows, weight_rows, raw_rows, blocked_rows, predicted_rows)

    def _apply_locality_bias(self, layer_idx: int, logits: np.ndarray, resident: set[int]) -> np.ndarray:
        """float32 logits + sticky bonus / exploration penalty / residency bonus (streamed_moe_router.py:331-363)."""
        cfg = self.locality_config
        if not cfg.enabled:
            return logits
        out = logits.astype(np.float32).copy()
        k = min(self.experts_per_token, logits.size)
        raw = _topk_order(logits, k)
        floor = np.float32(logits[raw[-1]]) - np.float32(abs(float(cfg.sticky_candidate_margin)))
        scores = self.sticky_scores.get(layer_idx, {})
        if scores and cfg.sticky_strength > 0:
            eligible = [int(e) for e in scores if logits[int(e)] >= floor]
            if eligible:
                bonus = np.array([scores[e] for e in eligible], dtype=np.float32) * np.float32(cfg.sticky_strength)
                if cfg.semantic_guard and cfg.max_sticky_bonus > 0:
                    bonus = np.minimum(bonus, np.float32(cfg.max_sticky_bonus))
                out[eligible] += bonus
        if cfg.max_hot_experts_per_layer > 0 and len(scores) >= cfg.max_hot_experts_per_layer:
            hot = set(sorted(scores, key=scores.get, reverse=True)[:cfg.max_hot_experts_per_layer])
            allowed = hot | set(raw[:max(1, self.experts_per_token // 2)])
            mask = np.ones(out.size, dtype=bool)
            mask[sorted(allowed)] = False
            out[mask] -= np.float32(abs(float(cfg.exploration_margin)))
        if resident and cfg.cache_aware_strength > 0:
            ids = np.array(sorted(resident), dtype=np.int64)
            threshold = np.float32(np.max(logits)) - np.float32(abs(float(cfg.exploration_margin)))
            eligible = ids[logits[ids] >= threshold]
            if eligible.size:
                out[eligible] += np.float32(cfg.cache_aware_strength)
        return out

    def _guarded_expert_selection(self, logits: np.ndarray, adjusted_logits: np.ndarray, raw_experts: list[int],
                                  adjusted_experts: list[int], k: int) -> tuple[list[int], list[float], bool]:
        """Keeps at least ``min_raw_overlap`` raw experts (streamed_moe_router.py:365-394)."""
        cfg = self.locality_config
        if not (cfg.enabled and cfg.semantic_guard):
            return list(adjusted_experts), [float(adjusted_logits[e]) for e in adjusted_experts], False
        raw = list(raw_experts[:k])
        chosen = list(adjusted_experts[:k])
        need = min(max(int(cfg.min_raw_overlap), 0), k)
        blocked = False
        while len(set(raw) & set(chosen)) < need:
            missing = [e for e in raw if e not in chosen]
            foreign = [e for e in chosen if e not in raw]
            if not missing or not foreign:
                break
            weakest = min(foreign, key=lambda e: float(adjusted_logits[e]))
            chosen[chosen.index(weakest)] = missing[0]
            blocked = True
        chosen.sort(key=lambda e: float(adjusted_logits[e]), reverse=True)
        return chosen, [float(logits[e]) for e in chosen], blocked

    def _update_sticky_scores(self, layer_idx: int, experts: list[int], weights: list[float]) -> None:
        cfg = self.locality_config
        if not cfg.enabled:
            return
        scores = self.sticky_scores.setdefault(layer_idx, {})
        for e in list(scores):
            scores[e] *= float(cfg.sticky_decay)
            if scores[e] < 1e-4:
                del scores[e]
        for e, w in zip(experts, weights):
            scores[int(e)] = scores.get(int(e), 0.0) + float(w)
        cap = cfg.max_hot_experts_per_layer
        if cap > 0 and len(scores) > 2 * cap:
            keep = set(sorted(scores, key=scores.get, reverse=True)[:cap])
            for e in [e for e in scores if e not in keep]:
                del scores[e]

    @property
    def workload_scores(self) -> dict[int, dict[int, float]]:
        """Per-layer workload scores as the reference keeps them (a fresh dict per layer, in the
        reference's insertion order); assigning a dict of dicts replaces them."""
        return {layer: st.as_dict() for layer, st in self._workload.items()}

    @workload_scores.setter
    def workload_scores(self, value: dict) -> None:
        self._workload = {int(layer): _WorkloadScores.from_dict(scores) for layer, scores in value.items()}

    def _update_workload_scores(self, layer_idx: int, experts: list[int], weights: list[float]) -> None:
        """streamed_moe_router.py:413-424: decay every score, drop those below 1e-4, add the token's
        weights (the decay is applied lazily, see _WorkloadScores)."""
        cfg = self.locality_config
        decay = 1.0 - 1.0 / max(float(cfg.workload_window), 1.0)
        st = self._workload.get(layer_idx)
        if st is None:
            st = self._workload[layer_idx] = _WorkloadScores()
        st.update(experts, weights, decay)
        history = self.recent_history.setdefault(layer_idx, deque(maxlen=max(int(cfg.prediction_window), 1)))
        history.extend(int(e) for e, _ in zip(experts, weights))

    def predict_experts(self, layer_idx: int, limit: int | None = None) -> list[int]:
        """Experts likely next for ``layer_idx`` (streamed_moe_router.py:426-440)."""
        cfg = self.locality_config
        if not (cfg.enabled and cfg.predictive_prefetch):
            return []
        scores: Counter[int] = Counter()
        st = self._workload.get(layer_idx)
        for e, v in (st.as_dict() if st is not None else {}).items():
            scores[int(e)] += float(v)
        for e, v in self.sticky_scores.get(layer_idx, {}).items():
            scores[int(e)] += 0.75 * float(v)
        for e in self.recent_history.get(layer_idx, ()):
            scores[int(e)] += 0.50
        if not scores:
            return []
        return [int(e) for e, _ in scores.most_common(max(int(limit or self.experts_per_token), 1))]

    # ---- active-expert cap (streamed_moe_router.py:442-476) --------------------------------

    def _cap_bounds(self) -> tuple[int, int]:
        """(lowest, highest) per-layer cap the dynamic controller may reach."""
        cfg = self.locality_config
        return max(int(cfg.min_active_experts_per_token), 1), int(cfg.max_active_experts_per_token
                                                                  or self.experts_per_token)

    def _effective_expert_count(self, layer_idx: int, expert_count: int) -> int:
        """Experts per token for this call: ``experts_per_token`` limited by the
        expert count and, with locality enabled, by the static cap and the
        layer's dynamic cap.  A layer's dynamic cap starts at the static cap
        (or ``experts_per_token``) brought into the controller's bounds."""
        cfg = self.locality_config
        limits = [self.experts_per_token, expert_count]
        if cfg.enabled:
            if cfg.active_experts_per_token_cap > 0:
                limits.append(int(cfg.active_experts_per_token_cap))
            if cfg.dynamic_active_expert_cap:
                lo, hi = self._cap_bounds()
                start = min(max(cfg.active_experts_per_token_cap or self.experts_per_token, lo), hi)
                limits.append(self.dynamic_caps.setdefault(layer_idx, start))
        return max(min(limits), 1)

    def _adapt_active_cap(self, layer_idx: int, position: int, before: dict, after: dict) -> None:
        """One step of the dynamic cap controller after a routed call.

        The cache traffic of the call (hit / miss / eviction counts between
        the two snapshots) decides: an eviction share at or above
        ``cap_eviction_pressure_threshold`` lowers the cap by one (not below
        the lower bound); otherwise a call without evictions whose hit share
        reaches ``cap_hit_rate_expand_threshold`` raises it by one (not above
        the upper bound).  A layer seen here first starts from the static cap
        (or ``experts_per_token``).
        """
        cfg = self.locality_config
        if not (cfg.enabled and cfg.dynamic_active_expert_cap):
            return
        delta = {name: int(after.get(name, 0)) - int(before.get(name, 0)) for name in ("hits", "misses", "evictions")}
        lookups = max(delta["hits"] + delta["misses"], 1)
        lo, hi = self._cap_bounds()
        cap = self.dynamic_caps.setdefault(layer_idx, cfg.active_experts_per_token_cap or self.experts_per_token)
        step, reason = 0, ""
        if cap > lo and delta["evictions"] / lookups >= float(cfg.cap_eviction_pressure_threshold):
            step, reason = -1, "eviction_pressure"
        elif cap < hi and delta["evictions"] == 0 and delta["hits"] / lookups >= float(cfg.cap_hit_rate_expand_threshold):
            step, reason = +1, "stable_high_hit_rate"
        if step:
            self.dynamic_caps[layer_idx] = cap + step
            self.stats.record_cap_event(layer_idx, position, cap, cap + step, reason, delta["hits"], delta["misses"],
                                        delta["evictions"])

    @staticmethod
    def _cache_snapshot(expert_store) -> dict:
        st = expert_store.cache.stats
        return {"hits": st.hits, "misses": st.misses, "evictions": st.evictions}
