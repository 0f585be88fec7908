"""Host logic of the reference-shaped API: expert cache eviction, routing
telemetry and routing-locality selection.  Expected values are worked out by
hand from the rules each docstring cites; nothing here touches a GPU."""

from __future__ import annotations

import json
import math

import numpy as np
import pytest
import torch

from klcquant_amd import mxfp4_expert as mx
from klcquant_amd import streamed_moe_router as smr


def item(n=4):
    return torch.zeros(n, dtype=torch.uint8)


def test_fp4_table_is_the_e2m1_code_table():
    # E2M1: sign bit 3, exponent bits 2..1 (bias 1), mantissa bit 0; code 1 is the subnormal 0.5
    for code in range(16):
        s, e, m = code >> 3, (code >> 1) & 3, code & 1
        mag = (m * 0.5) if e == 0 else (1 + m / 2) * 2.0 ** (e - 1)
        assert mx.FP4_VALUES[code] == (-mag if s else mag)
        assert math.copysign(1.0, mx.FP4_VALUES[code]) == (-1.0 if s else 1.0)


def test_cache_disabled_budget_stores_nothing():
    c = mx.ExpertWeightCache(0)
    c.put((0, 1, "down_proj"), item())
    assert not c.contains((0, 1, "down_proj")) and c.current_bytes == 0


def test_cache_evicts_least_recently_used():
    c = mx.ExpertWeightCache(12)  # three 4-byte items
    a, b, d, e = (0, 0, "gate_up_proj"), (0, 1, "gate_up_proj"), (0, 2, "gate_up_proj"), (0, 3, "gate_up_proj")
    for key in (a, b, d):  # clock 1, 2, 3
        c.put(key, item())
    assert c.get(a) is not None  # clock 4; recency order b, d, a
    c.put(e, item())  # clock 5, 16 bytes > 12: b is the least recently used
    assert not c.contains(b) and c.contains(a) and c.contains(d) and c.contains(e)
    assert list(c.eviction_log) == [b]
    assert c.stats.evictions == 1 and c.stats.hits == 1 and c.current_bytes == 12
    assert c.to_json()["evicted_lifetime"]["mean_accesses"] == 3  # born at clock 2, evicted at 5
    assert c.get(b) is None and c.stats.misses == 1
    assert c.eviction_reasons["global_pressure"] == 1


def test_cache_holds_protect_until_their_window_ends():
    c = mx.ExpertWeightCache(8)
    a, b, d = (1, 0, "down_proj"), (1, 1, "down_proj"), (1, 2, "down_proj")
    c.put(a, item())  # clock 1
    c.put(b, item())  # clock 2
    c.get(a)  # clock 3; order b, a
    c.hold([b], 100)  # b held until clock 103
    c.put(d, item())  # clock 4; order b, a, d: b is held, so a (next least recent) goes
    assert c.contains(b) and c.contains(d) and not c.contains(a)
    assert c.stats.protected_eviction_skips == 0
    # once the window has passed, b is ordinary again
    c2 = mx.ExpertWeightCache(8)
    c2.put(a, item())  # 1
    c2.put(b, item())  # 2
    c2.hold([a], 2)  # a held until clock 4
    for _ in range(3):
        c2.get(b)  # clocks 3, 4, 5; order a, b
    c2.put(d, item())  # clock 6: a's hold ended at 4, so a goes
    assert not c2.contains(a) and c2.contains(b)


def test_cache_hold_before_arrival_and_all_held():
    c = mx.ExpertWeightCache(8)
    a, b, d = (1, 0, "down_proj"), (1, 1, "down_proj"), (1, 2, "down_proj")
    c.put(a, item())
    c.put(b, item())
    c.set_future_scores([a, b, d], protect_window=100)  # the reference's name; d is not resident yet
    c.put(d, item())  # d arrives held; every candidate is held: the least recently used (a) goes
    assert not c.contains(a) and c.contains(b) and c.contains(d)
    assert c.stats.protected_eviction_skips == 1


def test_cache_pinned_items_survive():
    c = mx.ExpertWeightCache(8)
    a, b, d = (2, 0, "down_proj"), (2, 1, "down_proj"), (2, 2, "down_proj")
    c.put(a, item(), pin=True)
    c.put(b, item())
    c.put(d, item())  # a is the least recent but pinned: b goes
    assert c.contains(a) and not c.contains(b) and c.stats.evictions == 1
    assert c.get(a) is not None and c.stats.pinned_hits == 1
    assert c.pinned == {a}


def test_cache_layer_quota_evicts_from_the_over_quota_layer():
    c = mx.ExpertWeightCache(16, layer_count=2, layer_aware=True)  # quota 8 bytes per layer
    l0 = [(0, i, "down_proj") for i in range(3)]
    for key in l0:
        c.put(key, item())
    for key in l0:
        c.get(key)
    new = (1, 0, "down_proj")
    c.put(new, item())  # 16 bytes: at budget, nothing evicted
    assert c.stats.evictions == 0
    newer = (1, 1, "down_proj")
    c.put(newer, item())  # layer 0 holds 12 of its 8 bytes (layer 1: 8 of 8): layer 0's oldest goes
    assert c.contains(new) and c.contains(newer)
    assert list(c.eviction_log) == [l0[0]]
    assert c.eviction_reasons["layer_quota_pressure"] == 1


def test_cache_adaptive_quota_follows_relative_hit_rates():
    c = mx.ExpertWeightCache(16, layer_count=2, layer_aware=True, adaptive_layer_quota=True,
                             adaptive_layer_quota_strength=1.5)
    hot, cold = (0, 0, "down_proj"), (1, 0, "down_proj")
    c.put(hot, item())
    c.put(cold, item())
    assert c.layer_quota(0) == 8.0  # fewer than 32 lookups: the even split
    for _ in range(32):
        c.get(hot)  # layer 0: 32 of 32 found
    for i in range(32):
        c.get(cold if i % 2 else (1, 9, "down_proj"))  # layer 1: 16 of 32 found
    # mean hit rate 0.75: quota 8 * (1 + 1.5 * (1.0 - 0.75)) and 8 * (1 + 1.5 * (0.5 - 0.75))
    assert c.layer_quota(0) == pytest.approx(11.0) and c.layer_quota(1) == pytest.approx(5.0)
    assert c.to_json()["adaptive_layer_quota"] is True


def test_cache_eviction_sequence_matches_the_committed_fixture():
    """A scripted mix of puts, lookups, holds and pins over 3 layers with layer quotas; the victims
    and counters are the committed fixture (tests/golden/make_cache_golden.py)."""
    from pathlib import Path

    import sys
    sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
    import make_cache_golden as g

    want = json.loads((Path(__file__).resolve().parent / "golden" / "expert_cache_eviction.json").read_text())
    assert g.run_script() == want


def test_cache_to_json_is_serialisable_and_consistent():
    c = mx.ExpertWeightCache(8)
    c.put((0, 0, "gate_up_proj"), item())
    c.get((0, 0, "gate_up_proj"))
    c.get((0, 9, "gate_up_proj"))
    js = c.to_json()
    json.dumps(js)
    assert js["hits"] == 1 and js["misses"] == 1 and js["hit_rate"] == 0.5
    assert js["resident_items"] == 1 and js["resident_bytes"] == 4
    assert js["layer_activity"] == [{"layer": 0, "hits": 1, "misses": 1, "hit_rate": 0.5, "evictions": 0,
                                     "loaded_mb": 0.0, "hit_mb": round(4 / 2**20, 6)}]


def test_store_requires_a_gpu_device(tmp_path):
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {}}))
    with pytest.raises(ValueError, match="GPU"):
        mx.Mxfp4ExpertStore(tmp_path, tmp_path, torch.device("cpu"))


def test_router_stats_closed_forms():
    st = smr.RouterStats()
    st.record_route(3, 10, [1, 2], [0.5, 0.5], [1, 2], False)
    st.record_route(3, 12, [2, 5], [1.0, 0.0], [2, 4], True, predicted_experts=[2, 7])
    js = st.to_json()
    json.dumps(js)
    loc = js["locality"]
    assert js["routed_tokens"] == 2
    assert loc["total_expert_activations"] == 4 and loc["unique_expert_activations"] == 3
    assert loc["reuse_distance"] == {"count": 1, "mean": 2.0, "p50": 2, "p90": 2, "max": 2}
    assert loc["reuse_density"] == 0.25
    assert math.isclose(loc["routing_entropy_mean"], math.log(2) / 2)
    # expert (3,2) twice, (3,1) and (3,5) once: H = -(1/2 ln 1/2 + 2 * 1/4 ln 1/4)
    assert math.isclose(loc["routing_entropy_distribution"], 1.5 * math.log(2))
    assert loc["guarded_adjustments"] == 1 and loc["mean_raw_route_overlap"] == 1.5
    assert loc["prediction_accuracy"] == {"sample_count": 1, "mean_precision": 0.5, "mean_recall": 0.5,
                                          "exact_match_rate": 0.0}
    assert loc["active_expert_set_size_over_time"] == [{"position": 10, "active_expert_count": 2},
                                                       {"position": 12, "active_expert_count": 2}]


def test_router_stats_thrash_and_correlation():
    st = smr.RouterStats()
    st.record_route(0, 0, [1], [1.0], [1], False)
    st.record_cache_delta(0, 0, [1], {"hits": 0, "misses": 0, "evictions": 0}, {"hits": 0, "misses": 2, "evictions": 1})
    st.record_cache_delta(0, 1, [1], {"hits": 0, "misses": 2, "evictions": 1}, {"hits": 2, "misses": 2, "evictions": 1})
    loc = st.to_json()["locality"]
    assert loc["cache_evictions_observed"] == 1 and loc["evictions_per_activation"] == 1.0
    assert loc["expert_thrash_mode"] is True
    assert loc["cache_hit_eviction_correlation"] == {"sample_count": 2, "correlation": -1.0}


def test_topk_order_ties_and_nan():
    v = np.array([1.0, 3.0, 3.0, np.nan, 2.0], dtype=np.float32)
    assert smr._topk_order(v, 4) == [3, 1, 2, 4]


def make_router(**cfg):
    return smr.StreamedMoERouter(4, 7.0, smr.RoutingLocalityConfig(enabled=True, **cfg))


def test_sticky_bonus_pulls_in_a_recent_expert_within_the_margin():
    r = make_router(sticky_strength=0.5)
    r.sticky_scores[0] = {6: 0.2, 7: 1.0}
    logits = np.array([2.0, 1.9, 1.8, 1.7, 0.0, 0.0, 1.5, 1.0], dtype=np.float32)
    adj = r._apply_locality_bias(0, logits, set())
    # floor = 1.7 - 0.5 = 1.2: expert 6 (1.5) gets +0.1, expert 7 (1.0) is below the floor
    assert adj[6] == np.float32(1.5) + np.float32(0.2) * np.float32(0.5) and adj[7] == np.float32(1.0)
    assert smr._topk_order(adj, 4) == [0, 1, 2, 3]
    r.sticky_scores[0] = {6: 1.2}  # +0.6 lifts expert 6 to 2.1, above every raw logit
    adj = r._apply_locality_bias(0, logits, set())
    assert smr._topk_order(adj, 4) == [6, 0, 1, 2]


def test_semantic_guard_caps_bonus_and_restores_raw_experts():
    r = make_router(sticky_strength=10.0, semantic_guard=True, max_sticky_bonus=0.25, min_raw_overlap=4)
    r.sticky_scores[0] = {5: 1.0}
    logits = np.array([2.0, 1.9, 1.8, 1.7, 0.0, 1.6], dtype=np.float32)
    adj = r._apply_locality_bias(0, logits, set())
    assert adj[5] == np.float32(1.6) + np.float32(0.25)
    raw = smr._topk_order(logits, 4)
    picked = smr._topk_order(adj, 4)
    assert picked == [0, 1, 5, 2]
    experts, values, blocked = r._guarded_expert_selection(logits, adj, raw, picked, 4)
    assert experts == [0, 1, 2, 3] and blocked  # all four raw experts must stay
    assert values == [2.0, float(np.float32(1.9)), float(np.float32(1.8)), float(np.float32(1.7))]


def test_exploration_penalty_and_cache_bonus():
    r = make_router(max_hot_experts_per_layer=1, exploration_margin=0.25, cache_aware_strength=1.0)
    r.sticky_scores[0] = {3: 1.0}
    logits = np.array([1.0, 0.9, 0.8, 0.7, 0.6], dtype=np.float32)
    adj = r._apply_locality_bias(0, logits, {4})
    # allowed = hot {3} + first two raw experts {0, 1}; 2 and 4 lose 0.25; 4 is resident but
    # below max - 0.25 = 0.75, so it gets no bonus
    want = logits.copy()
    want[[2, 4]] -= np.float32(0.25)
    assert np.array_equal(adj, want)


def test_predictions_caps_and_adaptation():
    r = make_router(predictive_prefetch=True, prediction_window=4, workload_window=2,
                    dynamic_active_expert_cap=True, max_active_experts_per_token=4)
    r._update_workload_scores(0, [1, 2], [0.75, 0.25])
    r._update_sticky_scores(0, [1, 2], [0.75, 0.25])
    # scores: workload {1: .75, 2: .25}, sticky * .75 {1: .5625, 2: .1875}, history +.5 each
    assert r.predict_experts(0, 1) == [1] and r.predict_experts(0) == [1, 2]
    assert r._effective_expert_count(0, 128) == 4
    r._adapt_active_cap(0, 5, {"hits": 0, "misses": 0, "evictions": 0}, {"hits": 0, "misses": 4, "evictions": 2})
    assert r.dynamic_caps[0] == 3 and r._effective_expert_count(0, 128) == 3
    assert r.stats.cap_events[-1]["reason"] == "eviction_pressure"
    r._adapt_active_cap(0, 6, {"hits": 0, "misses": 0, "evictions": 0}, {"hits": 8, "misses": 1, "evictions": 0})
    assert r.dynamic_caps[0] == 4


def test_router_rejects_unknown_precision():
    with pytest.raises(ValueError):
        smr.StreamedMoERouter(matmul_precision="fp8")


def _eager_workload_update(scores: dict, experts, weights, decay: float) -> int:
    """The update as streamed_moe_router.py:413-424 writes it: every score decays each call.
    Returns the number of scores it dropped."""
    dropped = 0
    for e in list(scores):
        scores[e] *= decay
        if scores[e] < 1e-4:
            del scores[e]
            dropped += 1
    for e, w in zip(experts, weights):
        scores[int(e)] = scores.get(int(e), 0.0) + float(w)
    return dropped


def _same_items(a: dict, b: dict) -> bool:
    if list(a) != list(b):
        return False
    return all((x == y) or (math.isnan(x) and math.isnan(y)) for x, y in zip(a.values(), b.values()))


@pytest.mark.parametrize("seed", range(6))
def test_lazy_workload_scores_equal_the_eager_update(seed):
    """The lazily decayed workload scores equal the reference's eager loop after every call: values bit
    for bit, deletions below 1e-4, dict order (re-added experts move to the end), NaN weights, repeated
    experts in one call and a workload_window changed mid-run."""
    rng = np.random.default_rng(seed)
    r = make_router(predictive_prefetch=True, prediction_window=8, workload_window=3)
    eager: dict[int, dict] = {0: {}, 1: {}}
    dropped = 0
    for call in range(400):
        if call == 200:
            r.locality_config.workload_window = 5
        layer = int(rng.integers(0, 2))
        n = int(rng.integers(1, 5))
        experts = [int(e) for e in rng.integers(0, 12, size=n)]
        weights = [float(w) for w in (rng.random(n) * (10.0 ** rng.integers(-5, 1, size=n)))]
        if rng.random() < 0.05:  # values the router never produces, but the rule must still match
            weights[0] = [float("nan"), float("inf"), -0.5, 0.0, -0.0, 1e-300][int(rng.integers(0, 6))]
        decay = 1.0 - 1.0 / max(float(r.locality_config.workload_window), 1.0)
        dropped += _eager_workload_update(eager[layer], experts, weights, decay)
        r._update_workload_scores(layer, experts, weights)
        if call % 7 == 0 or call > 390:
            got = r.workload_scores
            for lyr in (0, 1):
                assert _same_items(got.get(lyr, {}), eager[lyr]), (call, lyr)
    assert dropped > 20  # scores fell below 1e-4 and were dropped (and some re-added) along the way


def test_workload_scores_assignment_and_predictions():
    r = make_router(predictive_prefetch=True, prediction_window=4, workload_window=2)
    r.workload_scores = {0: {5: 1.0, 3: 0.25}}
    r._update_workload_scores(0, [3], [0.5])
    assert r.workload_scores == {0: {5: 0.5, 3: 0.625}}
    assert r.predict_experts(0, 2) == [3, 5]
