"""The oracle's routing against torch's, on the committed golden vectors.

tests/golden/router_e{32,128}.npz hold what the reference's torch CPU ops
(streamed_moe_router.py:268-284, 497, 512-513) produced for 2048 seeded
tokens of the 20B-shape (E = 32) and 120B-shape (E = 128) layers; see
tests/golden/make_router_golden.py.
"""

from __future__ import annotations

import zlib
from pathlib import Path

import numpy as np
import pytest

from klcquant_amd import moe, synth
from oracle import experts, router

GOLDEN = Path(__file__).resolve().parent / "golden"
HIDDEN = 2880


def load_case(name: str):
    g = np.load(GOLDEN / f"{name}.npz", allow_pickle=False)
    workload, n_exp = int(g["workload"]), int(g["n_experts"])
    # the router tensors of moe.synthetic_host_layer(workload, 0, ...), without its experts
    host = {
        "router_weight": synth.random_normal_bf16(synth.tensor_seed(workload, "router_weight"), n_exp * HIDDEN,
                                                  0.0, 0.02).reshape(n_exp, HIDDEN),
        "router_bias": synth.random_normal_bf16(synth.tensor_seed(workload, "router_bias"), n_exp, 0.0, 0.01),
    }
    x = moe.synthetic_hidden(workload, g["ids"].shape[0], HIDDEN)
    return g, x, host


def torch_logits(g, ours: np.ndarray) -> np.ndarray:
    """torch's F.linear logits: the correctly rounded ones patched where the fixture records a difference."""
    out = ours.copy()
    d = g["logit_diffs"]
    out[d[:, 0], d[:, 1]] = d[:, 2].astype(np.uint16)
    return out


@pytest.mark.parametrize("name,max_diff_tokens", [("router_e32", 16), ("router_e128", 48)])
def test_oracle_routing_equals_torch_on_golden_tokens(name, max_diff_tokens):
    g, x, host = load_case(name)
    ours = router.router_logits(x, host["router_weight"], host["router_bias"])
    theirs = torch_logits(g, ours)
    # the patched rows reproduce torch's logits exactly: every row's CRC matches
    crc = np.array([zlib.crc32(theirs[t].tobytes()) for t in range(theirs.shape[0])], dtype=np.uint32)
    assert np.array_equal(crc, g["logits_crc"])
    # F.linear's float32 accumulation order moves one logit by one bf16 ulp on a few tokens
    diff_tokens = np.unique(g["logit_diffs"][:, 0])
    assert len(diff_tokens) <= max_diff_tokens
    # top-k order (ties included) and bf16 softmax weights are torch's on every token
    ids, values = router.topk(theirs, 4)
    assert np.array_equal(ids, g["ids"].astype(np.int64))
    assert np.array_equal(router.softmax_weights(values), g["weights"])
    # on the oracle's own (correctly rounded) logits only the tokens with a differing logit may route differently
    own_ids, own_vals = router.topk(ours, 4)
    same = np.ones(ids.shape[0], bool)
    same[diff_tokens] = False
    assert np.array_equal(own_ids[same], ids[same])
    assert np.array_equal(router.softmax_weights(own_vals)[same], g["weights"][same])
    changed = int(np.count_nonzero(np.any(own_ids != ids, axis=1)))
    print(f"{name}: {len(diff_tokens)} tokens with a differing F.linear logit, {changed} of them route differently")


@pytest.mark.parametrize("name", ["router_e32", "router_e128"])
def test_oracle_combine_equals_torch_bits(name):
    g = np.load(GOLDEN / f"{name}.npz", allow_pickle=False)
    n = g["combine_crc"].shape[0]
    outs = synth.random_normal_f32(int(g["combine_seed"]), n * 4 * HIDDEN, 0.0, 64.0).reshape(n, 4, HIDDEN)
    got = experts.combine(outs, g["weights"][:n])
    crc = np.array([zlib.crc32(got[t].tobytes()) for t in range(n)], dtype=np.uint32)
    assert np.array_equal(crc, g["combine_crc"])


def test_golden_ties_are_present():
    """The fixtures exercise the tie order: boundary and in-set ties among their tokens."""
    for name in ("router_e32", "router_e128"):
        g, x, host = load_case(name)
        logits = torch_logits(g, router.router_logits(x, host["router_weight"], host["router_bias"]))
        vals = np.sort(synth.bf16_bits_to_f32(logits), axis=1)[:, ::-1]
        ties = np.any(vals[:, :4] == vals[:, 1:5], axis=1)
        assert int(ties.sum()) >= 40, name


def boundary_cases():
    """tests/golden/router_boundary.npz (make_router_boundary_golden.py): per case the token's hidden row, the
    crafted router (weight row f = row e, bias vector) and what torch's CPU ops made of it."""
    g = np.load(GOLDEN / "router_boundary.npz", allow_pickle=False)
    routers = {}
    for ri, name in enumerate(("router_e32", "router_e128")):
        gg, x, host = load_case(name)
        routers[ri] = (x, host, int(gg["n_experts"]))
    cases = []
    for i in range(g["token"].shape[0]):
        x, host, n_exp = routers[int(g["router"][i])]
        e, f = int(g["e"][i]), int(g["f"][i])
        w = host["router_weight"].copy()
        if f >= 0:
            w[f] = g["w_row"][i]
        cases.append(dict(x=x[int(g["token"][i])][None, :], w=w, b=g["bias"][i][:n_exp], e=e, f=f,
                          ids=g["ids"][i].astype(np.int64), weights=g["weights"][i],
                          logits=g["logits"][i][:n_exp], oracle_same=bool(g["oracle_same"][i])))
    return cases


def test_oracle_on_crafted_boundary_routers():
    """Routers crafted so that the logit where torch's F.linear differs from the correctly rounded value is a
    selected one (44 cases) or sits at the top-4 boundary against a copy of its own row (40 cases)."""
    cases = boundary_cases()
    assert len(cases) >= 80
    n_diff = 0
    for c in cases:
        ours = router.router_logits(c["x"], c["w"], c["b"])[0]
        theirs = c["logits"]
        # torch's row differs from the correctly rounded one at e (and at f, the copy of row e) only
        differ = set(np.nonzero(ours != theirs)[0].tolist())
        assert c["e"] in differ and differ <= {c["e"], c["f"]}
        srt = np.argsort(-synth.bf16_bits_to_f32(theirs), kind="stable")
        if c["f"] < 0:
            assert srt[3] == c["e"]  # e is torch's 4th largest
        else:
            assert {int(srt[3]), int(srt[4])} == {c["e"], c["f"]}  # e and f are torch's 4th and 5th
        # the oracle's top-k (torch's order) on torch's own logits gives torch's routing
        ids, vals = router.topk(theirs[None, :], 4)
        assert np.array_equal(ids[0], c["ids"])
        assert np.array_equal(router.softmax_weights(vals)[0], c["weights"])
        # on the correctly rounded logits the routing is torch's exactly where the fixture says so
        own_ids, own_vals = router.topk(ours[None, :], 4)
        same = np.array_equal(own_ids[0], c["ids"]) and np.array_equal(router.softmax_weights(own_vals)[0],
                                                                         c["weights"])
        assert same == c["oracle_same"]
        n_diff += not same
    # these cases are where the correctly rounded router and torch's part ways
    assert n_diff == sum(not c["oracle_same"] for c in cases) and n_diff > 0
    print(f"{len(cases)} crafted boundary cases, {n_diff} route differently from torch")
