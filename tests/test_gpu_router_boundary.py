"""GPU routing on routers crafted so that torch's F.linear rounding decides it.

tests/golden/router_boundary.npz (tests/golden/make_router_boundary_golden.py)
holds 84 routers built from the benchmark routers: in each, the one logit of
a token where torch's CPU ``F.linear`` (float32 accumulation) lands one bf16
ulp from the correctly rounded ``bf16(f32(x . w) + b)`` is either the 4th
selected logit (44 cases) or sits at the top-4 boundary against another
expert whose logit equals it on one side and not on the other (40 cases).
The reference routes with torch's logits (streamed_moe_router.py:268-284);
the GPU routes with the correctly rounded ones.  Here the GPU must equal the
oracle (correctly rounded logits, torch's top-k order, torch's softmax) bit
for bit, and it routes the token differently from torch exactly where the
fixture recorded that the correctly rounded logits do: that count is the
whole of the divergence.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor
from klcquant_amd import moe, ops
from oracle import router as orr
from test_golden_router import boundary_cases

pytestmark = pytest.mark.gpu

K = 4


def test_crafted_boundary_routing(gpu):
    cases = boundary_cases()
    layers = {}
    n_diff_torch = 0
    for c in cases:
        n_exp = c["w"].shape[0]
        want_logits = orr.router_logits(c["x"], c["w"], c["b"])
        want_ids, want_vals = orr.topk(want_logits, K)
        want_w = orr.softmax_weights(want_vals)
        x = bf16_tensor(c["x"], gpu)
        wt, bt = bf16_tensor(c["w"], gpu), bf16_tensor(c["b"], gpu)
        # the standalone router kernels
        logits = ops.router_logits(x, wt, bt)
        ids, _, weights = ops.topk_softmax(logits, K)
        # the one-launch decode router inside the layer (small experts: only the routing is compared)
        if n_exp not in layers:
            layers[n_exp] = moe.MoELayer(moe.MoELayerWeights.synthetic(7, 0, c["x"].shape[1], 64, n_exp, gpu), K)
        layer = layers[n_exp]
        layer.w.router_weight.copy_(wt)
        layer.w.router_bias.copy_(bt)
        lids = torch.empty((1, K), dtype=torch.int32, device=gpu)
        lw = torch.empty((1, K), dtype=torch.bfloat16, device=gpu)
        layer.forward(x, ids=lids, weights=lw)
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(logits), want_logits)
        for got_ids, got_w in ((ids, weights), (lids, lw)):
            assert np.array_equal(got_ids.cpu().numpy(), want_ids)
            assert np.array_equal(bf16_bits(got_w), want_w)
        same_as_torch = np.array_equal(want_ids[0], c["ids"]) and np.array_equal(want_w[0], c["weights"])
        assert same_as_torch == c["oracle_same"]
        n_diff_torch += not same_as_torch
    assert n_diff_torch == sum(not c["oracle_same"] for c in cases)
    print(f"{len(cases)} crafted boundary routers: GPU == oracle on all; {n_diff_torch} route differently "
          f"from torch's F.linear rounding", flush=True)
