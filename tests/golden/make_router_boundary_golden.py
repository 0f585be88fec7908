"""Writes tests/golden/router_boundary.npz: crafted routers where a logit on
which torch's ``F.linear`` differs from the correctly rounded value decides
the routing.

The reference's router (streamed_moe_router.py:268-284) takes the top-4 of
``F.linear(hidden, W, b)`` in bf16.  torch's CPU ``F.linear`` accumulates the
dot product in float32, so on a few tokens one logit lands one bf16 ulp away
from the correctly rounded ``bf16(f32(x . w) + b)`` that the GPU router (and
the oracle) compute.  tests/golden/router_e{32,128}.npz record every such
logit (token t, expert e) of the benchmark routers; on those routers none of
them is selected or sits at the top-4 boundary.  This script builds, for
each recorded (t, e), routers on which it does, keeping row e of W and b[e]
(so torch's logit e keeps its differing value):

* ``selected``: three other experts get bias +8, every expert but e and those
  three gets bias -8, so e is the 4th selected expert and the 5th logit is far
  below: the selected set is the same for torch and the correctly rounded
  logits, the softmax weights see the differing value;
* ``boundary``: as above, and another expert f (not e, not one of the three)
  gets a copy of row e and bias b[e] shifted by the smallest number of bf16
  ulps (either direction, up to 64) for which torch sees logits e and f as
  equal and the correctly rounded logits do not, or the other way round.  e
  and f are then the 4th and 5th largest, so which of them is selected
  depends on the differing bit (and, where one side ties, on torch's tie
  order).

For every case torch's own CPU ops (``F.linear``, ``torch.topk(logits.float(),
4)``, ``torch.softmax(...).to(bf16)``) give the ids and weights that are
stored; the reference itself is not imported.  Stored per case: the router
(``name``: 0 = E32, 1 = E128), token, e, f (-1 for ``selected``), the bias
vector, torch's ids, weights and logits row, and whether the correctly
rounded logits route the token the same way (``oracle_same``).  Run from the
repository root:  python tests/golden/make_router_boundary_golden.py
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "kcapw-klcquant_amd"))

from klcquant_amd import moe, synth  # noqa: E402

HIDDEN = 2880
TOKENS = 2048
K = 4
ROUTERS = [("router_e32", 0, 32), ("router_e128", 2, 128)]
BOOST = 0x4100  # +8.0
SINK = 0xC100   # -8.0


def bf16_tensor(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)


def bits_of(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def correctly_rounded(x_bits: np.ndarray, w_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    xf = synth.bf16_bits_to_f32(x_bits).astype(np.float64)
    wf = synth.bf16_bits_to_f32(w_bits).astype(np.float64)
    bf = synth.bf16_bits_to_f32(b_bits)
    out = np.empty(w_bits.shape[0], dtype=np.uint16)
    for e in range(w_bits.shape[0]):
        dot = np.float32(math.fsum(xf * wf[e]))  # bf16 products are exact in float64
        out[e] = synth.f32_to_bf16_bits(np.array([np.float32(dot + bf[e])], dtype=np.float32))[0]
    return out


def torch_route(x_bits, w_bits, b_bits):
    logits = torch.nn.functional.linear(bf16_tensor(x_bits), bf16_tensor(w_bits), bf16_tensor(b_bits))
    top = torch.topk(logits.float(), k=K)
    wts = torch.softmax(top.values, dim=-1).to(torch.bfloat16)
    return bits_of(logits), top.indices.numpy().astype(np.int16), bits_of(wts)


def own_route(logit_bits):
    top = torch.topk(torch.from_numpy(synth.bf16_bits_to_f32(logit_bits)), k=K)
    return top.indices.numpy().astype(np.int16), bits_of(torch.softmax(top.values, dim=-1).to(torch.bfloat16))


def bf16_step(bits: int, n: int) -> int:
    """The bf16 value n ulps away from `bits` (finite, same sign side for small n)."""
    v = synth.bf16_bits_to_f32(np.array([bits], dtype=np.uint16))[0]
    out = bits
    for _ in range(abs(n)):
        up = (n > 0) == (v >= 0)
        out = out + 1 if up else out - 1
        if (out & 0x7FFF) == 0:  # stepped through zero: stop (never reached for the router biases)
            break
    return out


def main() -> None:
    cases = {k: [] for k in ("router", "token", "e", "f", "bias", "w_row", "ids", "weights", "logits",
                             "oracle_same")}
    for ri, (name, workload, n_exp) in enumerate(ROUTERS):
        g = np.load(Path(__file__).resolve().parent / f"{name}.npz", allow_pickle=False)
        host = moe.synthetic_host_layer(workload, 0, HIDDEN, HIDDEN, n_exp)
        x_all = moe.synthetic_hidden(workload, TOKENS, HIDDEN)
        w, b = host["router_weight"], host["router_bias"]
        for t, e, torch_bits in g["logit_diffs"]:
            t, e = int(t), int(e)
            x = x_all[t]
            others = [i for i in range(n_exp) if i != e]
            boosted = others[:3]
            # case "selected"
            bias = np.full(n_exp, SINK, dtype=np.uint16)
            bias[boosted] = BOOST
            bias[e] = b[e]
            variants = [(-1, bias, w)]
            # case "boundary": f = the next expert after the boosted ones, row e copied into it
            f = others[3]
            wf = w.copy()
            wf[f] = w[e]
            for direction in (1, -1):
                for n in range(1, 65):
                    bb = bias.copy()
                    bb[f] = bf16_step(int(b[e]), direction * n)
                    tl, _, _ = torch_route(x, wf, bb)
                    ol = correctly_rounded(x, wf[[e, f]], bb[[e, f]])
                    if (tl[e] == tl[f]) != (ol[0] == ol[1]):
                        variants.append((f, bb, wf))
                        break
            for ff, bb, ww in variants:
                tl, tids, twts = torch_route(x, ww, bb)
                if tl[e] != np.uint16(torch_bits):
                    raise AssertionError(f"{name} token {t}: torch's logit {e} changed with the other rows")
                oids, owts = own_route(correctly_rounded(x, ww, bb))
                cases["router"].append(ri)
                cases["token"].append(t)
                cases["e"].append(e)
                cases["f"].append(ff)
                cases["bias"].append(np.pad(bb, (0, 128 - n_exp)))
                cases["w_row"].append(ww[ff] if ff >= 0 else np.zeros(HIDDEN, np.uint16))
                cases["ids"].append(tids)
                cases["weights"].append(twts)
                cases["logits"].append(np.pad(tl, (0, 128 - n_exp)))
                cases["oracle_same"].append(bool(np.array_equal(oids, tids) and np.array_equal(owts, twts)))
    out = {k: np.array(v) for k, v in cases.items()}
    out["torch_version"] = np.array(torch.__version__)
    np.savez_compressed(Path(__file__).resolve().parent / "router_boundary.npz", **out)
    n = len(out["token"])
    sel = int(np.count_nonzero(out["f"] < 0))
    print(f"{n} cases ({sel} selected, {n - sel} boundary); the correctly rounded logits route "
          f"{int(np.count_nonzero(~out['oracle_same']))} of them differently from torch")


if __name__ == "__main__":
    main()
