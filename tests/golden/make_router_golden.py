"""Writes tests/golden/router_*.npz: torch CPU routing of seeded tokens.

The reference routes one token per call with torch CPU ops
(streamed_moe_router.py:268-284): ``F.linear`` on the 1-D bf16 hidden state,
``torch.topk(logits.float(), k)``, ``torch.softmax(values).to(bf16)``; and
combines the expert outputs in slot order (:497, 512-513):
``output += out.to(bf16) * weights[pos]``.  This script runs exactly those
torch ops (the reference itself is not imported) on the seeded inputs of the
benchmark workloads and stores what they produced:

* ``ids [T, k] int16``, ``weights [T, k] uint16`` (bf16 patterns);
* ``logits_crc [T] uint32``: CRC-32 of each token's bf16 logits row;
* ``logit_diffs [D, 3] int32``: (token, expert, torch bits) for every logit
  where torch's ``F.linear`` differs from the correctly rounded
  ``bf16(f32(x . w) + b)`` (the float32 dot product rounded once from its
  exact value, computed here with ``math.fsum``), so a test can rebuild
  torch's logits exactly from correctly rounded ones;
* ``combine_crc [Tc] uint32``: CRC-32 of the bf16 combine output of the
  first Tc tokens for seeded float32 expert outputs N(0, 64^2) (seed
  ``combine_seed``) and the torch weights above.

Inputs come from ``klcquant_amd.synth`` (counter-based, identical on host and
GPU): workload w, layer 0, ``synthetic_hidden(w, T, H)``.  Run from the
repository root:  python tests/golden/make_router_golden.py
"""

from __future__ import annotations

import math
import sys
import zlib
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "kcapw-klcquant_amd"))

from klcquant_amd import moe, synth  # noqa: E402

HIDDEN = 2880
TOKENS = 2048
COMBINE_TOKENS = 256
K = 4
CASES = {
    # name: (workload seed namespace, experts) -- the 20B-shape layer (E = 32)
    # and the 120B-shape decode layer (E = 128) of the benchmark
    "router_e32": (0, 32),
    "router_e128": (2, 128),
}


def bf16_tensor(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)


def bits_of(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    return synth.f32_to_bf16_bits(np.asarray(x, dtype=np.float32))


def correctly_rounded_logits(x_bits: np.ndarray, w_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    xf = synth.bf16_bits_to_f32(x_bits).astype(np.float64)
    wf = synth.bf16_bits_to_f32(w_bits).astype(np.float64)
    bf = synth.bf16_bits_to_f32(b_bits)
    out = np.empty(w_bits.shape[0], dtype=np.uint16)
    for e in range(w_bits.shape[0]):
        dot = np.float32(math.fsum(xf * wf[e]))  # bf16 products are exact in float64
        out[e] = f32_to_bf16(np.array([np.float32(dot + bf[e])]))[0]
    return out


def make(name: str, workload: int, n_exp: int) -> dict:
    host = moe.synthetic_host_layer(workload, 0, HIDDEN, HIDDEN, n_exp)
    x = moe.synthetic_hidden(workload, TOKENS, HIDDEN)
    w = bf16_tensor(host["router_weight"])
    b = bf16_tensor(host["router_bias"])
    ids = np.zeros((TOKENS, K), dtype=np.int16)
    weights = np.zeros((TOKENS, K), dtype=np.uint16)
    crc = np.zeros(TOKENS, dtype=np.uint32)
    diffs = []
    for t in range(TOKENS):
        hidden = bf16_tensor(x[t])
        logits = torch.nn.functional.linear(hidden, w, b)
        top = torch.topk(logits.float(), k=K)
        wts = torch.softmax(top.values, dim=-1).to(torch.bfloat16)
        ids[t] = top.indices.numpy()
        weights[t] = bits_of(wts)
        lb = bits_of(logits)
        crc[t] = zlib.crc32(lb.tobytes())
        exact = correctly_rounded_logits(x[t], host["router_weight"], host["router_bias"])
        for e in np.nonzero(lb != exact)[0]:
            diffs.append((t, int(e), int(lb[e])))
    # slot-order bf16 combine of seeded float32 expert outputs with the torch weights
    combine_seed = 1000 * workload + 900
    outs = synth.random_normal_f32(combine_seed, COMBINE_TOKENS * K * HIDDEN, 0.0, 64.0).reshape(COMBINE_TOKENS, K, HIDDEN)
    combine_crc = np.zeros(COMBINE_TOKENS, dtype=np.uint32)
    for t in range(COMBINE_TOKENS):
        output = torch.zeros(HIDDEN, dtype=torch.bfloat16)
        wts = bf16_tensor(weights[t])
        for pos in range(K):
            weighted = torch.from_numpy(outs[t, pos]).to(torch.bfloat16) * wts[pos]
            output += weighted
        combine_crc[t] = zlib.crc32(bits_of(output).tobytes())
    return {
        "ids": ids, "weights": weights, "logits_crc": crc,
        "logit_diffs": np.array(diffs, dtype=np.int32).reshape(-1, 3),
        "combine_crc": combine_crc, "combine_seed": np.int64(combine_seed),
        "workload": np.int64(workload), "n_experts": np.int64(n_exp), "hidden": np.int64(HIDDEN),
        "torch_version": np.array(torch.__version__),
        "threads": np.int64(torch.get_num_threads()),
    }


def main() -> None:
    out_dir = Path(__file__).resolve().parent
    for name, (workload, n_exp) in CASES.items():
        data = make(name, workload, n_exp)
        np.savez_compressed(out_dir / f"{name}.npz", **data)
        tokens_with_diff = len(set(data["logit_diffs"][:, 0].tolist()))
        print(f"{name}: {TOKENS} tokens, {len(data['logit_diffs'])} logits differ from the correctly rounded value "
              f"on {tokens_with_diff} tokens", flush=True)


if __name__ == "__main__":
    main()
