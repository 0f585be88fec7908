"""Writes tests/golden/expert_cache_eviction.json: ExpertWeightCache's victims
and counters for a fixed script of operations.

The script: 600 seeded operations over 3 layers x 12 experts x 2 projections
of 4-, 6- and 8-byte entries against a 96-byte budget with layer-aware
quotas: lookups that insert on a miss (the store's pattern), holds of a few
upcoming experts (protect / prefetch hints), and two pins.  The fixture holds
every victim in order and the final counters; a change of eviction policy
shows up as a different sequence.  Run from the repository root:
python tests/golden/make_cache_golden.py
"""

from __future__ import annotations

import json
import random
import sys
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "kcapw-klcquant_amd"))

from klcquant_amd.mxfp4_expert import ExpertWeightCache  # noqa: E402

PROJS = ("gate_up_proj", "down_proj")


def run_script() -> dict:
    rng = random.Random(20261202)
    cache = ExpertWeightCache(96, layer_count=3, layer_aware=True)
    victims = []
    for step in range(600):
        layer = rng.randrange(3)
        # a skewed expert popularity: low ids are hot
        expert = min(int(rng.expovariate(0.35)), 11)
        op = rng.random()
        if op < 0.12:
            cache.hold([(layer, e, p) for e in (expert, (expert + 1) % 12) for p in PROJS], window=rng.choice((8, 32)))
        else:
            for proj in PROJS:
                key = (layer, expert, proj)
                if cache.get(key) is None:
                    before = len(cache.eviction_log)
                    size = 4 + 2 * ((expert + layer) % 3)
                    cache.put(key, torch.zeros(size, dtype=torch.uint8), pin=(step in (50, 51) and proj == "down_proj"))
                    victims.extend([list(v) for v in list(cache.eviction_log)[before:]])
    js = cache.to_json()
    keep = ("hits", "misses", "evictions", "resident_bytes", "resident_items", "pinned_items",
            "protected_eviction_skips", "eviction_reasons", "layer_activity", "evicted_lifetime")
    return {"victims": victims, "counters": {k: js[k] for k in keep}}


if __name__ == "__main__":
    out = Path(__file__).resolve().parent / "expert_cache_eviction.json"
    data = run_script()
    out.write_text(json.dumps(data, indent=0, sort_keys=True) + "\n")
    print(f"{len(data['victims'])} evictions written to {out}")
