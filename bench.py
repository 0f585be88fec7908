"""Benchmark: gpt-oss-120B-shape MoE layer decode on one MI355X.

Workload: one MoE layer, hidden = intermediate = 2880, 128 MXFP4 experts,
top-4, router 2880 -> 128, executor-default float32 expert matmuls, bf16
activations ~ N(0, 1), seeded synthetic weights (codes uniform, E8M0 scales
uniform in 118..124).  A step is one layer forward over one batch of B tokens
(router -> top-k/softmax -> dispatch -> gate_up + SwiGLU -> down -> combine),
inputs already resident in HBM.  Steps rotate over --layers independent
layers (1.69 GB of packed experts each), so expert bytes come from HBM and not
from a cache left warm by the previous step.

Prints one JSON line.  ``value`` is microseconds per token at the headline
batch (64); ``per_batch`` holds B = 1, 8, 64.  ``stack`` is the 36-layer
MoE-only decode (RMSNorm -> MoE -> residual per layer, 60.9 GB of experts
resident, 64 sequences x 32 steps), ``prefill`` one layer over 2048 tokens
with Zipf(1.1)-skewed routing (grouped GEMM), and ``dequant`` the standalone
MXFP4 -> bf16 dequant of 128 down_proj experts, and ``loader`` the expert
store's misses (page-cache-warm shard -> packed experts in HBM) against the
safe_open chain they replace, ``lm_head`` the gpt-oss logits pass with
the greedy token, and ``attention`` the decode attention core on an fp16 KV
ring; all are extra lines of the same run.  ``roofline`` is for the
dominant kernel (the gate_up GEMV): algorithmic bytes (packed weights of the
experts the batch touches + activations in + SwiGLU output) over its average
duration measured with HIP events recorded by the library between its
kernels, in a second timed pass over the same steps.

Before each batch size is measured, its steps run untimed for at least 150 ms:
the GPU reaches its working clocks only after ~20-30 ms of sustained load.
Then come the per-kernel events pass (K steps), the W untimed warm-up steps,
and the K timed steps.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "kcapw-klcquant_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HIDDEN = 2880
INTER = 2880
EXPERTS = 128
TOPK = 4
WORKLOAD = 2  # seed namespace of the 120B-shape decode workload
HBM_PEAK_GBPS = 8000.0
STATIC_SCRATCH_BYTES = 32 * 1024 * 1024  # KLC_STATIC_SCRATCH_BYTES
SETTLE_MS = 150.0  # untimed steps before each batch size's measurement
GATE_UP_EXPERT_BYTES = 2 * INTER * (HIDDEN // 32) * 17  # 8,812,800: codes + E8M0 scales
DOWN_EXPERT_BYTES = HIDDEN * (INTER // 32) * 17  # 4,406,400
KERNELS = ["router_logits", "topk_softmax", "dispatch", "gate_up", "down", "combine"]
# rocprofv3 FETCH_SIZE + WRITE_SIZE of the gate_up launches at B = 64, scaled by
# the same counters on a copy kernel of known size (written by hand from the
# counter runs; the file states the commands)
TRAFFIC_PROFILE = ROOT / "profiles" / "moe_gemv_gate_up_120b_b64_hbm_traffic.txt"


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batches", default="1,8,64")
    ap.add_argument("--headline-batch", type=int, default=64)
    ap.add_argument("--layers", type=int, default=8, help="independent layers the steps rotate over")
    ap.add_argument("--inputs", type=int, default=16, help="distinct input batches the steps rotate over")
    ap.add_argument("--cpu-tokens", type=int, default=10, help="timed tokens of the CPU baseline sample (0 = skip)")
    ap.add_argument("--precision", default="fp32", choices=["fp32", "bf16"])
    ap.add_argument("--graph", action="store_true",
                    help="replay one HIP graph per step in the headline pass instead of launching its kernels")
    ap.add_argument("--skip-dequant", action="store_true", help="skip the standalone dequant measurement")
    ap.add_argument("--skip-config0", action="store_true", help="skip the 20B-shape single-token layer line")
    ap.add_argument("--prefill-tokens", type=int, default=2048, help="tokens of the prefill measurement (0 = skip)")
    ap.add_argument("--stack-layers", type=int, default=36, help="layers of the stacked decode (0 = skip)")
    ap.add_argument("--stack-steps", type=int, default=32, help="decode steps of the stacked decode")
    ap.add_argument("--skip-lm-head", action="store_true", help="skip the lm_head logits measurement")
    ap.add_argument("--route-calls", type=int, default=300,
                    help="timed single-token StreamedMoERouter.route() calls (0 = skip)")
    ap.add_argument("--skip-attention", action="store_true", help="skip the decode attention measurement")
    ap.add_argument("--loader-experts", type=int, default=16,
                    help="experts of the expert-store miss measurement (0 = skip)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 1 GiB -> 1 GiB float32 copy kernel 5 times (HBM counter calibration)")
    return ap.parse_args()


def measured_traffic() -> int | None:
    """HBM bytes per gate_up launch (B = 64, fp32) from the committed counter summary, if present."""
    try:
        text = TRAFFIC_PROFILE.read_text()
    except OSError:
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", text, re.M)
    return int(m.group(1)) if m else None


def copy_calibration(torch, dev) -> None:
    n = 1 << 28  # float32 elements: 1 GiB read and 1 GiB written per launch
    src = torch.ones(n, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(5):
        torch.mul(src, 2.0, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"copy_kernel": "torch.mul(float32 [2^28], 2.0)", "bytes_read": n * 4, "bytes_written": n * 4,
                      "launches": 5}), flush=True)


def layer_bytes(unique_experts: int, n_tok: int, n_exp: int = EXPERTS) -> int:
    """Algorithmic HBM bytes of one layer step."""
    weights = unique_experts * (GATE_UP_EXPERT_BYTES + DOWN_EXPERT_BYTES)
    biases = unique_experts * (2 * INTER + HIDDEN) * 2
    router = n_exp * HIDDEN * 2 + n_exp * 2
    acts = n_tok * HIDDEN * 2 * 2  # hidden in, output out (bf16)
    return weights + biases + router + acts


def kernel_breakdown(interval_us, n_tok: int, path: str) -> dict:
    """Per-kernel times from the library's KLC_LAYER_EVENTS events.  A batch that runs as one launch
    (path "fused", up to 16 tokens) records the first event before it and the other six after it.
    One token runs three launches (router, gate_up, down with the combine).
    Batches of up to 128 tokens run router, top-k and dispatch as one launch (router_decode_kernel),
    so their events 1 and 2 follow it back to back.  Intervals between back-to-back events measure
    only the event records and are reported apart."""
    us = [round(float(v), 3) for v in interval_us]
    if path == "fused":
        return {"fused_layer": us[0], "event_records_only": round(sum(us[1:]), 3)}
    if n_tok == 1 and path == "gemv":
        # one token: router without dispatch, gate_up by slot, down GEMV + combine in one launch
        return {"router_topk": us[0], "gate_up": us[3], "down_combine": us[4],
                "event_records_only": round(us[1] + us[2] + us[5], 3)}
    if n_tok <= 128:
        return {"router_topk_dispatch": us[0], "gate_up": us[3], "down": us[4], "combine": us[5],
                "event_records_only": round(us[1] + us[2], 3)}
    return dict(zip(KERNELS, us))


def config0_bench(torch, dev, steps: int, warmup: int, precision: str, n_layers: int = 8) -> dict:
    """The gpt-oss-20B-shape layer (E = 32, top-4) decoding one token per step, fp32 expert math: the
    single-token layer of the 20B model.  Steps rotate over n_layers seeded layers (425 MB of packed
    experts each) and 16 inputs; per-kernel times from the library's events in a second pass."""
    import numpy as np

    from klcquant_amd import _native, moe

    n_exp = 32
    layers = [moe.MoELayer(moe.MoELayerWeights.synthetic(0, l, HIDDEN, INTER, n_exp, dev), TOPK, 7.0, precision)
              for l in range(n_layers)]
    xs = [torch.from_numpy(moe.synthetic_hidden(0, 1, HIDDEN, step=s).view(np.int16)).view(torch.bfloat16).to(dev)
          for s in range(16)]
    out = torch.empty((1, HIDDEN), dtype=torch.bfloat16, device=dev)
    t0 = time.perf_counter()
    s = 0
    while (time.perf_counter() - t0) * 1e3 < SETTLE_MS or s < 4:
        layers[s % n_layers].forward(xs[s % 16], out=out)
        s += 1
        if s % 16 == 0:
            torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(_native.LAYER_EVENTS)] for _ in range(steps)]
    for row in evs:
        for e in row:
            e.record()
    torch.cuda.synchronize()
    for s in range(steps):
        layers[s % n_layers].forward(xs[s % 16], out=out, events=evs[s])
    for s in range(warmup):
        layers[s % n_layers].forward(xs[s % 16], out=out)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(steps):
        layers[s % n_layers].forward(xs[s % 16], out=out)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    kern = np.array([[evs[s][i].elapsed_time(evs[s][i + 1]) for i in range(len(KERNELS))] for s in range(steps)])
    moved = layer_bytes(TOPK, 1, n_exp)  # a single token's top-4 are 4 distinct experts
    del layers
    torch.cuda.empty_cache()
    return {"workload": "gpt-oss-20B-shape MoE layer: H=I=2880, 32 MXFP4 experts, top-4, 1 token per step, "
                        "fp32 expert math", "us_per_token": round(dt * 1e6, 3), "tokens_per_s": round(1 / dt, 1),
            "bytes_per_token": moved, "hbm_gbps": round(moved / dt / 1e9, 1),
            "frac_of_peak": round(moved / dt / 1e9 / HBM_PEAK_GBPS, 4),
            "kernel_us_mean": kernel_breakdown(kern.mean(axis=0) * 1e3, 1, "gemv"), "steps": steps}


def gate_up_bytes(unique_experts: int, n_tok: int) -> int:
    """Algorithmic bytes of one gate_up launch: weights + bias + fp32 activations + fp32 SwiGLU output."""
    return (unique_experts * (GATE_UP_EXPERT_BYTES + 2 * INTER * 2) + n_tok * HIDDEN * 4
            + n_tok * TOPK * INTER * 4)


def dequant_bench(torch, dev, reps: int = 10) -> dict:
    """Standalone MXFP4 -> bf16 dequant of 128 down_proj experts ([2880, 90, 16] codes +
    [2880, 90] E8M0 scales each, checkpoint layout) into [128, 2880, 2880] bf16."""
    import numpy as np

    from klcquant_amd import ops

    n, rows, groups = EXPERTS, HIDDEN, INTER // 32
    blocks = torch.empty((n, rows, groups, 16), dtype=torch.uint8, device=dev)
    scales = torch.empty((n, rows, groups), dtype=torch.uint8, device=dev)
    ops.synth_fill(blocks, 1000 * 1 + 7, 0)
    ops.synth_fill(scales, 1000 * 1 + 8, 1, 118, 124)
    out = torch.empty((n, groups * 32, rows), dtype=torch.bfloat16, device=dev)
    from klcquant_amd import _native as nat

    def launch():
        nat.call("klc_mxfp4_dequant", ops._ptr(blocks), ops._ptr(scales), ops._ptr(out), n, rows, groups,
                 nat.DTYPE_BF16, ops._stream(dev))

    for _ in range(3):
        launch()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    torch.cuda.synchronize()
    ev[0].record()
    for i in range(reps):
        launch()
        ev[i + 1].record()
    torch.cuda.synchronize()
    us = float(np.mean([ev[i].elapsed_time(ev[i + 1]) for i in range(reps)])) * 1e3
    moved = n * rows * groups * 17 + n * rows * groups * 32 * 2
    del blocks, scales, out
    return {"workload": "128 x down_proj [2880 x 2880] MXFP4 -> bf16 (checkpoint layout in, [in, out] out)",
            "us": round(us, 2), "bytes": moved, "gbps": round(moved / (us * 1e-6) / 1e9, 1),
            "frac_of_peak": round(moved / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)}


def stack_bench(torch, dev, n_layers: int, n_seqs: int, n_steps: int, precision: str) -> dict:
    """36-layer MoE-only decode: per layer h += moe(rms_norm(h)), every expert resident in HBM;
    n_seqs sequences x n_steps decode steps (a step = one token per sequence through all layers)."""
    import numpy as np

    from klcquant_amd import moe

    t0 = time.perf_counter()
    stack = moe.MoEStack.synthetic(4, n_layers, HIDDEN, INTER, EXPERTS, dev, precision=precision)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t0
    xs = [torch.from_numpy(moe.synthetic_hidden(4, n_seqs, HIDDEN, step=s).view(np.int16)).view(torch.bfloat16)
          .to(dev) for s in range(n_steps)]
    out = torch.empty_like(xs[0])
    ids = [[torch.empty((n_seqs, TOPK), dtype=torch.int32, device=dev) for _ in range(n_layers)]
           for _ in range(n_steps)]
    for s in range(2):
        stack(xs[s], out=out)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(n_steps):
        stack(xs[s], out=out, ids=ids[s])
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    uniq = [len(np.unique(t.cpu().numpy())) for row in ids for t in row]
    moved = float(sum(layer_bytes(u, n_seqs) for u in uniq)) + n_steps * n_layers * (HIDDEN * 2 + n_seqs * HIDDEN * 4)
    resident = sum(int(l.w.gate_up.numel() + l.w.down.numel()) for l in stack.layers)
    del stack
    torch.cuda.empty_cache()
    return {"workload": f"{n_layers}-layer MoE-only stack, gpt-oss-120B shape, rms_norm -> MoE -> residual, "
                        f"{n_seqs} sequences x {n_steps} decode steps",
            "tokens_per_s": round(n_seqs * n_steps / dt, 1), "ms_per_step": round(dt * 1e3 / n_steps, 3),
            "us_per_layer": round(dt * 1e6 / n_steps / n_layers, 2), "hbm_gbps": round(moved / dt / 1e9, 1),
            "frac_of_peak": round(moved / dt / 1e9 / HBM_PEAK_GBPS, 4), "resident_gb": round(resident / 1e9, 2),
            "unique_experts_mean": round(float(np.mean(uniq)), 2), "build_s": round(build_s, 1)}


def prefill_bench(torch, dev, n_tok: int, reps: int) -> dict:
    """One 120B-shape MoE layer over a prefill chunk of n_tok tokens with Zipf(1.1)-skewed routing.

    The workload is defined in bfloat16 (bf16 x bf16 products summed in float32, the down input rounded to
    bfloat16, as the reference's matmul_precision="bf16" path); the same layers are also timed with float32
    expert math (the down input as hi + lo bfloat16 planes), reported under "fp32".
    """
    import numpy as np

    from klcquant_amd import moe, synth

    workload = 3
    host = moe.synthetic_host_layer(workload, 0, HIDDEN, INTER, EXPERTS)
    x_host = moe.synthetic_hidden(workload, n_tok, HIDDEN)
    bias, target = synth.zipf_router_bias(x_host, host["router_weight"], TOPK, 1.1, 1000 * workload + 11)
    del host
    weights_l = [moe.MoELayerWeights.synthetic(workload, l, HIDDEN, INTER, EXPERTS, dev, bias) for l in range(2)]
    x = torch.from_numpy(x_host.view(np.int16)).view(torch.bfloat16).to(dev)
    out = torch.empty_like(x)
    ids = torch.empty((n_tok, TOPK), dtype=torch.int32, device=dev)

    def timed(precision):
        layers = [moe.MoELayer(w, TOPK, 7.0, precision) for w in weights_l]
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(7)] for _ in range(reps)]
        for row in evs:  # torch creates the HIP event on its first record
            for ev in row:
                ev.record()
        settle = time.perf_counter() + 0.15  # clocks ramp over the first tens of ms
        while time.perf_counter() < settle:
            layers[0].forward(x, out=out)
            torch.cuda.synchronize()
        # per-kernel times from an event pass; the layer time from a pass without events (an event
        # record between two kernels costs a few us)
        for r in range(reps):
            layers[r % 2].forward(x, out=out, ids=ids if r == 0 else None, events=evs[r])
        torch.cuda.synchronize()
        kern = np.array([[evs[r][i].elapsed_time(evs[r][i + 1]) for i in range(6)] for r in range(reps)]).mean(axis=0)
        t0 = time.perf_counter()
        for r in range(reps):
            layers[r % 2].forward(x, out=out)
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / reps
        return dt, kern

    dt, kern = timed("bf16")
    dt32, kern32 = timed("fp32")
    counts = np.bincount(ids.cpu().numpy().ravel(), minlength=EXPERTS)
    flop = n_tok * TOPK * (2 * 2 * INTER * HIDDEN + 2 * HIDDEN * INTER) + 2 * n_tok * HIDDEN * EXPERTS
    weights = int(np.count_nonzero(counts)) * (GATE_UP_EXPERT_BYTES + DOWN_EXPERT_BYTES)
    expert_ms = float(kern[3] + kern[4])
    bf16_peak = 2.5e15
    del weights_l
    torch.cuda.empty_cache()
    return {
        "workload": f"gpt-oss-120B-shape MoE layer, prefill of {n_tok} tokens in bf16, top-4 of 128, "
                    "Zipf(1.1) router bias",
        "precision": "bf16",
        "us_per_layer": round(dt * 1e6, 1), "tokens_per_s": round(n_tok / dt, 1),
        "kernel_us_mean": {k: round(float(v) * 1e3, 2) for k, v in zip(KERNELS, kern)},
        "flop": flop, "tflops": round(flop / dt / 1e12, 1),
        "mfma_util_bf16": round(flop / (expert_ms * 1e-3) / bf16_peak, 4),
        # the scaled FP4 MFMA is not used: its 128-term sums lose up to 1.6e-4 of sum|terms| (float32:
        # 4.6e-7), and with three FP8 activation planes 12 of 737280 expert outputs of a 256-token 120B-shape
        # expert still fail 1e-2 + 2e-2|ref| (tests/test_gpu_fp4_mfma.py)
        "scaled_fp4_mfma": {"used": False, "worst_block_err_over_sum_abs_terms": 1.641e-4,
                            "float32_sum_worst": 4.589e-7, "failing_outputs_3_fp8_planes": 12,
                            "profile": "profiles/scaled_fp4_mfma_accumulation_error.txt"},
        "weight_gbps": round(weights / (expert_ms * 1e-3) / 1e9, 1),
        "fp32": {"us_per_layer": round(dt32 * 1e6, 1), "tokens_per_s": round(n_tok / dt32, 1),
                 "kernel_us_mean": {k: round(float(v) * 1e3, 2) for k, v in zip(KERNELS, kern32)},
                 "mfma_util_bf16": round(flop / (float(kern32[3] + kern32[4]) * 1e-3) / bf16_peak, 4)},
        "expert_load": {"max": int(counts.max()), "mean": round(float(counts.mean()), 2),
                        "min": int(counts.min()), "max_over_mean": round(float(counts.max() / counts.mean()), 2),
                        "hottest_share": round(float(counts.max() / counts.sum()), 4),
                        "zipf_target_share": round(target, 4), "experts_touched": int(np.count_nonzero(counts)),
                        "top8": sorted((int(c) for c in counts), reverse=True)[:8]},
    }


def loader_bench(torch, dev, n_experts: int, rounds: int = 3) -> dict:
    """Expert-store misses of 120B-shape experts from a page-cache-resident shard.

    ``native``: Mxfp4ExpertStore.packed_expert (shard -> pinned staging ring ->
    pack kernel reading the staging over PCIe, asynchronous on the side
    stream).  ``safe_open_chain``: the
    per-miss chain the store replaces (safe_open slice -> pin_memory -> .to
    -> the same pack kernel), on the same slices.  The shard is fsync'ed
    before timing (no writeback under the reads); the two legs run in
    alternating order over ``rounds`` rounds (a fresh store each round) and
    the medians are reported.
    Expert 0 of every round is untimed (shard open, staging, allocator), and
    the packed matrices of the two legs are compared.
    """
    import statistics
    import tempfile

    import numpy as np
    from safetensors import safe_open
    from safetensors.torch import save_file

    from klcquant_amd import ops
    from klcquant_amd.mxfp4_expert import Mxfp4ExpertStore

    rng = np.random.default_rng(11)
    prefix = "model.layers.0.mlp.experts"
    shapes = {"gate_up_proj": (2 * INTER, HIDDEN // 32), "down_proj": (HIDDEN, INTER // 32)}
    tensors = {}
    for proj, (rows, groups) in shapes.items():
        tensors[f"{prefix}.{proj}_blocks"] = torch.from_numpy(
            rng.integers(0, 256, (n_experts, rows, groups, 16), dtype=np.uint8))
        tensors[f"{prefix}.{proj}_scales"] = torch.from_numpy(
            rng.integers(118, 125, (n_experts, rows, groups), dtype=np.uint8))
    with tempfile.TemporaryDirectory() as tmp:
        path = Path(tmp) / "model-00001-of-00001.safetensors"
        save_file(tensors, str(path))
        with open(path, "rb+") as fh:
            os.fsync(fh.fileno())
        (Path(tmp) / "model.safetensors.index.json").write_text(
            json.dumps({"weight_map": {name: path.name for name in tensors}}))
        del tensors
        side = torch.cuda.Stream(dev)

        def reference_chain(e, proj):
            with safe_open(str(path), framework="pt", device="cpu") as handle:
                b = handle.get_slice(f"{prefix}.{proj}_blocks")[e]
                s = handle.get_slice(f"{prefix}.{proj}_scales")[e]
            with torch.cuda.stream(side):
                b_dev = b.contiguous().pin_memory().to(dev, non_blocking=True)
                s_dev = s.contiguous().pin_memory().to(dev, non_blocking=True)
                packed = ops.mxfp4_pack(b_dev, s_dev)[0]
            side.synchronize()
            return packed

        times = {"native": [], "safe_open_chain": [], "copy": []}
        same = True
        for r in range(rounds):
            store = Mxfp4ExpertStore(tmp, tmp, dev, dtype=torch.bfloat16, cache_bytes=1 << 40)
            got = {}
            for label in (("native", "safe_open_chain") if r % 2 == 0 else ("safe_open_chain", "native")):
                got[label] = {}
                for e in range(n_experts):
                    if e == 1:
                        torch.cuda.synchronize()
                        t0 = time.perf_counter()
                    for proj in shapes:
                        got[label][(e, proj)] = (store.packed_expert(0, e, proj) if label == "native"
                                                 else reference_chain(e, proj))
                torch.cuda.synchronize()
                times[label].append(time.perf_counter() - t0)
            same = same and all(torch.equal(got["native"][k], got["safe_open_chain"][k]) for k in got["native"])
            # the shard -> device copy alone (gate_up blocks, 8.3 MB per expert)
            name = f"{prefix}.gate_up_proj_blocks"
            shard = store.index.shard(name)
            shard.copy_rows_to_device(name, 0, 1, dev, side)
            t0 = time.perf_counter()
            for e in range(1, n_experts):
                shard.copy_rows_to_device(name, e, 1, dev, side)
            times["copy"].append(time.perf_counter() - t0)
            del store, got, shard
        torch.cuda.empty_cache()
    med = {k: statistics.median(v) for k, v in times.items()}
    bytes_loaded = (n_experts - 1) * (GATE_UP_EXPERT_BYTES + DOWN_EXPERT_BYTES)
    copy_bytes = (n_experts - 1) * 2 * INTER * (HIDDEN // 32) * 16
    return {
        "experts_timed": n_experts - 1,
        "rounds": rounds,
        "bytes_per_expert": GATE_UP_EXPERT_BYTES + DOWN_EXPERT_BYTES,
        "native_us_per_expert": round(med["native"] * 1e6 / (n_experts - 1), 1),
        "native_gbps": round(bytes_loaded / med["native"] / 1e9, 2),
        "safe_open_chain_us_per_expert": round(med["safe_open_chain"] * 1e6 / (n_experts - 1), 1),
        "safe_open_chain_gbps": round(bytes_loaded / med["safe_open_chain"] / 1e9, 2),
        "copy_rows_to_device_gbps": round(copy_bytes / med["copy"] / 1e9, 2),
        "native_gbps_rounds": [round(bytes_loaded / t / 1e9, 2) for t in times["native"]],
        "safe_open_chain_gbps_rounds": [round(bytes_loaded / t / 1e9, 2) for t in times["safe_open_chain"]],
        "packed_equal": bool(same),
    }


def layer_tensor_bench(torch, dev, n_layers: int = 4, rounds: int = 3) -> dict:
    """The executor's per-layer dense tensors (120B shapes, bf16: attention
    projections and biases, sinks, norms, router, expert biases; 56 MB per
    layer) from a page-cache-resident shard to HBM.

    ``native``: LayerTensorLoader (open shard, one staged batch copy per
    shard).  ``safe_open_chain``: the executor's path
    (streamed_transformer_executor.py:318-370: safe_open per load,
    get_tensor, pin_memory().to(device), synchronize).  Layer 0 of each leg
    is untimed; legs alternate over ``rounds`` and the medians are reported;
    the tensors of both legs are compared.
    """
    import statistics
    import tempfile

    import numpy as np
    from safetensors import safe_open
    from safetensors.torch import save_file

    from klcquant_amd.layer_tensors import LayerTensorLoader, layer_tensor_names

    nq, nkv, d = 64, 8, 64
    shapes = {
        "input_layernorm.weight": (HIDDEN,), "self_attn.o_proj.bias": (HIDDEN,),
        "self_attn.o_proj.weight": (HIDDEN, nq * d), "self_attn.q_proj.bias": (nq * d,),
        "self_attn.k_proj.bias": (nkv * d,), "self_attn.v_proj.bias": (nkv * d,),
        "self_attn.q_proj.weight": (nq * d, HIDDEN), "self_attn.k_proj.weight": (nkv * d, HIDDEN),
        "self_attn.v_proj.weight": (nkv * d, HIDDEN), "self_attn.sinks": (nq,), "mlp.router.bias": (EXPERTS,),
        "mlp.router.weight": (EXPERTS, HIDDEN), "mlp.experts.gate_up_proj_bias": (EXPERTS, 2 * INTER),
        "mlp.experts.down_proj_bias": (EXPERTS, HIDDEN), "post_attention_layernorm.weight": (HIDDEN,),
    }
    rng = np.random.default_rng(12)
    tensors = {}
    for layer in range(n_layers):
        for suffix, shape in shapes.items():
            bits = rng.integers(0, 1 << 16, shape, dtype=np.uint16) & 0xBFFF  # finite bf16 patterns
            tensors[f"model.layers.{layer}.{suffix}"] = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
    layer_bytes_ = sum(int(np.prod(s)) * 2 for s in shapes.values())
    with tempfile.TemporaryDirectory() as tmp:
        path = Path(tmp) / "model-00001-of-00001.safetensors"
        save_file(tensors, str(path))
        with open(path, "rb+") as fh:
            os.fsync(fh.fileno())
        (Path(tmp) / "model.safetensors.index.json").write_text(
            json.dumps({"weight_map": {name: path.name for name in tensors}}))
        del tensors

        def reference_chain(layer):
            out = {}
            with safe_open(str(path), framework="pt", device="cpu") as handle:
                for name in layer_tensor_names(layer):
                    t = handle.get_tensor(name).to(torch.bfloat16)
                    out[name] = t.pin_memory().to(dev, non_blocking=True)
            torch.cuda.synchronize()
            return out

        times = {"native": [], "safe_open_chain": []}
        same = True
        for r in range(rounds):
            loader = LayerTensorLoader(tmp, dev, pin_layer_tensors=False)
            got = {}
            for label in (("native", "safe_open_chain") if r % 2 == 0 else ("safe_open_chain", "native")):
                got[label] = []
                for layer in range(n_layers):
                    if layer == 1:
                        torch.cuda.synchronize()
                        t0 = time.perf_counter()
                    got[label].append(loader.load(layer) if label == "native" else reference_chain(layer))
                torch.cuda.synchronize()
                times[label].append(time.perf_counter() - t0)
            same = same and all(torch.equal(a[n], b[n]) for a, b in zip(got["native"], got["safe_open_chain"])
                                for n in a)
            del loader, got
        torch.cuda.empty_cache()
    # the link's own rate for comparison: one pinned 64 MiB buffer -> HBM
    host = torch.empty(64 << 20, dtype=torch.uint8, pin_memory=True)
    devbuf = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    devbuf.copy_(host, non_blocking=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(5):
        devbuf.copy_(host, non_blocking=True)
    torch.cuda.synchronize()
    h2d = 5 * (64 << 20) / (time.perf_counter() - t0) / 1e9
    del host, devbuf
    med = {k: statistics.median(v) for k, v in times.items()}
    timed = (n_layers - 1) * layer_bytes_
    return {
        "layers_timed": n_layers - 1,
        "rounds": rounds,
        "bytes_per_layer": layer_bytes_,
        "native_us_per_layer": round(med["native"] * 1e6 / (n_layers - 1), 1),
        "native_gbps": round(timed / med["native"] / 1e9, 2),
        "safe_open_chain_us_per_layer": round(med["safe_open_chain"] * 1e6 / (n_layers - 1), 1),
        "safe_open_chain_gbps": round(timed / med["safe_open_chain"] / 1e9, 2),
        "pinned_h2d_gbps": round(h2d, 2),
        "tensors_equal": bool(same),
    }


def route_api_bench(torch, dev, weights, calls: int, precision: str) -> dict:
    """The drop-in call itself: StreamedMoERouter.route() on one token per call (how the reference's
    executor routes), resident store, with its read-back and RouterStats bookkeeping; median wall time
    per call, next to one klc_moe_layer call plus a host synchronisation on the same token."""
    import numpy as np

    from klcquant_amd import moe
    from klcquant_amd.mxfp4_expert import ResidentExpertStore
    from klcquant_amd.streamed_moe_router import StreamedMoERouter

    p = "model.layers.0.mlp"
    tensors = {f"{p}.router.weight": weights.router_weight, f"{p}.router.bias": weights.router_bias,
               f"{p}.experts.gate_up_proj_bias": weights.gate_up_bias,
               f"{p}.experts.down_proj_bias": weights.down_bias}
    store = ResidentExpertStore({0: weights})
    router = StreamedMoERouter(TOPK, 7.0, matmul_precision=precision)
    layer = moe.MoELayer(weights, TOPK, 7.0, precision)
    xs = [torch.from_numpy(moe.synthetic_hidden(WORKLOAD, 1, HIDDEN, step=s).view(np.int16)).view(torch.bfloat16)
          .to(dev) for s in range(8)]

    def timed(fn) -> float:
        for s in range(20):
            fn(s)
        torch.cuda.synchronize()
        t = []
        for s in range(calls):
            t0 = time.perf_counter()
            fn(s)
            t.append(time.perf_counter() - t0)
        return float(np.median(t)) * 1e6

    route_us = timed(lambda s: router.route(0, xs[s % 8][0], tensors, store, position=s))

    def layer_sync(s):
        layer.forward(xs[s % 8])
        torch.cuda.synchronize()

    return {"workload": "StreamedMoERouter.route(), one token per call, resident 120B-shape layer, median wall time",
            "route_us_per_call": round(route_us, 1), "layer_and_sync_us_per_call": round(timed(layer_sync), 1),
            "calls": calls}


def lm_head_bench(torch, dev, reps: int = 50) -> dict:
    """gpt-oss lm_head (201,088 x 2880 bf16, resident): one logits pass plus
    the greedy token, against the executor's chunked float32 matmul with a
    host copy per 4096-row chunk (streamed_transformer_executor.py:177-191)."""
    from klcquant_amd.lm_head import LmHead

    vocab = 201088
    g = torch.Generator(device=dev).manual_seed(17)
    w = (torch.randn((vocab, HIDDEN), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    x = torch.randn(HIDDEN, generator=g, device=dev)
    head = LmHead(w)
    out, token = head.logits_device(x)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        head.logits_device(x, out=out)
    end.record()
    end.synchronize()
    us = start.elapsed_time(end) * 1e3 / reps
    t0 = time.perf_counter()
    for _ in range(5):
        tok = head.greedy_token(x)
    greedy_us = (time.perf_counter() - t0) * 1e6 / 5

    def reference():
        parts = []
        for s in range(0, vocab, 4096):
            parts.append(torch.matmul(w[s:s + 4096].float(), x.float()).detach().cpu())
        logits = torch.cat(parts)
        return int(torch.argmax(torch.nan_to_num(logits, nan=-1e9, posinf=1e9, neginf=-1e9)).item())

    reference()
    t0 = time.perf_counter()
    for _ in range(3):
        ref_tok = reference()
    ref_us = (time.perf_counter() - t0) * 1e6 / 3
    nbytes = vocab * HIDDEN * 2
    del w, head
    torch.cuda.empty_cache()
    return {
        "workload": "gpt-oss lm_head 201088 x 2880 bf16 resident, logits + greedy token",
        "us": round(us, 2),
        "gbps": round(nbytes / (us * 1e-6) / 1e9, 1),
        "frac_of_peak": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
        "greedy_token_us_host": round(greedy_us, 1),
        "reference_chunked_us_host": round(ref_us, 1),
        "same_token_as_reference": bool(tok == ref_tok),
    }


def attention_bench(torch, dev, context: int = 4096, reps: int = 100) -> dict:
    """gpt-oss decode attention core (64 query / 8 KV heads, head_dim 64, fp16
    KV ring): RoPE + append + scores / softmax with sinks / value sum, at a
    full-attention context and at the 128-token sliding window, against the
    reference's per-step stack + repeat_interleave + einsum + softmax
    (streamed_attention.py:120-141, kv_cache_manager.py:50-56) on the same
    cache contents."""
    import ctypes

    from klcquant_amd import _native
    from klcquant_amd.attention import AttentionConfig, rope_cos_sin

    cfg = AttentionConfig(hidden_size=HIDDEN, num_heads=64, num_kv_heads=8, head_dim=64, rope_factor=32.0)
    nh, nkv, d, cap = 64, 8, 64, 8192
    g = torch.Generator(device=dev).manual_seed(23)
    kc = torch.randn((cap, nkv, d), generator=g, device=dev).to(torch.float16)
    vc = torch.randn((cap, nkv, d), generator=g, device=dev).to(torch.float16)
    q = torch.randn((nh, d), generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn((nkv, d), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((nkv, d), generator=g, device=dev).to(torch.bfloat16)
    sinks = torch.randn(nh, generator=g, device=dev).to(torch.bfloat16)
    cos, sin = rope_cos_sin(cfg, context, dev, torch.bfloat16)
    q_rot, k_rot = torch.empty_like(q), torch.empty_like(k)
    ctx = torch.empty((nh, d), dtype=torch.bfloat16, device=dev)
    P = ctypes.c_void_p
    stream = P(torch.cuda.current_stream(dev).cuda_stream)
    ws = torch.empty(_native.call("klc_attn_workspace_bytes", nh, d, cap), dtype=torch.uint8, device=dev)

    def step(count):
        _native.call("klc_rope_append", P(q.data_ptr()), P(k.data_ptr()), P(v.data_ptr()), P(cos.data_ptr()),
                     P(sin.data_ptr()), P(q_rot.data_ptr()), P(k_rot.data_ptr()), P(kc.data_ptr()), P(vc.data_ptr()),
                     count - 1, cap, nh, nkv, d, 1, stream)
        _native.call("klc_attn_decode", P(q_rot.data_ptr()), P(kc.data_ptr()), P(vc.data_ptr()), P(sinks.data_ptr()),
                     cap, 0, count, nh, nkv, d, 1, P(ws.data_ptr()), ws.numel(), P(ctx.data_ptr()), stream)

    out = {"workload": f"gpt-oss decode attention core, 64/8 heads x 64, fp16 KV ring, sinks; context {context} and window 128"}
    for label, count in (("full", context), ("window128", 128)):
        step(count)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            step(count)
        end.record()
        end.synchronize()
        us = start.elapsed_time(end) * 1e3 / reps
        kv_bytes = 2 * count * nkv * d * 2
        out[f"{label}_us"] = round(us, 2)
        out[f"{label}_kv_gbps"] = round(kv_bytes / (us * 1e-6) / 1e9, 1)
    # the reference's per-step work on the same cache: a list of per-token tensors stacked every step
    keys = [kc[i] for i in range(context)]
    values = [vc[i] for i in range(context)]

    def reference():
        kk, vv = torch.stack(keys, 0), torch.stack(values, 0)
        kh = kk.repeat_interleave(nh // nkv, dim=1).transpose(0, 1)
        vh = vv.repeat_interleave(nh // nkv, dim=1).transpose(0, 1)
        scores = torch.einsum("hd,htd->ht", q.float(), kh.float()) / 8.0
        comb = torch.cat([scores, sinks.float().reshape(-1, 1)], dim=-1)
        comb = comb - comb.max(dim=-1, keepdim=True).values
        probs = torch.softmax(comb, dim=-1)[..., :-1].to(vh.dtype)
        return torch.einsum("ht,htd->hd", probs, vh.contiguous())

    reference()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(10):
        reference()
    torch.cuda.synchronize()
    out["reference_full_us_host"] = round((time.perf_counter() - t0) * 1e6 / 10, 1)
    del kc, vc, ws, keys, values
    torch.cuda.empty_cache()
    return out


def _cpu_layer(workload: int, n_exp: int, router_bias=None):
    """torch_ref.Layer with the seeded router and biases of (workload, layer 0); experts are added per sample."""
    import numpy as np
    import torch

    from klcquant_amd import synth
    from oracle import torch_ref

    def t_bf16(bits):
        return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16)).view(torch.bfloat16)

    seed = {n: synth.tensor_seed(workload, n, 0) for n in synth.TENSOR_IDS}
    rw = synth.random_normal_bf16(seed["router_weight"], n_exp * HIDDEN, 0.0, 0.02).reshape(n_exp, HIDDEN)
    rb = synth.random_normal_bf16(seed["router_bias"], n_exp, 0.0, 0.01) if router_bias is None else router_bias
    gub = synth.random_normal_bf16(seed["gate_up_bias"], n_exp * 2 * INTER, 0.0, 0.01).reshape(n_exp, -1)
    db = synth.random_normal_bf16(seed["down_bias"], n_exp * HIDDEN, 0.0, 0.01).reshape(n_exp, -1)
    return torch_ref.Layer(t_bf16(rw), t_bf16(rb), t_bf16(gub), t_bf16(db), {}, TOPK), seed, t_bf16


def _cpu_route_sample(layer, seed, xs, warmups: int, precision: str = "fp32") -> dict:
    """Single-token route() calls over xs: cold (every call dequantizes its experts) and warm (the
    dequantized matrices cached); medians over the calls after ``warmups``; ``precision`` is the
    reference's matmul_precision."""
    import statistics

    import torch

    from klcquant_amd import synth

    for e in sorted({e for x in xs for e in layer.select(x)}):  # checkpoint tensors as the store reads them
        parts = (synth.mxfp4_expert_slice(seed["gate_up_blocks"], seed["gate_up_scales"], e, 2 * INTER, HIDDEN)
                 + synth.mxfp4_expert_slice(seed["down_blocks"], seed["down_scales"], e, HIDDEN, INTER))
        layer.experts[e] = tuple(torch.from_numpy(p) for p in parts)

    def timed(warm: bool) -> list[float]:
        out = []
        for i, x in enumerate(xs):
            t0 = time.perf_counter()
            layer.route(x, warm, precision)
            if i >= warmups:
                out.append(time.perf_counter() - t0)
        return out

    cold = timed(False)
    for x in xs:  # fill the warm store with the sample's experts
        layer.route(x, True, precision)
    warm = timed(True)
    return {"warm_us_per_token": round(statistics.median(warm) * 1e6, 1),
            "cold_us_per_token": round(statistics.median(cold) * 1e6, 1),
            "tokens_timed": len(xs) - warmups, "unique_experts": len(layer.experts)}


def cpu_baseline(n_tokens: int, warmups: int = 2) -> dict:
    """The reference path restated in torch CPU ops (oracle/torch_ref.py), on the host cores.

    The reference routes one token per route() call (streamed_moe_router.py:257-329), so every decode
    and prefill configuration is a sequence of single-token calls; each is timed on a bounded sample and
    the totals for the full configuration are extrapolated from the per-call medians (labelled so):
    * 0: the 20B-shape layer (E = 32), single-token calls, cold and warm;
    * 1: dequantize_mxfp4_matrix over 8 of the 128 down_proj matrices, scaled to 128;
    * 2: the 120B-shape layer (E = 128), single-token calls (B = 8 and 64 are B calls per step);
    * 3: single-token calls of the Zipf(1.1)-biased 2048-token prefill layer, scaled to 2048 tokens;
    * 4: one stack layer per token = rms_norm + route() + residual, scaled to 64 tokens x 36 layers.
    Cold: cache_bytes = 0, every call dequantizes its 4 experts from MXFP4 (the miss path with the
    checkpoint in RAM); warm: the dequantized matrices are cached (the hit path with its .float()
    copies).  ``value`` is configuration 2's warm per-token time."""
    import statistics

    import numpy as np
    import torch

    from klcquant_amd import moe, synth
    from oracle import torch_ref

    n = warmups + n_tokens
    configs = {}
    # 0: 20B shape, E = 32
    layer, seed, _ = _cpu_layer(0, 32)
    xs = [torch.from_numpy(r.view(np.int16)).view(torch.bfloat16)
          for r in moe.synthetic_hidden(0, n, HIDDEN, step=12345)]
    configs["0"] = {"workload": "gpt-oss-20B-shape MoE layer (E = 32, top-4), single-token route() calls",
                    **_cpu_route_sample(layer, seed, xs, warmups)}
    del layer
    # 2: 120B shape, E = 128
    layer, seed, t_bf16 = _cpu_layer(WORKLOAD, EXPERTS)
    xs = [t_bf16(row) for row in moe.synthetic_hidden(WORKLOAD, n, HIDDEN, step=12345)]
    c2 = _cpu_route_sample(layer, seed, xs, warmups)
    configs["2"] = {"workload": "gpt-oss-120B-shape MoE layer (E = 128, top-4), single-token route() calls",
                    **c2,
                    "us_per_step_extrapolated": {str(b): round(b * c2["warm_us_per_token"], 1) for b in (1, 8, 64)}}
    # 4: rms_norm + residual of a 64-row batch, measured; route() per token from configuration 2
    h = t_bf16(moe.synthetic_hidden(4, 64, HIDDEN))
    w_norm = t_bf16(moe.synthetic_norm_weight(4, 0, HIDDEN))
    moe_out = t_bf16(moe.synthetic_hidden(5, 64, HIDDEN))

    def norm_residual():
        x = h.clone()
        normed = x * torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + 1e-5).to(x.dtype) * w_norm
        x += moe_out
        return normed

    for _ in range(3):
        norm_residual()
    t = []
    for _ in range(20):
        t0 = time.perf_counter()
        norm_residual()
        t.append(time.perf_counter() - t0)
    nr_us = statistics.median(t) * 1e6
    layer_us = 64 * c2["warm_us_per_token"] + nr_us
    configs["4"] = {"workload": "36-layer MoE-only stack, 64 sequences: rms_norm -> route() per token -> residual",
                    "extrapolated": "36 layers x (64 warm single-token route() calls of configuration 2 + the "
                                    "measured rms_norm and residual of the 64-row batch)",
                    "rms_norm_residual_us_per_batch": round(nr_us, 1),
                    "ms_per_step": round(36 * layer_us / 1e3, 1),
                    "tokens_per_s": round(64 / (36 * layer_us * 1e-6), 2)}
    del layer
    # 1: dequantize_mxfp4_matrix over 128 down_proj matrices (8 timed)
    d = []
    for e in range(10):
        b, sc = synth.mxfp4_expert_slice(synth.tensor_seed(1, "down_blocks"), synth.tensor_seed(1, "down_scales"),
                                         e, HIDDEN, INTER)
        bt, st = torch.from_numpy(b), torch.from_numpy(sc)
        t0 = time.perf_counter()
        torch_ref.dequantize(bt, st, torch.bfloat16)
        if e >= 2:
            d.append(time.perf_counter() - t0)
    per = statistics.median(d)
    moved = EXPERTS * HIDDEN * (INTER // 32) * 17 + EXPERTS * HIDDEN * INTER * 2
    configs["1"] = {"workload": "dequantize_mxfp4_matrix, 128 x down_proj [2880, 90, 16] -> bf16 [2880, 2880]",
                    "matrices_timed": len(d), "us_per_matrix": round(per * 1e6, 1),
                    "s_total_extrapolated": round(per * EXPERTS, 3),
                    "gbps": round(moved / (per * EXPERTS) / 1e9, 2)}
    # 3: the Zipf(1.1) prefill layer, single-token calls (6 timed)
    x_host = moe.synthetic_hidden(3, 2048, HIDDEN)
    rw = synth.random_normal_bf16(synth.tensor_seed(3, "router_weight"), EXPERTS * HIDDEN, 0.0, 0.02)
    bias, _ = synth.zipf_router_bias(x_host, rw.reshape(EXPERTS, HIDDEN), TOPK, 1.1, 1000 * 3 + 11)
    layer, seed, _ = _cpu_layer(3, EXPERTS, bias)
    xs = [t_bf16(row) for row in x_host[:warmups + 6]]
    c3 = _cpu_route_sample(layer, seed, xs, warmups, "bf16")
    configs["3"] = {"workload": "gpt-oss-120B-shape layer with Zipf(1.1) router bias, 2048 prefill tokens as "
                                "single-token route() calls, matmul_precision bf16", **c3,
                    "extrapolated": "2048 x the per-call medians",
                    "s_total_warm": round(2048 * c3["warm_us_per_token"] / 1e6, 2),
                    "s_total_cold": round(2048 * c3["cold_us_per_token"] / 1e6, 2),
                    "tokens_per_s_warm": round(1e6 / c3["warm_us_per_token"], 2)}
    del layer
    return {
        "value": c2["warm_us_per_token"],
        "unit": "us/token",
        "cores": int(torch.get_num_threads()),
        "kind": "port",
        "sample": (f"median of {n_tokens} single-token route() calls after {warmups} warm-ups (B = 1: the reference "
                   "routes one token per call), the 120B-shape layer, the reference's torch CPU ops in its "
                   "float32 matmul mode: warm = dequantized experts cached (the hit path); cold = every call "
                   "dequantizes its 4 experts from MXFP4 (cache_bytes = 0); configs holds every configuration"),
        "warm_us_per_token": c2["warm_us_per_token"],
        "cold_us_per_token": c2["cold_us_per_token"],
        "unique_experts": c2["unique_experts"],
        "configs": {k: configs[k] for k in sorted(configs)},
    }


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); this build has no multi-GPU path",
              file=sys.stderr)
        return 2
    import numpy as np
    import torch

    from klcquant_amd import _native, moe

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    _native.load()
    dev = torch.device("cuda:0")
    if args.copy_calibration:
        copy_calibration(torch, dev)
        return 0
    batches = [int(b) for b in args.batches.split(",") if b]
    print(f"[bench] building {args.layers} layers of {EXPERTS} experts on {torch.cuda.get_device_name(0)}",
          file=sys.stderr, flush=True)
    layers = [moe.MoELayer(moe.MoELayerWeights.synthetic(WORKLOAD, l, HIDDEN, INTER, EXPERTS, dev), TOPK, 7.0,
                           args.precision) for l in range(args.layers)]
    torch.cuda.synchronize()

    per_batch = []
    for n_tok in batches:
        xs = [torch.from_numpy(moe.synthetic_hidden(WORKLOAD, n_tok, HIDDEN, step=s).view(np.int16))
              .view(torch.bfloat16).to(dev) for s in range(args.inputs)]
        out = torch.empty((n_tok, HIDDEN), dtype=torch.bfloat16, device=dev)
        # the steps cycle through n_pairs distinct (layer, input batch) pairs
        n_pairs = math.lcm(args.layers, args.inputs)
        ids = torch.empty((n_pairs, n_tok, TOPK), dtype=torch.int32, device=dev)
        graphs = None
        if args.graph and _native.load().klc_moe_workspace_bytes(n_tok, HIDDEN, INTER, EXPERTS, TOPK) <= \
                STATIC_SCRATCH_BYTES:
            # one HIP graph per (layer, input) pair: a step is one graph launch from the host
            graphs = [layers[j % args.layers].capture_graph(xs[j % args.inputs], out, ids=ids[j])
                      for j in range(n_pairs)]

        def step(s: int) -> None:
            if graphs is not None:
                graphs[s % n_pairs].replay()
            else:
                layers[s % args.layers].forward(xs[s % args.inputs], out=out, ids=ids[s % n_pairs])

        # settle: the GPU reaches its working clocks only after ~20-30 ms of sustained load (a cold
        # 20-step run of B = 64 measures ~7 % slow), so every batch size first runs at least
        # SETTLE_MS of untimed steps
        t_settle = time.perf_counter()
        s = 0
        while (time.perf_counter() - t_settle) * 1e3 < SETTLE_MS or s < 4:
            step(s)
            s += 1
            if s % 16 == 0:
                torch.cuda.synchronize()
        torch.cuda.synchronize()
        # per-kernel times: the same steps with events around each kernel
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(_native.LAYER_EVENTS)] for _ in range(args.steps)]
        for row in evs:
            for e in row:
                e.record()
        torch.cuda.synchronize()
        for s in range(args.steps):
            layers[s % args.layers].forward(xs[s % args.inputs], out=out, events=evs[s])
        torch.cuda.synchronize()
        for s in range(args.warmup):
            step(s)
        torch.cuda.synchronize()
        # the headline timing: W untimed steps, then K timed steps, no events between kernels
        t0 = time.perf_counter()
        for s in range(args.steps):
            step(s)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        kern_ms = np.array([[evs[s][i].elapsed_time(evs[s][i + 1]) for i in range(len(KERNELS))]
                            for s in range(args.steps)])
        ids_np = ids.cpu().numpy()
        uniq = np.array([len(np.unique(ids_np[s % n_pairs])) for s in range(args.steps)])
        ms_step = dt * 1e3 / args.steps
        bytes_total = float(sum(layer_bytes(int(u), n_tok) for u in uniq))
        gu_bytes = float(sum(gate_up_bytes(int(u), n_tok) for u in uniq))
        path = layers[0].layer_path(n_tok)
        gu_ms = float(kern_ms[:, 3].sum())
        rec = {
            "batch": n_tok,
            "us_per_token": round(ms_step * 1e3 / n_tok, 3),
            "us_per_step": round(ms_step * 1e3, 3),
            "tokens_per_s": round(n_tok / (ms_step * 1e-3), 1),
            "unique_experts_mean": round(float(uniq.mean()), 2),
            "layer_hbm_gbps": round(bytes_total / (dt * 1e9 / 1.0) / 1.0, 1),
            "layer_frac_of_peak": round(bytes_total / dt / 1e9 / HBM_PEAK_GBPS, 4),
            "layer_path": path,
            "kernel_us_mean": kernel_breakdown(kern_ms.mean(axis=0) * 1e3, n_tok, path),
            # the one-launch layer has no separate gate_up kernel to time
            "gate_up_gbps": round(gu_bytes / (gu_ms * 1e-3) / 1e9, 1) if path != "fused" else None,
            "gate_up_bytes_per_launch": round(gu_bytes / args.steps),
            "hip_graph": graphs is not None,
        }
        per_batch.append(rec)
        print(f"[bench] B={n_tok}: {rec['us_per_step']} us/step, {rec['us_per_token']} us/token, "
              f"{rec['layer_hbm_gbps']} GB/s layer, gate_up {rec['gate_up_gbps']} GB/s, "
              f"kernels {rec['kernel_us_mean']}", file=sys.stderr, flush=True)

    head = next((r for r in per_batch if r["batch"] == args.headline_batch), per_batch[-1])
    gu_achieved = head["gate_up_gbps"]
    result = {
        "metric": "MoE layer us/token & HBM GB/s (% of peak), 120B shape, batch 1-64",
        "value": head["us_per_token"],
        "unit": "us/token",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["us_per_step"] / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "gpt-oss-120B-shape MoE layer decode: H=I=2880, 128 MXFP4 experts, top-4, fp32 expert math",
            "global_batch": head["batch"],
            "batches": batches,
            "layers_rotated": args.layers,
            "precision": args.precision,
            "parallelism": "single GPU",
        },
        "hbm_gbps": head["layer_hbm_gbps"],
        "hbm_frac_of_peak": head["layer_frac_of_peak"],
        "per_batch": per_batch,
        "roofline": {
            "bound": "hbm",
            "kernel": "moe_gemv_mfma_kernel<gate_up>",
            "achieved": gu_achieved,
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(gu_achieved / HBM_PEAK_GBPS, 4) if gu_achieved is not None else None,
            "traffic": measured_traffic() if head["batch"] == 64 and args.precision == "fp32" else None,
            "algorithmic_bytes_per_launch": round(head["gate_up_bytes_per_launch"]),
        },
    }
    if not args.skip_config0:
        result["config0"] = config0_bench(torch, dev, args.steps, args.warmup, args.precision)
        print(f"[bench] config0: {result['config0']}", file=sys.stderr, flush=True)
    if args.route_calls > 0:
        result["route_api"] = route_api_bench(torch, dev, layers[0].w, args.route_calls, args.precision)
        print(f"[bench] route(): {result['route_api']}", file=sys.stderr, flush=True)
    if args.prefill_tokens > 0:
        result["prefill"] = prefill_bench(torch, dev, args.prefill_tokens, 20)
        print(f"[bench] prefill: {result['prefill']}", file=sys.stderr, flush=True)
    if args.stack_layers > 0:
        del layers
        torch.cuda.empty_cache()
        result["stack"] = stack_bench(torch, dev, args.stack_layers, 64, args.stack_steps, args.precision)
        print(f"[bench] stack: {result['stack']}", file=sys.stderr, flush=True)
    if not args.skip_attention:
        result["attention"] = attention_bench(torch, dev)
        print(f"[bench] attention: {result['attention']}", file=sys.stderr, flush=True)
    if not args.skip_lm_head:
        result["lm_head"] = lm_head_bench(torch, dev)
        print(f"[bench] lm_head: {result['lm_head']}", file=sys.stderr, flush=True)
    if args.loader_experts > 1:
        result["loader"] = loader_bench(torch, dev, args.loader_experts)
        result["loader"]["layer_tensors"] = layer_tensor_bench(torch, dev)
        print(f"[bench] loader: {result['loader']}", file=sys.stderr, flush=True)
    if not args.skip_dequant:
        result["dequant"] = dequant_bench(torch, dev)
        print(f"[bench] dequant: {result['dequant']}", file=sys.stderr, flush=True)
    if args.cpu_tokens > 0:
        print(f"[bench] CPU baseline: {args.cpu_tokens} tokens through the torch CPU restatement", file=sys.stderr,
              flush=True)
        result["cpu_baseline"] = cpu_baseline(args.cpu_tokens)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
