"""One MoE layer with every expert resident in HBM in the packed row-tile layout.

This is the batched form of the reference's per-token path
(streamed_moe_router.py:257-315 and :483-522 for each row of ``hidden``):
router logits -> top-k/softmax -> expert-sorted dispatch -> gate_up + SwiGLU
-> down -> weighted combine, enqueued on the current stream with no host
synchronisation.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _native as nat
from . import ops, synth


@dataclass
class MoELayerWeights:
    """Device-resident weights of one MoE layer (E experts, hidden H, intermediate I)."""

    router_weight: torch.Tensor  # [E, H] bf16
    router_bias: torch.Tensor  # [E] bf16
    gate_up: torch.Tensor  # [E, packed bytes of a [2I rows, H/32 groups] matrix] uint8
    gate_up_bias: torch.Tensor  # [E, 2I] bf16
    down: torch.Tensor  # [E, packed bytes of a [H rows, I/32 groups] matrix] uint8
    down_bias: torch.Tensor  # [E, H] bf16
    hidden: int
    inter: int
    gate_up_table: torch.Tensor = field(init=False)
    down_table: torch.Tensor = field(init=False)

    def __post_init__(self) -> None:
        dev = self.router_weight.device
        self.gate_up_table = ops.pointer_table(self.gate_up, dev)
        self.down_table = ops.pointer_table(self.down, dev)

    @property
    def n_experts(self) -> int:
        return int(self.router_weight.shape[0])

    @property
    def device(self) -> torch.device:
        return self.router_weight.device

    def expert_bytes(self) -> int:
        """Packed bytes of one expert (gate_up + down, blocks + scales)."""
        return int(self.gate_up.shape[1] + self.down.shape[1])

    @classmethod
    def from_checkpoint(cls, router_weight, router_bias, gate_up_blocks, gate_up_scales, gate_up_bias, down_blocks,
                        down_scales, down_bias, device: torch.device | str = "cuda") -> "MoELayerWeights":
        """Packs checkpoint-layout tensors (``[E, out, G, 16]`` / ``[E, out, G]``)."""
        dev = torch.device(device)

        def to_dev(t, dtype):
            return torch.as_tensor(t).to(device=dev, dtype=dtype).contiguous()

        e = router_weight.shape[0]
        hidden = router_weight.shape[1]
        inter = down_blocks.shape[2] * 32
        if tuple(gate_up_blocks.shape[:2]) != (e, 2 * inter) or gate_up_blocks.shape[2] * 32 != hidden:
            raise ValueError(f"gate_up blocks shape {tuple(gate_up_blocks.shape)} does not match E={e} H={hidden} I={inter}")
        if tuple(down_blocks.shape[:2]) != (e, hidden):
            raise ValueError(f"down blocks shape {tuple(down_blocks.shape)} does not match E={e} H={hidden}")
        gu = ops.mxfp4_pack(to_dev(gate_up_blocks, torch.uint8), to_dev(gate_up_scales, torch.uint8))
        dn = ops.mxfp4_pack(to_dev(down_blocks, torch.uint8), to_dev(down_scales, torch.uint8))
        return cls(to_dev(router_weight, torch.bfloat16), to_dev(router_bias, torch.bfloat16), gu,
                   to_dev(gate_up_bias, torch.bfloat16), dn, to_dev(down_bias, torch.bfloat16), hidden, inter)

    @classmethod
    def synthetic(cls, workload: int, layer: int, hidden: int, inter: int, n_experts: int,
                  device: torch.device | str = "cuda", router_bias_override: np.ndarray | None = None
                  ) -> "MoELayerWeights":
        """Seeded synthetic layer, bit-identical to :func:`synthetic_host_layer`.

        MXFP4 codes and scales are generated on the GPU (klc_synth_fill) in
        checkpoint layout and packed; the normal-distributed tensors are small
        and generated on the host.
        """
        dev = torch.device(device)
        seeds = {name: synth.tensor_seed(workload, name, layer) for name in synth.TENSOR_IDS}
        rw = synth.random_normal_bf16(seeds["router_weight"], n_experts * hidden, 0.0, 0.02).reshape(n_experts, hidden)
        rb = synth.random_normal_bf16(seeds["router_bias"], n_experts, 0.0, 0.01)
        if router_bias_override is not None:
            rb = np.asarray(router_bias_override, dtype=np.uint16)
        gub = synth.random_normal_bf16(seeds["gate_up_bias"], n_experts * 2 * inter, 0.0, 0.01).reshape(n_experts, -1)
        db = synth.random_normal_bf16(seeds["down_bias"], n_experts * hidden, 0.0, 0.01).reshape(n_experts, -1)

        def bf16_dev(a):
            return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(dev)

        def packed(rows, in_dim, seed_b, seed_s):
            groups = in_dim // 32
            blocks = torch.empty((n_experts, rows, groups, 16), dtype=torch.uint8, device=dev)
            scales = torch.empty((n_experts, rows, groups), dtype=torch.uint8, device=dev)
            ops.synth_fill(blocks, seed_b, 0)
            ops.synth_fill(scales, seed_s, 1, 118, 124)
            out = ops.mxfp4_pack(blocks, scales)
            del blocks, scales  # the checkpoint-layout staging copy is not kept
            return out

        gu = packed(2 * inter, hidden, seeds["gate_up_blocks"], seeds["gate_up_scales"])
        dn = packed(hidden, inter, seeds["down_blocks"], seeds["down_scales"])
        return cls(bf16_dev(rw), bf16_dev(rb), gu, bf16_dev(gub), dn, bf16_dev(db), hidden, inter)


def synthetic_host_layer(workload: int, layer: int, hidden: int, inter: int, n_experts: int,
                         router_bias_override: np.ndarray | None = None) -> dict:
    """The same seeded layer as :meth:`MoELayerWeights.synthetic`, as numpy arrays in checkpoint layout."""
    seeds = {name: synth.tensor_seed(workload, name, layer) for name in synth.TENSOR_IDS}
    rb = synth.random_normal_bf16(seeds["router_bias"], n_experts, 0.0, 0.01)
    if router_bias_override is not None:
        rb = np.asarray(router_bias_override, dtype=np.uint16)
    gub, gus = synth.mxfp4_expert_tensors(seeds["gate_up_blocks"], seeds["gate_up_scales"], n_experts, 2 * inter, hidden)
    db, ds = synth.mxfp4_expert_tensors(seeds["down_blocks"], seeds["down_scales"], n_experts, hidden, inter)
    return {
        "router_weight": synth.random_normal_bf16(seeds["router_weight"], n_experts * hidden, 0.0, 0.02).reshape(n_experts, hidden),
        "router_bias": rb,
        "gate_up_blocks": gub,
        "gate_up_scales": gus,
        "gate_up_bias": synth.random_normal_bf16(seeds["gate_up_bias"], n_experts * 2 * inter, 0.0, 0.01).reshape(n_experts, -1),
        "down_blocks": db,
        "down_scales": ds,
        "down_bias": synth.random_normal_bf16(seeds["down_bias"], n_experts * hidden, 0.0, 0.01).reshape(n_experts, -1),
    }


def synthetic_hidden(workload: int, n_tokens: int, hidden: int, step: int = 0) -> np.ndarray:
    """bf16 bit patterns ``[n_tokens, hidden]`` of N(0, 1) activations."""
    seed = synth.tensor_seed(workload, "hidden") + 7919 * step
    return synth.random_normal_bf16(seed, n_tokens * hidden).reshape(n_tokens, hidden)


class MoELayer:
    """Runs one MoE layer on batches of tokens (bf16 ``[B, H]`` in, bf16 ``[B, H]`` out)."""

    PATHS = {"auto": nat.PATH_AUTO, "gemv": nat.PATH_GEMV, "gemm": nat.PATH_GEMM, "fused": nat.PATH_FUSED}

    def __init__(self, weights: MoELayerWeights, experts_per_token: int = 4, swiglu_limit: float = 7.0,
                 precision: str = "fp32", path: str = "auto") -> None:
        if precision not in ops.PRECISIONS:
            raise ValueError(f"unknown matmul precision {precision!r}")
        if path not in self.PATHS:
            raise ValueError(f"unknown expert path {path!r} (auto, gemv, gemm or fused)")
        self.w = weights
        self.k = min(int(experts_per_token), weights.n_experts)
        self.limit = float(swiglu_limit)
        self.precision = precision
        self.path = path
        self._ws: dict[int, torch.Tensor] = {}
        # the one-launch layer's status word of the last call, copied to the host without a sync
        self._pending_status: tuple | None = None

    def workspace(self, n_tokens: int) -> torch.Tensor:
        ws = self._ws.get(n_tokens)
        if ws is None:
            nbytes = ops.workspace_bytes(n_tokens, self.w.hidden, self.w.inter, self.w.n_experts, self.k)
            # zero-filled once: it carries completion counters that every call resets
            ws = torch.zeros(nbytes, dtype=torch.uint8, device=self.w.device)
            self._ws[n_tokens] = ws
        return ws

    def forward(self, x: torch.Tensor, out: torch.Tensor | None = None, ids: torch.Tensor | None = None,
                weights: torch.Tensor | None = None, events: list | None = None,
                residual: torch.Tensor | None = None) -> torch.Tensor:
        """Fused layer (klc_moe_layer); optional ``ids``/``weights`` receive the routing.

        ``residual``: bf16 ``[B, H]`` added to the output (``out`` may be it).

        ``events``: optional list of ``KLC_LAYER_EVENTS`` recorded
        ``torch.cuda.Event`` objects, re-recorded around the six kernels.

        More tokens than one library call takes (:meth:`max_tokens_per_call`)
        run as consecutive calls on row chunks; every token's routing, expert
        outputs and combine depend on that token alone, so the result is the
        one a single call would give.
        """
        ops._check_gpu("hidden", x, torch.bfloat16, 2)
        n_tok, hidden = x.shape
        if hidden != self.w.hidden:
            raise ValueError(f"hidden size {hidden} != layer hidden {self.w.hidden}")
        if residual is not None:
            ops._check_gpu("residual", residual, torch.bfloat16, 2)
            if residual.shape != x.shape:
                raise ValueError(f"residual shape {tuple(residual.shape)} != hidden shape {tuple(x.shape)}")
        if out is None:
            out = torch.empty_like(x)
        chunk = self.max_tokens_per_call()
        if n_tok > chunk:
            if events is not None:
                raise ValueError(f"events are recorded around one call of at most {chunk} tokens, got {n_tok}")
            for t0 in range(0, n_tok, chunk):
                t1 = min(n_tok, t0 + chunk)
                self.forward(x[t0:t1], out=out[t0:t1], ids=None if ids is None else ids[t0:t1],
                             weights=None if weights is None else weights[t0:t1],
                             residual=None if residual is None else residual[t0:t1])
            return out
        ws = self.workspace(n_tok)
        w = self.w
        if self.path == "fused":
            self._check_fused_status(block=False)
        ev = None
        if events is not None:
            if len(events) != nat.LAYER_EVENTS:
                raise ValueError(f"need {nat.LAYER_EVENTS} events, got {len(events)}")
            ev = (ctypes.c_void_p * nat.LAYER_EVENTS)(*[e.cuda_event for e in events])
        nat.call("klc_moe_layer", ops._ptr(x), ops._ptr(w.router_weight), ops._ptr(w.router_bias),
                 ops._ptr(w.gate_up_table), ops._ptr(w.gate_up_bias), ops._ptr(w.down_table), ops._ptr(w.down_bias),
                 n_tok, hidden, w.inter, w.n_experts, self.k, self.limit, ops.PRECISIONS[self.precision],
                 self.PATHS[self.path], ops._ptr(ws), ws.numel(), ops._ptr(out), ops._ptr(residual), ops._ptr(ids),
                 ops._ptr(weights), ev, ops._stream(x.device))
        if self.path == "fused":
            self._copy_fused_status(n_tok)
        return out

    __call__ = forward

    def _copy_fused_status(self, n_tokens: int) -> None:
        """Queues a copy of the one-launch layer's status word to pinned host memory (no sync)."""
        w = self.w
        off = nat.call("klc_moe_layer_status_offset", n_tokens, w.hidden, w.inter, w.n_experts, self.k)
        if off < 0:
            return
        host = torch.empty(4, dtype=torch.uint8, pin_memory=True)
        host.copy_(self._ws[n_tokens][off:off + 4], non_blocking=True)
        event = torch.cuda.Event()
        event.record(torch.cuda.current_stream(w.device))
        self._pending_status = (event, host)

    def _check_fused_status(self, block: bool) -> None:
        """Raises if a wait of the last one-launch call ran out (its outputs are then poisoned: NaN
        outputs and weights, ids -1).  Without ``block`` an unfinished call is checked at a later one."""
        if self._pending_status is None:
            return
        event, host = self._pending_status
        if block:
            event.synchronize()
        elif not event.query():
            return
        self._pending_status = None
        if int(host.numpy().view(np.uint32)[0]) & 1:
            raise RuntimeError("one-launch MoE layer: a cross-workgroup wait ran out (the GPU's compute units "
                               "were held by other work); that call's outputs are NaN and its ids -1, and this "
                               "layer's workspace keeps the failure flag")

    def check_fused_status(self) -> None:
        """Synchronises with the last one-launch call and raises if one of its waits ran out."""
        self._check_fused_status(block=True)

    def forward_static_scratch(self, x: torch.Tensor, out: torch.Tensor | None = None,
                               ids: torch.Tensor | None = None, weights: torch.Tensor | None = None,
                               residual: torch.Tensor | None = None) -> torch.Tensor:
        """:meth:`forward` without a workspace (klc_moe_layer_static_scratch).

        The library's static per-GPU scratch is used instead of a workspace
        tensor, so nothing is allocated when ``out`` is given: for callers
        that cannot allocate (HIP graph capture, serving loops).  Calls on one
        GPU share that scratch and must be ordered on one stream.
        """
        ops._check_gpu("hidden", x, torch.bfloat16, 2)
        if x.shape[1] != self.w.hidden:
            raise ValueError(f"hidden size {x.shape[1]} != layer hidden {self.w.hidden}")
        if residual is not None:
            ops._check_gpu("residual", residual, torch.bfloat16, 2)
            if residual.shape != x.shape:
                raise ValueError(f"residual shape {tuple(residual.shape)} != hidden shape {tuple(x.shape)}")
        if out is None:
            out = torch.empty_like(x)
        w = self.w
        nat.call("klc_moe_layer_static_scratch", ops._ptr(x), ops._ptr(w.router_weight), ops._ptr(w.router_bias),
                 ops._ptr(w.gate_up_table), ops._ptr(w.gate_up_bias), ops._ptr(w.down_table), ops._ptr(w.down_bias),
                 x.shape[0], w.hidden, w.inter, w.n_experts, self.k, self.limit, ops.PRECISIONS[self.precision],
                 self.PATHS[self.path], ops._ptr(out), ops._ptr(residual), ops._ptr(ids), ops._ptr(weights), None,
                 ops._stream(x.device))
        return out

    def capture_graph(self, x: torch.Tensor, out: torch.Tensor, ids: torch.Tensor | None = None,
                      weights: torch.Tensor | None = None, residual: torch.Tensor | None = None
                      ) -> "torch.cuda.CUDAGraph":
        """A HIP graph of one :meth:`forward_static_scratch` call on these buffers.

        ``graph.replay()`` then runs the layer's kernels with one launch from
        the host, on the same tensors (refill ``x`` in place to route new
        tokens).  The layer runs on the library's static scratch, so the call
        allocates nothing and records no memset; one eager call made first
        sets up that scratch on the device.  Replays share the scratch with
        every other static-scratch call on the GPU: order them on one stream.
        """
        self.forward_static_scratch(x, out=out, ids=ids, weights=weights, residual=residual)
        torch.cuda.synchronize(x.device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self.forward_static_scratch(x, out=out, ids=ids, weights=weights, residual=residual)
        return graph

    def max_tokens_per_call(self) -> int:
        """Tokens one klc_moe_layer call takes: the layer takes at most
        KLC_LAYER_MAX_TOKENS tokens (and KLC_DISPATCH_MAX_PAIRS token-slot
        pairs); the decode GEMVs, when forced (path "gemv"), at most 65535
        work units of 4 pairs."""
        n = ops.max_tokens_per_call(self.k)
        if self.path == "gemv":
            n = min(n, (4 * 65535 - 3 * self.w.n_experts) // self.k)
        return n

    def uses_gemm(self, n_tokens: int) -> bool:
        """Whether :meth:`forward` runs the grouped GEMM for ``n_tokens`` tokens (the library's rule)."""
        return self.layer_path(n_tokens) == "gemm"

    def fused_status(self, n_tokens: int) -> int:
        """The one-launch layer's status word in this layer's workspace for ``n_tokens`` (0: every wait
        of every launch ended on its condition; bit 0: some wait ran out).  Synchronises the device."""
        w = self.w
        off = nat.call("klc_moe_layer_status_offset", n_tokens, w.hidden, w.inter, w.n_experts, self.k)
        if off < 0 or n_tokens not in self._ws:
            return 0
        return int(self._ws[n_tokens][off:off + 4].cpu().numpy().view(np.uint32)[0])

    def layer_path(self, n_tokens: int) -> str:
        """The path :meth:`forward` takes for ``n_tokens`` tokens on the current stream (the library's
        rule, klc_moe_layer_path): ``"gemv"``, ``"gemm"``, or ``"fused"`` (the whole layer in one
        launch, batches of at most 16 tokens; only when this layer's path is ``"fused"``)."""
        w = self.w
        code = nat.call("klc_moe_layer_path", n_tokens, w.hidden, w.inter, w.n_experts, self.k,
                        self.PATHS[self.path], ops._stream(w.device))
        return {nat.PATH_GEMV: "gemv", nat.PATH_GEMM: "gemm", nat.PATH_FUSED: "fused"}[code]

    def forward_detailed(self, x: torch.Tensor, routing: tuple[torch.Tensor, torch.Tensor] | None = None) -> dict:
        """Step-by-step path exposing every intermediate (same kernels as :meth:`forward`).

        ``routing`` optionally supplies precomputed ``(ids int32 [B, k],
        weights bf16 [B, k])`` (the routing-locality path decides the experts on
        the host); otherwise the GPU router selects them.
        """
        w = self.w
        logits = ops.router_logits(x, w.router_weight, w.router_bias)
        values = None
        if routing is None:
            ids, values, weights = ops.topk_softmax(logits, self.k)
        else:
            ids, weights = routing
            ops._check_gpu("ids", ids, torch.int32, 2)
            ops._check_gpu("weights", weights, torch.bfloat16, 2)
        k = ids.shape[1]
        disp = ops.dispatch(ids, w.n_experts)
        gemm = self.uses_gemm(x.shape[0])
        gated, gated_raw = ops.gate_up(w.gate_up_table, w.gate_up_bias, x, k, disp, w.hidden, w.inter, self.limit,
                                       self.precision, want_raw=True, gemm=gemm)
        eo = ops.down(w.down_table, w.down_bias, gated, disp, w.hidden, w.inter, self.precision, gemm=gemm)
        out = ops.combine(eo, weights, x.shape[0], k)
        return {"out": out, "logits": logits, "ids": ids, "values": values, "weights": weights,
                "offsets": disp.offsets, "sorted_pairs": disp.sorted_pairs, "active": disp.active,
                "n_active": disp.n_active, "units": disp.units, "gated": gated_raw, "gated_act": gated,
                "expert_out": eo}


def synthetic_norm_weight(workload: int, layer: int, hidden: int) -> np.ndarray:
    """bf16 bit patterns of a layer's RMSNorm weight, 1 + N(0, 0.05)."""
    return synth.random_normal_bf16(synth.tensor_seed(workload, "norm_weight", layer), hidden, 1.0, 0.05)


class MoEStack:
    """Stacked MoE decode: per layer ``h += moe(rms_norm(h))``.

    The MoE-only view of the executor's layer loop
    (streamed_transformer_executor.py:247-260): post-attention RMSNorm
    (streamed_attention.py:27-28), the routed experts, and the residual add,
    fused into the layer's combine.  All layers stay resident in HBM.
    """

    def __init__(self, layers: list[MoELayerWeights], norm_weights: list[torch.Tensor], experts_per_token: int = 4,
                 swiglu_limit: float = 7.0, precision: str = "fp32", eps: float = 1e-5) -> None:
        if len(layers) != len(norm_weights):
            raise ValueError(f"{len(layers)} layers but {len(norm_weights)} norm weights")
        self.layers = [MoELayer(w, experts_per_token, swiglu_limit, precision) for w in layers]
        self.norm_weights = norm_weights
        self.eps = float(eps)
        self._normed: dict[tuple, torch.Tensor] = {}

    def forward(self, hidden: torch.Tensor, out: torch.Tensor | None = None, trace: list | None = None,
                ids: list | None = None) -> torch.Tensor:
        """Runs every layer on bf16 ``hidden [B, H]``; returns the final hidden state.

        ``trace``: if a list, receives a copy of the hidden state after each
        layer.  ``ids``: if a list of int32 ``[B, k]`` tensors (one per layer),
        they receive each layer's routing.
        """
        ops._check_gpu("hidden", hidden, torch.bfloat16, 2)
        h = out if out is not None else torch.empty_like(hidden)
        if h.data_ptr() != hidden.data_ptr():
            h.copy_(hidden)
        key = tuple(hidden.shape)
        normed = self._normed.get(key)
        if normed is None:
            normed = self._normed[key] = torch.empty_like(hidden)
        for i, (layer, nw) in enumerate(zip(self.layers, self.norm_weights)):
            ops.rms_norm(h, nw, self.eps, out=normed)
            layer.forward(normed, out=h, residual=h, ids=None if ids is None else ids[i])
            if trace is not None:
                trace.append(h.clone())
        return h

    __call__ = forward

    @classmethod
    def synthetic(cls, workload: int, n_layers: int, hidden: int, inter: int, n_experts: int,
                  device: torch.device | str = "cuda", **kwargs) -> "MoEStack":
        dev = torch.device(device)
        layers = [MoELayerWeights.synthetic(workload, l, hidden, inter, n_experts, dev) for l in range(n_layers)]
        norms = [torch.from_numpy(synthetic_norm_weight(workload, l, hidden).view(np.int16)).view(torch.bfloat16)
                 .to(dev) for l in range(n_layers)]
        return cls(layers, norms, **kwargs)
