"""The reference's MoE path as torch CPU ops — TEST AND BASELINE INFRASTRUCTURE ONLY.

The reference never runs on the GPU box, so its CPU cost is measured on this
restatement: the same torch operations, dtypes and rounding points as

* ``dequantize_mxfp4_matrix`` (mxfp4_expert.py:357-379): code lookup in a
  16-entry table of the target dtype, ``torch.ldexp`` by the E8M0 exponent,
  the ``[in, out]`` transposed copy;
* ``StreamedMoERouter.route`` with routing locality disabled
  (streamed_moe_router.py:268-284): bf16 ``F.linear``, ``topk`` of the float
  logits, bf16 softmax weights;
* ``_execute_mxfp4_experts`` and ``_apply_gate`` (:483-529) in the
  executor's default float32 matmul mode (streamed_transformer_executor.py:54):
  ``hidden.float() @ W.float() + b.float()``, interleaved gate/up clamped
  SwiGLU, the down matmul, and the slot-order bf16 combine; or in its
  ``matmul_precision="bf16"`` mode (:502-511): bf16 operands, the matmul
  results in bf16, then ``.float() + b.float()``.

Two variants, as the reference's expert store behaves:

* cold (``cache_bytes=0``): every call dequantizes its experts again (the
  miss path without the disk and PCIe part, the checkpoint being in RAM);
* warm: the dequantized bf16 matrices are already cached (the hit path,
  including its per-call ``.float()`` copies).

Only bench.py's ``cpu_baseline`` leg and tests/ use this module.
"""

from __future__ import annotations

import torch

FP4_TABLE = [+0.0, +0.5, +1.0, +1.5, +2.0, +3.0, +4.0, +6.0,
             -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]  # mxfp4_expert.py:17-34


def dequantize(blocks: torch.Tensor, scales: torch.Tensor, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """MXFP4 ``[out, G, 16]`` + E8M0 ``[out, G]`` -> ``[in, out]`` (mxfp4_expert.py:357-379)."""
    out_dim, groups, width = blocks.shape
    table = torch.tensor(FP4_TABLE, dtype=dtype)
    codes = blocks.reshape(out_dim * groups, width)
    vals = torch.empty(out_dim * groups, 2 * width, dtype=dtype)
    vals[:, 0::2] = table[(codes & 0x0F).long()]
    vals[:, 1::2] = table[(codes >> 4).long()]
    torch.ldexp(vals, scales.reshape(-1, 1).to(torch.int32) - 127, out=vals)
    return vals.reshape(out_dim, groups * 2 * width).transpose(0, 1).contiguous()


def swiglu(gate_up: torch.Tensor, limit: float = 7.0, alpha: float = 1.702) -> torch.Tensor:
    """``_apply_gate`` (streamed_moe_router.py:524-529)."""
    gate = gate_up[..., ::2].clamp(max=limit)
    up = gate_up[..., 1::2].clamp(min=-limit, max=limit)
    return (up + 1.0) * (gate * torch.sigmoid(gate * alpha))


class Layer:
    """One MoE layer's tensors on the host: router, biases, and the checkpoint-layout
    MXFP4 tensors of the experts it may select (``experts[e] = (gate_up_blocks,
    gate_up_scales, down_blocks, down_scales)``, torch uint8)."""

    def __init__(self, router_weight, router_bias, gate_up_bias, down_bias, experts: dict, k: int = 4,
                 limit: float = 7.0) -> None:
        self.router_weight, self.router_bias = router_weight, router_bias
        self.gate_up_bias, self.down_bias = gate_up_bias, down_bias
        self.experts = experts
        self.k, self.limit = k, limit
        self.cache: dict[tuple[int, str], torch.Tensor] = {}  # the warm store's dequantized matrices

    def select(self, hidden: torch.Tensor) -> list[int]:
        """The experts ``route`` picks for one token (router and top-k only)."""
        logits = torch.nn.functional.linear(hidden, self.router_weight, self.router_bias)
        return torch.topk(logits.float(), k=min(self.k, logits.numel())).indices.tolist()

    def matrix(self, expert: int, proj: str, warm: bool) -> torch.Tensor:
        key = (expert, proj)
        if warm and key in self.cache:
            return self.cache[key]
        gub, gus, db, ds = self.experts[expert]
        m = dequantize(gub, gus) if proj == "gate_up_proj" else dequantize(db, ds)
        if warm:
            self.cache[key] = m
        return m

    def route(self, hidden: torch.Tensor, warm: bool, precision: str = "fp32") -> tuple[torch.Tensor, list[int]]:
        """One 1-D token through router, top-k, experts and combine (bf16 hidden in, bf16 out);
        ``precision`` is the reference's matmul_precision ("fp32" or "bf16")."""
        if precision not in ("fp32", "bf16"):
            raise ValueError(f"unknown matmul precision {precision!r}")
        logits = torch.nn.functional.linear(hidden, self.router_weight, self.router_bias)
        top = torch.topk(logits.float(), k=min(self.k, logits.numel()))
        experts = top.indices.tolist()
        weights = torch.softmax(torch.tensor([float(v) for v in top.values], dtype=torch.float32), dim=-1)
        weights = weights.to(hidden.dtype)
        output = torch.zeros_like(hidden)
        for pos, e in enumerate(experts):
            gate_up = self.matrix(e, "gate_up_proj", warm)
            down = self.matrix(e, "down_proj", warm)
            if precision == "bf16":  # streamed_moe_router.py:502-511
                gu = (hidden.to(torch.bfloat16) @ gate_up.to(torch.bfloat16)).float() + self.gate_up_bias[e].float()
            else:
                gu = hidden.float() @ gate_up.float() + self.gate_up_bias[e].float()
            gated = swiglu(gu, self.limit)
            if precision == "bf16":
                out = (gated.to(torch.bfloat16) @ down.to(torch.bfloat16)).float() + self.down_bias[e].float()
            else:
                out = gated @ down.float() + self.down_bias[e].float()
            output += out.to(hidden.dtype) * weights[pos]
        return output, experts
