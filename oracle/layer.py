"""One MoE layer for a batch of tokens (test infrastructure only).

Composes the router (streamed_moe_router.py:268-284), the expert loop
(:483-522) and the combine for every token of a batch, as ``B`` independent
1-D ``route`` calls would.  Experts are evaluated per unique expert on all of
its tokens at once; the arithmetic per token is the same.
"""

from __future__ import annotations

import numpy as np

from . import experts as ex
from . import mxfp4, router
from .numerics import bf16_to_f32


def moe_layer(x_bits, router_w_bits, router_b_bits, gu_blocks, gu_scales, gu_bias_bits,
              d_blocks, d_scales, d_bias_bits, k: int = 4, limit: float = 7.0, precision: str = "fp32"):
    """Returns a dict with ``out`` (bf16 patterns ``[B, H]``), ``logits``,
    ``ids``, ``values``, ``weights``, ``gated [B, k, I]`` and ``expert_out [B, k, H]``.
    """
    x_bits = np.atleast_2d(np.asarray(x_bits, dtype=np.uint16))
    n_tok, hidden = x_bits.shape
    n_exp = router_w_bits.shape[0]
    logits = router.router_logits(x_bits, router_w_bits, router_b_bits)
    ids, values = router.topk(logits, k)
    k = ids.shape[1]
    weights = router.softmax_weights(values)
    x = bf16_to_f32(x_bits)
    inter = gu_blocks.shape[1] // 2
    gated = np.zeros((n_tok, k, inter), dtype=np.float32)
    out = np.zeros((n_tok, k, hidden), dtype=np.float32)
    for e in np.unique(ids):
        rows, slots = np.nonzero(ids == e)
        w_gu = mxfp4.dequantize(gu_blocks[e], gu_scales[e], "f32")
        w_d = mxfp4.dequantize(d_blocks[e], d_scales[e], "f32")
        g, o = ex.expert_ffn(x[rows], w_gu, gu_bias_bits[e], w_d, d_bias_bits[e], limit, precision)
        gated[rows, slots] = g
        out[rows, slots] = o
    return {
        "out": ex.combine(out, weights),
        "logits": logits,
        "ids": ids,
        "values": values,
        "weights": weights,
        "gated": gated,
        "expert_out": out,
        "num_experts": n_exp,
    }


def moe_layer_lazy(x_bits, router_w_bits, router_b_bits, expert_fn, gu_bias_bits, d_bias_bits, k: int = 4,
                   limit: float = 7.0, precision: str = "fp32", workers: int = 4):
    """``moe_layer`` for layers too large to hold on the host: ``expert_fn(e)``
    returns expert ``e``'s ``(gate_up_blocks, gate_up_scales, down_blocks,
    down_scales)`` in checkpoint layout, and only the experts the tokens
    select are built.  Experts are evaluated by ``workers`` threads; the
    arithmetic per token is ``moe_layer``'s.
    """
    from concurrent.futures import ThreadPoolExecutor

    x_bits = np.atleast_2d(np.asarray(x_bits, dtype=np.uint16))
    n_tok, hidden = x_bits.shape
    logits = router.router_logits(x_bits, router_w_bits, router_b_bits)
    ids, values = router.topk(logits, k)
    k = ids.shape[1]
    weights = router.softmax_weights(values)
    x = bf16_to_f32(x_bits)

    def run(e):
        gub, gus, db, ds = expert_fn(int(e))
        rows, slots = np.nonzero(ids == e)
        w_gu = mxfp4.dequantize(gub, gus, "f32")
        w_d = mxfp4.dequantize(db, ds, "f32")
        g, o = ex.expert_ffn(x[rows], w_gu, gu_bias_bits[e], w_d, d_bias_bits[e], limit, precision)
        return rows, slots, g, o

    inter = None
    gated = out = None
    with ThreadPoolExecutor(max_workers=max(int(workers), 1)) as pool:
        for rows, slots, g, o in pool.map(run, np.unique(ids)):
            if gated is None:
                inter = g.shape[1]
                gated = np.zeros((n_tok, k, inter), dtype=np.float32)
                out = np.zeros((n_tok, k, hidden), dtype=np.float32)
            gated[rows, slots] = g
            out[rows, slots] = o
    return {"out": ex.combine(out, weights), "logits": logits, "ids": ids, "values": values, "weights": weights,
            "gated": gated, "expert_out": out, "num_experts": router_w_bits.shape[0]}

