"""Router logits, top-k, softmax weights and dispatch (test infrastructure only).

Restates streamed_moe_router.py:268-284 with routing locality disabled (the
default, :14, :333-334 and :374-375), for a batch of tokens processed one row
at a time exactly as the 1-D ``route`` does.
"""

from __future__ import annotations

import numpy as np

from . import torch_cpu
from .numerics import bf16_to_f32, f32_to_bf16


def router_logits(x_bits: np.ndarray, w_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    """``F.linear(hidden, W, b)`` in bfloat16 (streamed_moe_router.py:269).

    bfloat16 products are exact in float64; the dot product is accumulated in
    float64, rounded once to float32, the float32 bias is added in float32 and
    the sum is rounded to bfloat16: ``bf16(f32(x . W) + b)``.  Returns uint16
    patterns ``[B, E]``.
    """
    x = bf16_to_f32(x_bits).astype(np.float64)
    w = bf16_to_f32(w_bits).astype(np.float64)
    b = bf16_to_f32(b_bits)
    acc = (np.atleast_2d(x) @ w.T).astype(np.float32)
    return f32_to_bf16(acc + b[None, :])


def topk(logits_bits: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    """``torch.topk(logits.float(), k)`` per row on CPU (streamed_moe_router.py:270-278).

    ``k = min(experts_per_token, E)`` (:442-451).  Values descend with NaN the
    largest; equal values come in the order torch's CPU kernel leaves them
    (libstdc++ ``nth_element`` + ``sort``, or ``partial_sort`` when
    ``k * 64 <= E``), restated in ``torch_cpu.topk_order``.
    """
    bits = np.atleast_2d(np.asarray(logits_bits, dtype=np.uint16))
    vals = bf16_to_f32(bits)
    k = min(int(k), vals.shape[1])
    keys = torch_cpu.order_key_bf16(bits)
    order = np.array([torch_cpu.topk_order(keys[r], k) for r in range(bits.shape[0])], dtype=np.int64)
    order = order.reshape(bits.shape[0], k)
    return order, np.take_along_axis(vals, order, axis=1)


def softmax_weights(values: np.ndarray) -> np.ndarray:
    """``torch.softmax(fp32 scores, dim=-1).to(bf16)`` (streamed_moe_router.py:281-282).

    The float32 softmax is torch's CPU kernel step for step
    (``torch_cpu.softmax_f32``), then rounded to bfloat16.
    """
    return f32_to_bf16(torch_cpu.softmax_f32(values))


def dispatch(ids: np.ndarray, num_experts: int):
    """Expert-sorted dispatch of the flattened (token, slot) pairs.

    No reference counterpart: the reference runs one token at a time.  A pair
    id is ``token * k + slot``; pairs are ordered by expert, then by pair id
    (a stable counting sort).  Returns ``(counts[E], offsets[E + 1],
    sorted_pairs[B * k], active_experts[U])``.
    """
    flat = np.asarray(ids, dtype=np.int64).reshape(-1)
    counts = np.bincount(flat, minlength=num_experts).astype(np.int64)
    offsets = np.zeros(num_experts + 1, dtype=np.int64)
    np.cumsum(counts, out=offsets[1:])
    order = np.argsort(flat, kind="stable").astype(np.int64)
    active = np.nonzero(counts)[0].astype(np.int64)
    return counts, offsets, order, active
