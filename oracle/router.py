"""Router logits, top-k, softmax weights and dispatch (test infrastructure only).

Restates streamed_moe_router.py:268-284 with routing locality disabled (the
default, :14, :333-334 and :374-375), for a batch of tokens processed one row
at a time exactly as the 1-D ``route`` does.
"""

from __future__ import annotations

import numpy as np

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
    """``torch.topk(logits.float(), k)`` per row (streamed_moe_router.py:270-278).

    ``k = min(experts_per_token, E)`` (:442-451).  Values descend; equal values
    are ordered by lower expert index first (the tie rule of this
    implementation; torch leaves it implementation defined).
    """
    vals = bf16_to_f32(np.atleast_2d(logits_bits))
    k = min(int(k), vals.shape[1])
    # NaN sorts first, as in torch.topk (NaN is treated as the largest value).
    key = np.where(np.isnan(vals), -np.inf, -vals)
    order = np.argsort(key, axis=1, kind="stable")[:, :k]
    return order.astype(np.int64), np.take_along_axis(vals, order, axis=1)


def softmax_weights(values: np.ndarray) -> np.ndarray:
    """``torch.softmax(fp32 scores).to(bf16)`` (streamed_moe_router.py:281-282).

    Computed in float64 and rounded to float32, then to bfloat16.
    """
    v = np.asarray(values, dtype=np.float32).astype(np.float64)
    m = v.max(axis=-1, keepdims=True)
    e = np.exp(v - m)
    w = (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)
    return f32_to_bf16(w)


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
