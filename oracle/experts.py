"""Selected-expert feed-forward and weighted combine (test infrastructure only).

Restates streamed_moe_router.py:483-529 (``_execute_mxfp4_experts`` and
``_apply_gate``) and the bias-only fallback (:317-322).
"""

from __future__ import annotations

import numpy as np

from .numerics import bf16_to_f32, f32_to_bf16, round_bf16

SWIGLU_ALPHA = 1.702  # streamed_moe_router.py:248


def swiglu(gate_up: np.ndarray, limit: float = 7.0, alpha: float = SWIGLU_ALPHA) -> np.ndarray:
    """``_apply_gate`` (streamed_moe_router.py:524-529) in float32.

    Columns are interleaved: even = gate, odd = up.  The gate is clamped from
    above only, the up projection to ``[-limit, limit]``;
    ``out = (up + 1) * gate * sigmoid(alpha * gate)``.
    """
    gu = np.asarray(gate_up, dtype=np.float32)
    lim = np.float32(limit)
    gate = np.minimum(gu[..., 0::2], lim)
    up = np.clip(gu[..., 1::2], -lim, lim)
    with np.errstate(over="ignore"):
        sig = np.float32(1.0) / (np.float32(1.0) + np.exp(-(gate * np.float32(alpha))))
    glu = gate * sig
    return ((up + np.float32(1.0)) * glu).astype(np.float32)


def _gemv_f32(act: np.ndarray, weight_in_out: np.ndarray) -> np.ndarray:
    """``act @ W`` with float64 accumulation rounded once to float32."""
    return (np.asarray(act, dtype=np.float64) @ np.asarray(weight_in_out, dtype=np.float64)).astype(np.float32)


def expert_ffn(x: np.ndarray, gate_up_w: np.ndarray, gate_up_b_bits: np.ndarray, down_w: np.ndarray,
               down_b_bits: np.ndarray, limit: float = 7.0, precision: str = "fp32"):
    """One expert on a batch of activations (streamed_moe_router.py:500-511).

    ``x`` is float32 ``[n, H]`` holding bfloat16 values; ``gate_up_w`` is the
    dequantized ``[H, 2I]`` and ``down_w`` the ``[I, H]`` matrix as float32.
    ``precision="fp32"`` (the executor default) multiplies in float32;
    ``"bf16"`` rounds each matmul result (and the down input) to bfloat16
    before the float32 bias add.  Returns ``(gated [n, I], out [n, H])``.
    """
    gu_b = bf16_to_f32(gate_up_b_bits)
    d_b = bf16_to_f32(down_b_bits)
    if precision == "bf16":
        gu = round_bf16(_gemv_f32(round_bf16(x), gate_up_w)) + gu_b
    elif precision == "fp32":
        gu = _gemv_f32(x, gate_up_w) + gu_b
    else:
        raise ValueError(f"unknown matmul precision {precision!r}")
    gated = swiglu(gu, limit)
    if precision == "bf16":
        out = round_bf16(_gemv_f32(round_bf16(gated), down_w)) + d_b
    else:
        out = _gemv_f32(gated, down_w) + d_b
    return gated.astype(np.float32), out.astype(np.float32)


def combine(expert_out: np.ndarray, weights_bits: np.ndarray) -> np.ndarray:
    """Weighted sum in top-k order (streamed_moe_router.py:497, 512-513).

    ``output`` starts as bfloat16 zeros; for each slot in order,
    ``output += out.to(bf16) * w`` with every operation rounded to bfloat16.
    ``expert_out`` is float32 ``[B, k, H]``; weights are bfloat16 ``[B, k]``.
    Returns uint16 patterns ``[B, H]``.
    """
    outs = np.asarray(expert_out, dtype=np.float32)
    w = bf16_to_f32(weights_bits)
    acc = np.zeros((outs.shape[0], outs.shape[2]), dtype=np.float32)
    for j in range(outs.shape[1]):
        term = round_bf16(round_bf16(outs[:, j, :]) * w[:, j:j + 1])
        acc = round_bf16(acc + term)
    return f32_to_bf16(acc)


def bias_only(down_bias_bits: np.ndarray, ids: np.ndarray, weights_bits: np.ndarray) -> np.ndarray:
    """``execute_experts=False`` fallback (streamed_moe_router.py:317-322).

    ``sum(down_bias[e_j] * w_j)`` with bfloat16 products and the sum
    accumulated in float32 in slot order, rounded once to bfloat16.
    """
    b = bf16_to_f32(down_bias_bits)
    w = bf16_to_f32(weights_bits)
    ids = np.atleast_2d(ids)
    acc = np.zeros((ids.shape[0], b.shape[1]), dtype=np.float32)
    for j in range(ids.shape[1]):
        acc = acc + round_bf16(b[ids[:, j]] * w[:, j:j + 1])
    return f32_to_bf16(acc)
