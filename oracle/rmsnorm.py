"""RMSNorm and residual add (test infrastructure only).

Restates streamed_attention.py:27-28 and the residual add at
streamed_transformer_executor.py:260, used by the stacked-layer workload.
"""

from __future__ import annotations

import numpy as np

from .numerics import bf16_to_f32, f32_to_bf16, round_bf16


def rms_norm(x_bits: np.ndarray, w_bits: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """``x * rsqrt(mean(x.float()**2) + eps).to(x.dtype) * w`` in bfloat16.

    The mean of squares is taken in float32 (here: float64, rounded once to
    float32), the reciprocal square root is rounded to bfloat16 before the two
    bfloat16 multiplies, each of which rounds to bfloat16.
    """
    x = bf16_to_f32(np.atleast_2d(x_bits))
    w = bf16_to_f32(w_bits)
    ms = np.mean(x.astype(np.float64) ** 2, axis=-1, keepdims=True).astype(np.float32)
    s = (ms + np.float32(eps)).astype(np.float32)
    r = (1.0 / np.sqrt(s.astype(np.float64))).astype(np.float32)
    r = round_bf16(r)
    return f32_to_bf16(round_bf16(x * r) * w)


def residual_add(h_bits: np.ndarray, d_bits: np.ndarray) -> np.ndarray:
    """``hidden += moe_out`` in bfloat16 (streamed_transformer_executor.py:260)."""
    return f32_to_bf16(bf16_to_f32(h_bits) + bf16_to_f32(d_bits))
