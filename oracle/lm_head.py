"""lm_head logits and greedy next token (test infrastructure only).

Restates StreamedTransformerExecutor.logits (streamed_transformer_executor.py:177-209:
``torch.matmul(W[chunk].float(), hidden.float())`` per 4096-row chunk,
concatenated on the host) and the greedy pick of its callers
(generation_runtime.py:118-122, inference_server.py:383-386:
``nan_to_num(nan=-1e9, posinf=1e9, neginf=-1e9)`` then ``argmax``, whose
ties go to the first index).  The products of a bfloat16 weight and a float32
activation are exact in float64; the dot product is accumulated in float64
and rounded once to float32, so the result is the correctly rounded value of
the reference's float32 dot product (whose own accumulation order is left to
the BLAS).
"""

from __future__ import annotations

import numpy as np

from .numerics import bf16_to_f32


def logits(w_bits: np.ndarray, x: np.ndarray, chunk_rows: int = 4096) -> np.ndarray:
    """float32 ``[V]``: f32(sum_h f64(w[v, h]) * f64(x[h])); w is uint16 bfloat16
    patterns ``[V, H]``, x float32 ``[H]``.  Chunked like the reference so a
    full vocabulary never needs a float64 copy of the whole matrix."""
    xd = np.asarray(x, dtype=np.float32).astype(np.float64)
    out = np.empty(w_bits.shape[0], dtype=np.float32)
    for start in range(0, w_bits.shape[0], chunk_rows):
        w = bf16_to_f32(w_bits[start:start + chunk_rows]).astype(np.float64)
        out[start:start + chunk_rows] = (w @ xd).astype(np.float32)
    return out


def nan_to_num(v: np.ndarray) -> np.ndarray:
    """``torch.nan_to_num(v, nan=-1e9, posinf=1e9, neginf=-1e9)`` in float32."""
    v = np.asarray(v, dtype=np.float32).copy()
    v[np.isnan(v)] = np.float32(-1e9)
    v[np.isposinf(v)] = np.float32(1e9)
    v[np.isneginf(v)] = np.float32(-1e9)
    return v


def greedy_token(raw_logits: np.ndarray) -> int:
    """``argmax(nan_to_num(raw))``, the first index among equal maxima."""
    return int(np.argmax(nan_to_num(raw_logits)))
