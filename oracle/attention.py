"""Decode attention: YaRN RoPE, sinks, sliding window (test infrastructure only).

Restates streamed_attention.py:27-152 for one decode token:
* ``yarn_inv_freq`` (:39-78) and the attention scaling (:30-36);
* the rotation of ``apply_rope`` (:88-98) in bfloat16, each torch op rounded
  to bfloat16 (a*cos, b*sin, their difference / sum);
* the scores of ``forward`` (:128-139): float32 ``q . k / sqrt(head_dim)``
  (here the exact dot product rounded once), the sink logit appended, the
  maximum subtracted, softmax in float32 and the probabilities rounded to
  bfloat16, then ``context = probs . values`` accumulated exactly and
  rounded to bfloat16 (torch's bf16 einsum accumulates in float32).
"""

from __future__ import annotations

import math

import numpy as np

from .numerics import bf16_to_f32, f32_to_bf16


def yarn_inv_freq(head_dim: int, base: float, factor: float, original_max: int, beta_fast: float,
                  beta_slow: float, truncate: bool = False) -> np.ndarray:
    """float64 ``[head_dim / 2]`` (streamed_attention.py:39-78)."""
    def correction_dim(rotations: float) -> float:
        return head_dim * math.log(original_max / (rotations * 2 * math.pi)) / (2 * math.log(base))

    low, high = correction_dim(beta_fast), correction_dim(beta_slow)
    if truncate:
        low, high = math.floor(low), math.ceil(high)
    low, high = max(low, 0.0), min(high, float(head_dim - 1))
    if low == high:
        high += 0.001
    ramp = np.clip((np.arange(head_dim // 2, dtype=np.float64) - low) / (high - low), 0.0, 1.0)
    pos = base ** (np.arange(0, head_dim, 2, dtype=np.float64) / head_dim)
    extrap, interp = 1.0 / pos, 1.0 / (factor * pos)
    keep = 1.0 - ramp  # the extrapolation share
    return interp * (1.0 - keep) + extrap * keep


def attention_scaling(factor: float) -> float:
    return 1.0 if factor <= 1.0 else 0.1 * math.log(factor) + 1.0


def rope_rotate(x_bits: np.ndarray, cos_bits: np.ndarray, sin_bits: np.ndarray) -> np.ndarray:
    """Rotates ``[..., head_dim]`` bfloat16 rows by bfloat16 cos/sin ``[head_dim / 2]``
    with a bfloat16 rounding after every op (streamed_attention.py:90-97)."""
    x = bf16_to_f32(x_bits)
    c, s = bf16_to_f32(cos_bits), bf16_to_f32(sin_bits)
    half = x.shape[-1] // 2
    a, b = x[..., :half], x[..., half:]
    r = lambda v: bf16_to_f32(f32_to_bf16(v))  # noqa: E731
    first = f32_to_bf16(r(r(a * c) - r(b * s)))
    second = f32_to_bf16(r(r(b * c) + r(a * s)))
    return np.concatenate([first, second], axis=-1)


def to_kv(x_f32: np.ndarray, kv: str) -> np.ndarray:
    """float32 values rounded to the KV cache's type (kv_cache_manager.py:104-107):
    "fp16" -> float16, "bf16" -> bfloat16; returned as float32."""
    x_f32 = np.asarray(x_f32, dtype=np.float32)
    if kv == "fp16":
        return x_f32.astype(np.float16).astype(np.float32)
    return bf16_to_f32(f32_to_bf16(x_f32))


def decode_attention(q_bits: np.ndarray, k_bits: np.ndarray, v_bits: np.ndarray, sinks_bits: np.ndarray | None,
                     window: int | None = None, kv: str = "bf16") -> tuple[np.ndarray, np.ndarray]:
    """q ``[NH, D]``, k/v ``[T, NKV, D]`` (bf16 patterns: the post-RoPE keys and
    the values before they are stored), sinks ``[NH]`` or None; the last
    ``window`` keys when given; ``kv`` the cache's type.  Returns (context
    bf16 ``[NH, D]``, probs ``[NH, T']`` as float32 values of the cache type)."""
    if window:
        k_bits, v_bits = k_bits[-window:], v_bits[-window:]
    nh, d = q_bits.shape
    rep = nh // k_bits.shape[1]
    q = bf16_to_f32(q_bits).astype(np.float64)
    k = np.repeat(to_kv(bf16_to_f32(k_bits), kv).astype(np.float64), rep, axis=1)  # [T, NH, D]
    v = np.repeat(to_kv(bf16_to_f32(v_bits), kv).astype(np.float64), rep, axis=1)
    scores = np.einsum("hd,thd->ht", q, k).astype(np.float32) / np.float32(math.sqrt(d))
    if sinks_bits is not None:
        combined = np.concatenate([scores, bf16_to_f32(sinks_bits)[:, None]], axis=1)
    else:
        combined = scores
    combined = combined - combined.max(axis=1, keepdims=True)
    e = np.exp(combined.astype(np.float64))
    p = (e / e.sum(axis=1, keepdims=True)).astype(np.float32)
    if sinks_bits is not None:
        p = p[:, :-1]
    probs = to_kv(p, kv)
    ctx = np.einsum("ht,thd->hd", probs.astype(np.float64), v)
    return f32_to_bf16(to_kv(ctx.astype(np.float32), kv)), probs
