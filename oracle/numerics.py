"""Rounding helpers for the oracle (test infrastructure only)."""

from __future__ import annotations

import numpy as np


def f32_to_bf16(x) -> np.ndarray:
    """float32 -> bfloat16 bit patterns (uint16), round to nearest even.

    NaN maps to a quiet NaN with the sign kept; +-inf and overflow behave as
    IEEE round-to-nearest (overflow goes to inf).
    """
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    is_nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    with np.errstate(over="ignore"):
        rounded = (u + np.uint32(0x7FFF) + lsb) >> np.uint32(16)
    out = np.where(is_nan, (u >> np.uint32(16)) | np.uint32(0x0040), rounded)
    return out.astype(np.uint16)


def bf16_to_f32(bits) -> np.ndarray:
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def round_bf16(x) -> np.ndarray:
    """float32 values rounded to the nearest bfloat16, returned as float32."""
    return bf16_to_f32(f32_to_bf16(x))


def bf16_ulp_distance(a_bits, b_bits) -> np.ndarray:
    """Distance in units in the last place between bfloat16 patterns (finite values)."""
    def ordered(v):
        v = np.asarray(v, dtype=np.uint16).astype(np.int32)
        return np.where(v & 0x8000, 0x8000 - (v & 0x7FFF), 0x8000 + v)
    return np.abs(ordered(a_bits) - ordered(b_bits))
