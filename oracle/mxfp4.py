"""MXFP4 -> dense dequant, restated from mxfp4_expert.py (test infrastructure only).

Reference semantics (mxfp4_expert.py:357-379):

* ``blocks[out, G, 16]`` holds two E2M1 codes per byte: the low nibble is the
  even input column, the high nibble the odd one (:375-376).
* each code maps through ``FP4_VALUES`` (:17-34) and is multiplied by
  ``2 ** (scale - 127)`` (:367, :377).  ``torch.ldexp`` forms the power of two
  in float32 and rounds the product to the target dtype, so the value is
  ``dtype(float32(LUT[c]) * float32(2 ** (e - 127)))``: exact for every finite
  case, +-inf on overflow, NaN for a zero code at ``e = 255`` (0 * inf).
* the result is returned transposed, ``[in = 32 * G, out]`` contiguous (:379).
* mismatched ``blocks.shape[:-1]`` vs ``scales.shape`` raises ValueError (:368-369).
"""

from __future__ import annotations

import numpy as np

from .numerics import f32_to_bf16

# mxfp4_expert.py:17-34 — bit 3 is the sign, bits 0-2 index the magnitude.
FP4_VALUES = [+0.0, +0.5, +1.0, +1.5, +2.0, +3.0, +4.0, +6.0,
              -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]


def dequant_values_f32(blocks: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Exact float32 values ``[out, G * 32]`` (not transposed) of one matrix."""
    blocks = np.asarray(blocks, dtype=np.uint8)
    scales = np.asarray(scales, dtype=np.uint8)
    if blocks.shape[:-1] != scales.shape:
        raise ValueError(f"MXFP4 block/scale shape mismatch: {blocks.shape=} {scales.shape=}")
    out_dim, groups, packed = blocks.shape
    lut = np.array(FP4_VALUES, dtype=np.float32)
    vals = np.empty((out_dim, groups, packed * 2), dtype=np.float32)
    vals[..., 0::2] = lut[blocks & 0x0F]
    vals[..., 1::2] = lut[blocks >> 4]
    with np.errstate(over="ignore", invalid="ignore"):
        pow2 = np.ldexp(np.float32(1.0), scales.astype(np.int32) - 127).astype(np.float32)
        vals *= pow2[..., None]
    return vals.reshape(out_dim, groups * packed * 2)


def dequantize(blocks: np.ndarray, scales: np.ndarray, dtype: str = "bf16") -> np.ndarray:
    """``dequantize_mxfp4_matrix`` (mxfp4_expert.py:357) for one matrix.

    Returns ``[in, out]``: uint16 bfloat16 patterns for ``"bf16"``, float16 for
    ``"f16"`` and float32 for ``"f32"``.
    """
    vals = dequant_values_f32(blocks, scales).T
    if dtype == "bf16":
        return np.ascontiguousarray(f32_to_bf16(vals))
    if dtype == "f16":
        with np.errstate(over="ignore"):
            return np.ascontiguousarray(vals.astype(np.float16))
    if dtype == "f32":
        return np.ascontiguousarray(vals)
    raise ValueError(f"unsupported dtype {dtype!r}")


def dequantize_batch(blocks: np.ndarray, scales: np.ndarray, dtype: str = "bf16") -> np.ndarray:
    """Dequantize ``[n, out, G, 16]`` / ``[n, out, G]`` into ``[n, in, out]``."""
    if blocks.shape[:-1] != scales.shape:
        raise ValueError(f"MXFP4 block/scale shape mismatch: {blocks.shape=} {scales.shape=}")
    return np.stack([dequantize(blocks[i], scales[i], dtype) for i in range(blocks.shape[0])])
