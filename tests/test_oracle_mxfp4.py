"""Pins the oracle's MXFP4 dequant against the OCP MX v1.0 definitions.

E2M1: sign bit 3, exponent bits 2-1 (bias 1), mantissa bit 0; exponent 0 is
subnormal (0.M * 2^0).  E8M0: 2^(e - 127).  The reference evaluates
``FP4_VALUES[c] * float32(2^(e - 127))`` in float32 and rounds to the target
dtype (mxfp4_expert.py:367-377), so 2^128 (e = 255) is inf and 0 * inf NaN.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import mxfp4
from oracle.numerics import bf16_to_f32

# The reference's table, mxfp4_expert.py:17-34 (the path's only known-answer table).
REFERENCE_FP4_VALUES = [+0.0, +0.5, +1.0, +1.5, +2.0, +3.0, +4.0, +6.0,
                        -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]


def e2m1_spec(code: int) -> float:
    sign = -1.0 if code & 8 else 1.0
    exp = (code >> 1) & 3
    man = code & 1
    if exp == 0:
        return sign * man * 0.5
    return sign * math.ldexp(1.0 + man / 2.0, exp - 1)


def expected_f32(code: int, e: int) -> float:
    """float32(E2M1 * float32(2^(e-127))) per IEEE, computed in float64."""
    pow2 = math.inf if e == 255 else math.ldexp(1.0, e - 127)
    v = e2m1_spec(code) * pow2 if not (pow2 == math.inf and e2m1_spec(code) == 0.0) else math.nan
    with np.errstate(over="ignore"):
        return float(np.float32(v))


def test_lut_matches_reference_table_and_spec():
    assert mxfp4.FP4_VALUES == REFERENCE_FP4_VALUES
    for c in range(16):
        v = e2m1_spec(c)
        assert v == REFERENCE_FP4_VALUES[c]
        assert math.copysign(1.0, v) == math.copysign(1.0, REFERENCE_FP4_VALUES[c])


def all_pairs():
    blocks = np.zeros((256, 1, 16), dtype=np.uint8)
    for b in range(16):
        blocks[:, 0, b] = (b << 4) | b  # codes b (low) and b (high)
    scales = np.arange(256, dtype=np.uint8).reshape(256, 1)
    return blocks, scales


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_all_code_scale_pairs_exact(dtype):
    blocks, scales = all_pairs()
    out = mxfp4.dequantize(blocks, scales, dtype)  # [32, 256]
    got = out if dtype == "f32" else bf16_to_f32(out)
    for e in range(256):
        for code in range(16):
            for col in (2 * code, 2 * code + 1):
                want = expected_f32(code, e)
                g = float(got[col, e])
                if math.isnan(want):
                    assert math.isnan(g), (e, code)
                else:
                    assert g == want and math.copysign(1, g) == math.copysign(1, want), (e, code, g, want)


def test_special_cases():
    blocks, scales = all_pairs()
    b = mxfp4.dequantize(blocks, scales, "bf16")
    # e = 0: subnormals survive in bfloat16 (6 * 2^-127)
    assert bf16_to_f32(b[2 * 7, 0]) == np.float32(6.0 * 2.0 ** -127)
    # e = 254: |value| >= 2 overflows to inf, 1.5 * 2^127 does not
    assert np.isinf(bf16_to_f32(b[2 * 4, 254])) and bf16_to_f32(b[2 * 3, 254]) == np.float32(1.5 * 2.0 ** 127)
    # e = 255: zero codes give NaN (0 * inf), others +-inf
    assert np.isnan(bf16_to_f32(b[0, 255])) and np.isnan(bf16_to_f32(b[2 * 8, 255]))
    assert bf16_to_f32(b[2, 255]) == np.inf and bf16_to_f32(b[2 * 9, 255]) == -np.inf
    # -0 keeps its sign
    assert b[2 * 8, 127] == 0x8000


def test_float16_rounding_cases():
    blocks, scales = all_pairs()
    h = mxfp4.dequantize(blocks, scales, "f16").view(np.uint16)
    assert h[2 * 7, 127 + 16] == 0x7C00          # 6 * 2^16 > 65504 -> inf
    assert h[2 * 1, 127 - 25] == 0x0000          # 0.5 * 2^-25 = 2^-26 < half an ulp -> 0
    assert h[2 * 2, 127 - 24] == 0x0001          # 1.0 * 2^-24: smallest subnormal
    assert h[2 * 3, 127 - 24] == 0x0002          # 1.5 * 2^-24: tie -> even
    assert h[2 * 1, 127 - 24] == 0x0000          # 0.5 * 2^-24: tie -> even (0)
    assert h[2 * 5, 127] == 0x4200               # 3.0


@pytest.mark.parametrize("half", [0, 1])
def test_layout_single_nibble_probe(half):
    out_dim, groups = 5, 3
    for o in range(out_dim):
        for g in range(groups):
            for byte in range(16):
                blocks = np.zeros((out_dim, groups, 16), dtype=np.uint8)
                scales = np.full((out_dim, groups), 127, dtype=np.uint8)
                blocks[o, g, byte] = 0x0F << (4 * half)
                m = mxfp4.dequantize(blocks, scales, "f32")
                assert m.shape == (groups * 32, out_dim)
                nz = np.argwhere(m != 0)
                assert nz.tolist() == [[g * 32 + 2 * byte + half, o]]
                assert m[g * 32 + 2 * byte + half, o] == -6.0


def test_scale_applies_per_row_and_group():
    blocks = np.full((2, 2, 16), 0x22, dtype=np.uint8)  # every code 2 (1.0)
    scales = np.array([[127, 128], [126, 130]], dtype=np.uint8)
    m = mxfp4.dequantize(blocks, scales, "f32")
    assert (m[:32, 0] == 1.0).all() and (m[32:, 0] == 2.0).all()
    assert (m[:32, 1] == 0.5).all() and (m[32:, 1] == 8.0).all()


def test_shape_mismatch_raises():
    with pytest.raises(ValueError, match="shape mismatch"):
        mxfp4.dequantize(np.zeros((4, 2, 16), np.uint8), np.zeros((4, 3), np.uint8))
