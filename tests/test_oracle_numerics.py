"""Pins the oracle's float32 -> bfloat16 rounding (round to nearest, ties to even)."""

from __future__ import annotations

import numpy as np

from oracle.numerics import bf16_to_f32, bf16_ulp_distance, f32_to_bf16


def bits_f32(u: int) -> np.ndarray:
    return np.array([u], dtype=np.uint32).view(np.float32)


def test_hand_worked_patterns():
    cases = {
        0x3F800000: 0x3F80,  # 1.0
        0x3F808000: 0x3F80,  # 1 + 2^-8: tie, low bit 0 -> down
        0x3F818000: 0x3F82,  # 1 + 3*2^-8: tie, low bit 1 -> up to even
        0x3F808001: 0x3F81,  # just above the tie -> up
        0x3F807FFF: 0x3F80,  # just below the tie -> down
        0x7F7F7FFF: 0x7F7F,  # largest finite bf16 stays
        0x7F7F8000: 0x7F80,  # tie above the largest finite -> even = inf
        0x7F800000: 0x7F80,  # +inf
        0xFF800000: 0xFF80,  # -inf
        0x80000000: 0x8000,  # -0
        0x00000001: 0x0000,  # smallest float32 subnormal rounds to +0
        0x00008000: 0x0000,  # tie at the bottom -> even (0)
        0x00018000: 0x0002,  # tie -> even
    }
    for src, want in cases.items():
        assert int(f32_to_bf16(bits_f32(src))[0]) == want, hex(src)


def test_nan_stays_nan():
    for src in (0x7FC00000, 0x7F800001, 0xFFFFFFFF, 0x7F80FFFF):
        out = int(f32_to_bf16(bits_f32(src))[0])
        assert (out & 0x7FFF) > 0x7F80, hex(src)


def test_every_bf16_pattern_round_trips():
    allbits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = (allbits & 0x7FFF) <= 0x7F80
    back = f32_to_bf16(bf16_to_f32(allbits))
    assert np.array_equal(back[finite], allbits[finite])


def test_nearest_and_ties_to_even_on_random_floats():
    rng = np.random.default_rng(7)
    u = rng.integers(0, 0x7F7F0000, size=200_000, dtype=np.uint64).astype(np.uint32)
    x = u.view(np.float32).astype(np.float64)
    r = f32_to_bf16(u.view(np.float32))
    lo = bf16_to_f32(r).astype(np.float64)
    nxt = bf16_to_f32((r.astype(np.uint32) + 1).astype(np.uint16)).astype(np.float64)
    prv = bf16_to_f32(np.maximum(r.astype(np.int64) - 1, 0).astype(np.uint16)).astype(np.float64)
    err = np.abs(x - lo)
    assert (err <= np.abs(x - nxt)).all() and (err <= np.abs(x - prv)).all()
    ties = (err == np.abs(x - nxt)) | ((err == np.abs(x - prv)) & (r > 0))
    assert ((r[ties] & 1) == 0).all()


def test_ulp_distance():
    assert bf16_ulp_distance(np.array([0x3F80]), np.array([0x3F81]))[0] == 1
    assert bf16_ulp_distance(np.array([0x0000]), np.array([0x8000]))[0] == 0
    assert bf16_ulp_distance(np.array([0x0001]), np.array([0x8001]))[0] == 2
