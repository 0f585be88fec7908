"""Host side of the scaled-MFMA measurement (tests/native/fp4_mfma_probe.hip).

Packs checkpoint-layout MXFP4 weights and float activations into the operand
layout of v_mfma_scale_f32_16x16x128_f8f6f4 (A = E2M1 codes + E8M0 scales per
32 k, B = FP8 E4M3 codes + E8M0 scales per 32 k) and computes exact sums to
measure the instruction against.  Activations that do not fit one FP8 operand
are split into planes: plane p quantizes what planes 0 .. p-1 left over, each
32-value block with its own power-of-two scale, and the MFMA accumulates the
planes one after another.
"""

from __future__ import annotations

import numpy as np

from oracle.mxfp4 import FP4_VALUES

E4M3_MAX = 448.0


def e4m3_values() -> np.ndarray:
    """float64 value of every FP8 E4M3 (OCP "fn": no infinities) code; NaN at 0x7f and 0xff."""
    c = np.arange(256)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 15
    m = c & 7
    mag = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * 2.0 ** (e - 7.0))
    v = sign * mag
    v[(c & 0x7F) == 0x7F] = np.nan
    return v


_E4M3 = e4m3_values()
_POS = _E4M3[:0x7F]  # codes 0 .. 126, increasing


def e4m3_encode(v: np.ndarray) -> np.ndarray:
    """Round to nearest E4M3 code, ties to the even code; |v| must not exceed 448."""
    v = np.asarray(v, dtype=np.float64)
    a = np.abs(v)
    if (a > E4M3_MAX).any():
        raise ValueError("value beyond the E4M3 range")
    hi = np.clip(np.searchsorted(_POS, a, side="left"), 0, 0x7E)
    lo = np.maximum(hi - 1, 0)
    d_hi = _POS[hi] - a
    d_lo = a - _POS[lo]
    pick_lo = (d_lo < d_hi) | ((d_lo == d_hi) & (lo % 2 == 0))
    code = np.where(pick_lo, lo, hi).astype(np.uint8)
    return np.where((v < 0) & (code != 0), code | 0x80, code).astype(np.uint8)


def block_scales(r: np.ndarray) -> np.ndarray:
    """E8M0 exponent per 32-value block (last axis): the smallest power of two that brings the block's
    largest magnitude within 448.  An all-zero block gets 2^0."""
    m = np.abs(r).max(axis=-1)
    _, ex = np.frexp(np.where(m > 0, m / E4M3_MAX, 1.0))  # m / 448 = f * 2^ex, f in [0.5, 1)
    s = np.where(m > 0, ex, 0)
    s = np.where((m > 0) & (np.ldexp(1.0, s - 1) * E4M3_MAX >= m), s - 1, s)  # exact powers of two
    return np.clip(s, -127, 127).astype(np.int64)


def fp8_planes(x: np.ndarray, n_planes: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Split ``x [n, K]`` (K a multiple of 32) into ``n_planes`` scaled E4M3 planes.

    Returns codes ``[P, n, K]`` uint8, E8M0 scales ``[P, n, K / 32]`` uint8 and what is left over
    ``[n, K]`` float64 (``x`` minus the sum of the planes)."""
    r = np.asarray(x, dtype=np.float64).copy()
    n, k = r.shape
    codes = np.zeros((n_planes, n, k), np.uint8)
    scales = np.zeros((n_planes, n, k // 32), np.uint8)
    for p in range(n_planes):
        blk = r.reshape(n, k // 32, 32)
        s = block_scales(blk)
        c = e4m3_encode(blk / np.ldexp(1.0, s)[..., None])
        codes[p] = c.reshape(n, k)
        scales[p] = (s + 127).astype(np.uint8)
        r -= (_E4M3[c] * np.ldexp(1.0, s)[..., None]).reshape(n, k)
    return codes, scales, r


def plane_values(codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """float64 ``[n, K]`` value of planes ``[P, n, K]`` with scales ``[P, n, K / 32]``, summed over P."""
    p, n, k = codes.shape
    v = _E4M3[codes].reshape(p, n, k // 32, 32) * np.ldexp(1.0, scales.astype(np.int64) - 127)[..., None]
    return v.reshape(p, n, k).sum(axis=0)


def pad_groups(blocks: np.ndarray, scales: np.ndarray, groups: int) -> tuple[np.ndarray, np.ndarray]:
    """Zero codes (value 0, scale 2^0) appended so that the row has ``groups`` 32-value groups."""
    rows, g, _ = blocks.shape
    b = np.zeros((rows, groups, 16), np.uint8)
    s = np.full((rows, groups), 127, np.uint8)
    b[:, :g] = blocks
    s[:, :g] = scales
    return b, s


def pack_a(blocks: np.ndarray, scales: np.ndarray) -> tuple[np.ndarray, np.ndarray, int]:
    """Checkpoint rows ``[rows, G, 16]`` / ``[rows, G]`` -> ``[rows/16][steps][16][64]`` codes and
    ``[rows/16][steps][16][4]`` scales (G padded to a multiple of 4).  Returns (codes, scales, steps)."""
    rows, g, _ = blocks.shape
    if rows % 16:
        raise ValueError("rows must be a multiple of 16")
    steps = (g + 3) // 4
    b, s = pad_groups(blocks, scales, 4 * steps)
    codes = b.reshape(rows // 16, 16, steps, 64).transpose(0, 2, 1, 3)
    sc = s.reshape(rows // 16, 16, steps, 4).transpose(0, 2, 1, 3)
    return np.ascontiguousarray(codes), np.ascontiguousarray(sc), steps


def pack_b(codes: np.ndarray, scales: np.ndarray, steps: int) -> tuple[np.ndarray, np.ndarray]:
    """Planes ``[P, n, K]`` / ``[P, n, K/32]`` (n a multiple of 16) -> ``[n/16][steps][P][16][128]``
    codes and ``[n/16][steps][P][16][4]`` scales, K zero-padded to ``128 * steps``.

    Within a token's 128 bytes of a step, lane group g (bytes 32 g .. 32 g + 31) holds k = 16 g .. 16 g + 15
    followed by k = 64 + 16 g .. 64 + 16 g + 15 (the FP8 operand's layout), while the group's scale is
    that of k-block g (k = 32 g .. 32 g + 31), as for the FP4 operand."""
    p, n, k = codes.shape
    if n % 16:
        raise ValueError("tokens must be a multiple of 16")
    c = np.zeros((p, n, 128 * steps), np.uint8)
    s = np.full((p, n, 4 * steps), 127, np.uint8)
    c[..., :k] = codes
    s[..., :k // 32] = scales
    c = c.reshape(p, n, steps, 2, 4, 16).transpose(0, 1, 2, 4, 3, 5)  # [.., half, group, 16] -> [.., group, half, 16]
    c = c.reshape(p, n // 16, 16, steps, 128).transpose(1, 3, 0, 2, 4)
    s = s.reshape(p, n // 16, 16, steps, 4).transpose(1, 3, 0, 2, 4)
    return np.ascontiguousarray(c), np.ascontiguousarray(s)


def fp4_int(blocks: np.ndarray) -> np.ndarray:
    """2 x the E2M1 values of ``[rows, G, 16]`` as int64 ``[rows, G * 32]`` (low nibble first)."""
    lut = (2 * np.array(FP4_VALUES)).astype(np.int64)
    rows, g, _ = blocks.shape
    v = np.empty((rows, g, 32), np.int64)
    v[..., 0::2] = lut[blocks & 0xF]
    v[..., 1::2] = lut[blocks >> 4]
    return v.reshape(rows, g * 32)


def e4m3_int(codes: np.ndarray) -> np.ndarray:
    """2^9 x the E4M3 values as int64 (codes must not be NaN)."""
    c = codes.astype(np.int64)
    e = (c >> 3) & 15
    m = c & 7
    mag = np.where(e == 0, m, (8 + m) << np.maximum(e - 1, 0))
    return np.where(c & 0x80, -mag, mag)


def exact_block_sums(blocks: np.ndarray, a_scales: np.ndarray, codes: np.ndarray, b_scales: np.ndarray,
                     lo: int) -> tuple[np.ndarray, np.ndarray]:
    """Exact ``A @ B^T`` and ``|A| @ |B|^T`` for one 128-deep step (4 groups): A ``[rows, 4, 16]`` codes with
    scales ``[rows, 4]``, B ``[n, 128]`` E4M3 codes with scales ``[n, 4]``, every scale in ``[lo, lo + 14]``.

    Products are integers times 2^(-10 + 2 (lo - 127)); sums of up to 128 of them stay below 2^57, so int64
    holds them exactly.  Returns float64 ``[n, rows]`` pairs (each rounded once, relative 2^-53)."""
    a = fp4_int(blocks).reshape(-1, 4, 32) << (a_scales.astype(np.int64) - lo)[..., None]
    b = e4m3_int(codes).reshape(-1, 4, 32) << (b_scales.astype(np.int64) - lo)[..., None]
    a = a.reshape(a.shape[0], 128)
    b = b.reshape(b.shape[0], 128)
    unit = 2.0 ** (-10 + 2 * (lo - 127))
    return (b @ a.T).astype(np.float64) * unit, (np.abs(b) @ np.abs(a).T).astype(np.float64) * unit
