"""Host side of the scaled-MFMA measurement: FP8 E4M3 coding, planes, operand packing, exact sums."""

from __future__ import annotations

import math

import numpy as np

import mx_operands as mx
from oracle import mxfp4 as omx
from oracle.numerics import bf16_to_f32
from klcquant_amd import synth


def test_e4m3_table_special_values():
    v = mx.e4m3_values()
    assert v[0x7E] == 448.0 and v[0xFE] == -448.0
    assert v[0x38] == 1.0 and v[0x08] == 2.0 ** -6 and v[0x01] == 2.0 ** -9 and v[0x07] == 7 * 2.0 ** -9
    assert np.isnan(v[0x7F]) and np.isnan(v[0xFF])
    finite = v[~np.isnan(v)]
    assert np.unique(finite).size == 253  # 254 codes, +0 and -0 equal


def test_e4m3_encode_round_trip_and_ties():
    v = mx.e4m3_values()
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F and c != 0x80])
    assert np.array_equal(mx.e4m3_encode(v[codes]), codes)
    assert mx.e4m3_encode(np.array([1.0625]))[0] == 0x38  # halfway 1 .. 1.125: even code
    assert mx.e4m3_encode(np.array([1.1875]))[0] == 0x3A  # halfway 1.125 .. 1.25: even code
    assert mx.e4m3_encode(np.array([-1.2]))[0] == 0xBA
    assert mx.e4m3_encode(np.array([2.0 ** -10]))[0] == 0x00  # halfway 0 .. 2^-9: even code
    rng = np.random.default_rng(3)
    x = rng.uniform(-448, 448, 20000)
    c = mx.e4m3_encode(x)
    fin = np.sort(np.unique(v[~np.isnan(v)]))
    nearest = fin[np.argmin(np.abs(fin[None, :] - x[:, None]), axis=1)]
    assert np.array_equal(np.abs(v[c]), np.abs(nearest))


def test_block_scales_bring_the_maximum_within_range():
    rng = np.random.default_rng(5)
    r = rng.standard_normal((500, 32)) * np.ldexp(1.0, rng.integers(-20, 20, (500, 1)))
    r[0] = 0
    r[1, 0] = 448.0  # exactly at the limit: scale 2^0
    r[2, 0] = 896.0
    s = mx.block_scales(r)
    m = np.abs(r).max(axis=1)
    assert s[0] == 0 and s[1] == 0 and s[2] == 1
    nz = m > 0
    assert (m[nz] / np.ldexp(1.0, s[nz]) <= 448).all()
    assert (m[nz] / np.ldexp(1.0, s[nz] - 1) > 448).all()


def test_planes_reconstruct_bf16_activations():
    x = bf16_to_f32(synth.random_normal_bf16(11, 64 * 2880)).astype(np.float64).reshape(64, 2880)
    prev = np.abs(x).reshape(64, 90, 32).max(axis=2)
    for planes in (1, 2, 3):
        c, s, r = mx.fp8_planes(x, planes)
        assert np.array_equal(mx.plane_values(c, s) + r, x)
        # each plane leaves at most 2^-4 of its block's largest value (E4M3 keeps 4 significant bits)
        blk = np.abs(r).reshape(64, 90, 32).max(axis=2)
        assert (blk <= prev * 2.0 ** (-4 * planes)).all(), planes


def test_packed_operands_follow_the_lane_layout():
    """Walk the packed arrays the way the probe kernel's lanes address them."""
    rng = np.random.default_rng(7)
    rows, g, n, planes = 32, 6, 32, 2
    blocks = rng.integers(0, 256, (rows, g, 16), dtype=np.uint8)
    a_sc = rng.integers(100, 150, (rows, g)).astype(np.uint8)
    codes = rng.integers(0, 256, (planes, n, g * 32), dtype=np.uint8)
    b_sc = rng.integers(100, 150, (planes, n, g)).astype(np.uint8)
    ac, asc, steps = mx.pack_a(blocks, a_sc)
    bc, bsc = mx.pack_b(codes, b_sc, steps)
    assert steps == 2
    fa, fas, fb, fbs = ac.ravel(), asc.ravel(), bc.ravel(), bsc.ravel()
    for rt in range(rows // 16):
        for s in range(steps):
            for lane in range(64):
                r, kb = lane % 16, lane // 16
                grp = 4 * s + kb
                ts = rt * steps + s
                a_bytes = fa[(ts * 16 + r) * 64 + kb * 16:][:16]
                want = blocks[16 * rt + r, grp] if grp < g else np.zeros(16, np.uint8)
                assert np.array_equal(a_bytes, want)
                assert fas[(ts * 16 + r) * 4 + kb] == (a_sc[16 * rt + r, grp] if grp < g else 127)
    for ct in range(n // 16):
        for s in range(steps):
            for p in range(planes):
                tsp = (ct * steps + s) * planes + p
                for lane in range(64):
                    r, kb = lane % 16, lane // 16
                    grp = 4 * s + kb
                    b_bytes = fb[(tsp * 16 + r) * 128 + kb * 32:][:32]
                    row = np.zeros(128 * steps, np.uint8)
                    row[:32 * g] = codes[p, 16 * ct + r]
                    k0 = 128 * s + 16 * kb
                    want = np.concatenate([row[k0:k0 + 16], row[k0 + 64:k0 + 80]])
                    assert np.array_equal(b_bytes, want)
                    assert fbs[(tsp * 16 + r) * 4 + kb] == (b_sc[p, 16 * ct + r, grp] if grp < g else 127)


def test_exact_block_sums_against_fsum():
    rng = np.random.default_rng(9)
    rows, n = 8, 8
    blocks = rng.integers(0, 256, (rows, 4, 16), dtype=np.uint8)
    a_sc = rng.integers(120, 135, (rows, 4)).astype(np.uint8)
    codes = rng.integers(0, 256, (n, 128), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x7E
    b_sc = rng.integers(120, 135, (n, 4)).astype(np.uint8)
    exact, mag = mx.exact_block_sums(blocks, a_sc, codes, b_sc, 120)
    a = omx.dequant_values_f32(blocks, a_sc).astype(np.float64)
    b = (mx.e4m3_values()[codes].reshape(n, 4, 32) * np.ldexp(1.0, b_sc.astype(int) - 127)[..., None]).reshape(n, 128)
    for t in range(n):
        for j in range(rows):
            terms = b[t] * a[j]
            assert exact[t, j] == math.fsum(terms)
            assert mag[t, j] == math.fsum(np.abs(terms))
