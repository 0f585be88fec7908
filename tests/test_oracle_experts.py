"""Pins the oracle's SwiGLU, expert GEMVs, combine and bias-only fallback."""

from __future__ import annotations

import math
from fractions import Fraction

import numpy as np

from klcquant_amd import synth
from oracle import experts, mxfp4
from oracle.numerics import bf16_to_f32, f32_to_bf16
from oracle.rmsnorm import residual_add, rms_norm


def swiglu_f64(gate, up, limit=7.0, alpha=1.702):
    g = min(gate, limit)
    u = max(min(up, limit), -limit)
    return (u + 1.0) * g / (1.0 + math.exp(-alpha * g))


def test_swiglu_clamps_and_interleave():
    gu = np.array([100.0, 100.0, 100.0, -100.0, 0.0, 3.0, 2.0, -1.0, -100.0, 5.0, 6.5, 6.5], dtype=np.float32)
    out = experts.swiglu(gu)
    assert out.shape == (6,)
    # gate clamped from above only, up clamped both ways, interleaved (gate, up) pairs
    want = [swiglu_f64(100, 100), swiglu_f64(100, -100), 0.0, 0.0, swiglu_f64(-100, 5), swiglu_f64(6.5, 6.5)]
    np.testing.assert_allclose(out.astype(np.float64), want, rtol=2e-6, atol=1e-30)
    assert out[3] == 0.0  # up = -1 -> (up + 1) = 0
    # swapping gate and up changes the answer: the interleave is not symmetric
    assert experts.swiglu(np.array([1.0, 3.0], np.float32))[0] != experts.swiglu(np.array([3.0, 1.0], np.float32))[0]


def test_swiglu_nan_propagates():
    assert np.isnan(experts.swiglu(np.array([np.nan, 1.0], np.float32))).all()
    assert np.isnan(experts.swiglu(np.array([1.0, np.nan], np.float32))).all()


def test_expert_ffn_against_exact_rational_gemv():
    hidden, inter = 64, 32
    x = bf16_to_f32(synth.random_normal_bf16(21, 2 * hidden).reshape(2, hidden))
    gub, gus = synth.mxfp4_expert_tensors(22, 23, 1, 2 * inter, hidden)
    db, ds = synth.mxfp4_expert_tensors(24, 25, 1, hidden, inter)
    wgu = mxfp4.dequantize(gub[0], gus[0], "f32")
    wd = mxfp4.dequantize(db[0], ds[0], "f32")
    gub_bits = synth.random_normal_bf16(26, 2 * inter, 0, 0.01)
    db_bits = synth.random_normal_bf16(27, hidden, 0, 0.01)
    gated, out = experts.expert_ffn(x, wgu, gub_bits, wd, db_bits, 7.0, "fp32")
    for t in range(2):
        gu = [np.float32(np.float32(float(sum(Fraction(float(x[t, i])) * Fraction(float(wgu[i, j]))
                                              for i in range(hidden)))) + bf16_to_f32(gub_bits[j:j + 1])[0])
              for j in range(2 * inter)]
        g = experts.swiglu(np.array(gu, dtype=np.float32))
        assert np.array_equal(g, gated[t])
        o = [np.float32(np.float32(float(sum(Fraction(float(g[i])) * Fraction(float(wd[i, h])) for i in range(inter))))
                        + bf16_to_f32(db_bits[h:h + 1])[0]) for h in range(hidden)]
        assert np.array_equal(np.array(o, np.float32), out[t])


def test_bf16_precision_rounds_matmul_inputs_and_outputs():
    hidden, inter = 64, 32
    x = bf16_to_f32(synth.random_normal_bf16(31, hidden).reshape(1, hidden))
    gub, gus = synth.mxfp4_expert_tensors(32, 33, 1, 2 * inter, hidden)
    db, ds = synth.mxfp4_expert_tensors(34, 35, 1, hidden, inter)
    wgu = mxfp4.dequantize(gub[0], gus[0], "f32")
    wd = mxfp4.dequantize(db[0], ds[0], "f32")
    zb = np.zeros(2 * inter, np.uint16)
    zd = np.zeros(hidden, np.uint16)
    g32, o32 = experts.expert_ffn(x, wgu, zb, wd, zd, 7.0, "fp32")
    g16, o16 = experts.expert_ffn(x, wgu, zb, wd, zd, 7.0, "bf16")
    # bf16 mode: the down result (zero bias) is a bfloat16 value
    assert np.array_equal(bf16_to_f32(f32_to_bf16(o16)), o16)
    assert not np.array_equal(o16, o32)
    np.testing.assert_allclose(o16, o32, rtol=0.05, atol=0.5)


def test_combine_accumulates_in_order_in_bfloat16():
    outs = np.array([[[256.0], [1.0], [-256.0]]], dtype=np.float32)  # [B=1, k=3, H=1]
    ones = f32_to_bf16(np.ones((1, 3), np.float32))
    # 256 + 1 = 257 rounds (tie) to 256 in bfloat16, then - 256 = 0; another order would give 1
    assert bf16_to_f32(experts.combine(outs, ones)).tolist() == [[0.0]]
    assert bf16_to_f32(experts.combine(outs[:, ::-1, :].copy(), ones)).tolist() == [[1.0]]


def test_combine_single_expert_weight_one_is_bf16_of_output():
    eo = synth.random_normal_f32(41, 3 * 50, 0, 30).reshape(3, 1, 50)
    w = f32_to_bf16(np.ones((3, 1), np.float32))
    assert np.array_equal(experts.combine(eo, w), f32_to_bf16(eo[:, 0, :]))


def test_combine_zero_weights_gives_zero():
    eo = synth.random_normal_f32(42, 2 * 4 * 8, 0, 30).reshape(2, 4, 8)
    w = np.zeros((2, 4), np.uint16)
    assert (bf16_to_f32(experts.combine(eo, w)) == 0).all()


def test_bias_only_closed_form():
    bias = f32_to_bf16(np.array([[1.0, 2.0], [4.0, -8.0], [0.5, 0.25]], np.float32))
    ids = np.array([[1, 2]])
    w = f32_to_bf16(np.array([[0.75, 0.25]], np.float32))
    got = bf16_to_f32(experts.bias_only(bias, ids, w))
    assert got.tolist() == [[4.0 * 0.75 + 0.5 * 0.25, -8.0 * 0.75 + 0.25 * 0.25]]


def test_rms_norm_and_residual():
    x = f32_to_bf16(np.array([[3.0, 4.0]], np.float32))
    w = f32_to_bf16(np.array([1.0, 2.0], np.float32))
    # mean(x^2) = 12.5, rsqrt ~ 0.28284 -> bf16 0.28320 (0x3E91), then bf16 multiplies
    r = bf16_to_f32(f32_to_bf16(np.array([1.0 / math.sqrt(12.5 + 1e-5)], np.float32)))[0]
    want = [bf16_to_f32(f32_to_bf16(np.array([3.0 * r], np.float32)))[0] * 1.0,
            bf16_to_f32(f32_to_bf16(np.array([4.0 * r], np.float32)))[0] * 2.0]
    assert bf16_to_f32(rms_norm(x, w)).tolist() == [[float(want[0]), float(want[1])]]
    a = f32_to_bf16(np.array([[256.0]], np.float32))
    b = f32_to_bf16(np.array([[1.0]], np.float32))
    assert bf16_to_f32(residual_add(a, b)).tolist() == [[256.0]]
