"""The seeded input generator: SplitMix64 reference sequence and distributions."""

from __future__ import annotations

import numpy as np

from klcquant_amd import synth
from oracle.numerics import f32_to_bf16


def test_splitmix64_published_sequence():
    # SplitMix64 (Vigna) started from state 1234567
    want = [6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431,
            16408922859458223821]
    assert [int(v) for v in synth.draws_from_state(1234567, 0, 5)] == want
    # counter form: any window equals the sequential stream
    assert list(synth.draws_from_state(1234567, 3, 2)) == list(synth.draws_from_state(1234567, 0, 5)[3:])


def test_seeded_draws_and_bytes():
    d = synth.draws(42, 0, 4)
    assert int(d[0]) == synth.mix64_int(synth.mix64_int(42) + 0x9E3779B97F4A7C15)
    b = synth.random_bytes(42, 29)
    assert np.array_equal(b[:8], d[:1].view(np.uint8))
    assert np.array_equal(b[24:29], d[3:4].view(np.uint8)[:5])


def test_integer_range_and_uniformity():
    v = synth.random_ints(7, 70_000, 118, 124)
    assert v.min() == 118 and v.max() == 124
    counts = np.bincount(v - 118, minlength=7)
    assert (np.abs(counts - 10_000) < 500).all()


def test_normals():
    z = synth.random_normal_f32(9, 200_000, 0.0, 2.0)
    assert abs(float(z.mean())) < 0.02 and abs(float(z.std()) - 2.0) < 0.02
    assert np.array_equal(synth.random_normal_bf16(9, 1000, 0, 2.0), f32_to_bf16(z[:1000]))
    assert np.array_equal(synth.f32_to_bf16_bits(z), f32_to_bf16(z))


def test_mxfp4_tensor_shapes_and_codes():
    blocks, scales = synth.mxfp4_expert_tensors(1, 2, 3, 64, 96)
    assert blocks.shape == (3, 64, 3, 16) and scales.shape == (3, 64, 3)
    nib = np.concatenate([(blocks & 15).ravel(), (blocks >> 4).ravel()])
    assert set(np.unique(nib)) == set(range(16))
    assert scales.min() >= 118 and scales.max() <= 124


def test_tensor_seed_layout():
    assert synth.tensor_seed(2, "gate_up_blocks", 3) == 2000 + 300 + 4


def test_expert_slice_equals_the_full_tensors():
    blocks, scales = synth.mxfp4_expert_tensors(41, 42, 5, 64, 96)
    for e in (0, 3, 4):
        b, s = synth.mxfp4_expert_slice(41, 42, e, 64, 96)
        assert np.array_equal(b, blocks[e]) and np.array_equal(s, scales[e])
