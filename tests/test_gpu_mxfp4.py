"""GPU parity: MXFP4 dequant and repack against the oracle (bit-exact)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import bf16_bits
from oracle import mxfp4 as omx
from klcquant_amd import ops, synth

pytestmark = pytest.mark.gpu


def all_pairs_matrix():
    """256 rows (row r uses scale byte r), one group: bytes pack codes 0..15 twice."""
    lo = np.arange(16, dtype=np.uint8) % 16
    hi = (np.arange(16, dtype=np.uint8) * 7 + 3) % 16
    row = (hi << 4) | lo
    blocks = np.tile(row, (256, 1)).reshape(256, 1, 16)
    scales = np.arange(256, dtype=np.uint8).reshape(256, 1)
    return blocks, scales


def same_bits_nan_aware(got, want, kind):
    if kind == "bf16":
        g = got.astype(np.uint32) << 16
        w = want.astype(np.uint32) << 16
        gn = ((g & 0x7FFFFFFF) > 0x7F800000)
        wn = ((w & 0x7FFFFFFF) > 0x7F800000)
    elif kind == "f16":
        g = got.view(np.uint16).astype(np.uint32)
        w = want.view(np.uint16).astype(np.uint32)
        gn = ((g & 0x7FFF) > 0x7C00)
        wn = ((w & 0x7FFF) > 0x7C00)
    else:
        g = got.view(np.uint32)
        w = want.view(np.uint32)
        gn = ((g & 0x7FFFFFFF) > 0x7F800000)
        wn = ((w & 0x7FFFFFFF) > 0x7F800000)
    assert np.array_equal(gn, wn), f"NaN pattern differs at {np.argwhere(gn != wn)[:5]}"
    ok = gn | (g == w)
    bad = np.argwhere(~ok)
    assert bad.size == 0, f"{bad.shape[0]} mismatches, first {bad[:5].tolist()}"


@pytest.mark.parametrize("dtype,kind", [(torch.bfloat16, "bf16"), (torch.float16, "f16"), (torch.float32, "f32")])
def test_dequant_all_code_scale_pairs(gpu, dtype, kind):
    blocks, scales = all_pairs_matrix()
    got = ops.mxfp4_dequant(torch.from_numpy(blocks).to(gpu), torch.from_numpy(scales).to(gpu), dtype)
    torch.cuda.synchronize()
    assert got.shape == (32, 256)
    g = bf16_bits(got) if kind == "bf16" else got.cpu().numpy()
    want = omx.dequantize(blocks, scales, kind)
    same_bits_nan_aware(g, want, kind)


@pytest.mark.parametrize("n_mat,out_dim,groups", [(3, 128, 6), (2, 192, 90), (1, 40, 3), (2, 72, 5), (1, 36, 3),
                                                   (2, 3080, 2), (1, 4096, 3), (1, 4104, 2), (2, 2880, 7),
                                                   (1, 1600, 5)])
def test_dequant_seeded_matches_oracle(gpu, n_mat, out_dim, groups):
    blocks, scales = synth.mxfp4_expert_tensors(11, 12, n_mat, out_dim, groups * 32, 0, 255)
    got = ops.mxfp4_dequant(torch.from_numpy(blocks).to(gpu), torch.from_numpy(scales).to(gpu), torch.bfloat16)
    torch.cuda.synchronize()
    want = omx.dequantize_batch(blocks, scales, "bf16")
    same_bits_nan_aware(bf16_bits(got), want, "bf16")


def test_dequant_single_matrix_shape_and_errors(gpu):
    blocks, scales = synth.mxfp4_expert_tensors(1, 2, 1, 64, 64)
    b = torch.from_numpy(blocks[0]).to(gpu)
    s = torch.from_numpy(scales[0]).to(gpu)
    out = ops.mxfp4_dequant(b, s, torch.bfloat16)
    assert out.shape == (64, 64)
    with pytest.raises(ValueError, match="shape mismatch"):
        ops.mxfp4_dequant(b, s[:, :1])


@pytest.mark.parametrize("rows,groups", [(128, 6), (5760, 90), (64, 1)])
def test_pack_roundtrip_through_packed_dequant(gpu, rows, groups):
    n_mat = 2
    blocks, scales = synth.mxfp4_expert_tensors(21, 22, n_mat, rows, groups * 32, 0, 255)
    b = torch.from_numpy(blocks).to(gpu)
    s = torch.from_numpy(scales).to(gpu)
    packed = ops.mxfp4_pack(b, s)
    assert packed.shape == (n_mat, ops.packed_bytes(rows, groups))
    direct = ops.mxfp4_dequant(b, s, torch.float32)
    via_packed = ops.mxfp4_dequant_packed(packed, rows, groups, torch.float32)
    torch.cuda.synchronize()
    d = direct.cpu().numpy().view(np.uint32)
    p = via_packed.cpu().numpy().view(np.uint32)
    nan = (d & 0x7FFFFFFF) > 0x7F800000
    assert np.array_equal(nan, (p & 0x7FFFFFFF) > 0x7F800000)
    assert np.array_equal(d[~nan], p[~nan])


@pytest.mark.parametrize("groups", [5, 37])
def test_pack_layout_positions(gpu, groups):
    """Block byte (row r, group g, byte j) lands at tile/g/row/j; the scale of (r, g) at byte s % 8 of the
    8-byte word (tile, s // 8, row in tile, g % 4), s = g // 4."""
    rows = 128
    blocks, scales = synth.mxfp4_expert_tensors(31, 32, 1, rows, groups * 32, 0, 255)
    packed = ops.mxfp4_pack(torch.from_numpy(blocks).to(gpu), torch.from_numpy(scales).to(gpu)).cpu().numpy()[0]
    rec = ((groups + 3) // 4 + 7) // 8 * 8  # scale bytes per (row, group % 4): one per 4-group step, padded to 8
    blk_bytes = rows // 64 * groups * 1024
    assert packed.size == blk_bytes + rows * 4 * rec

    def word(r, p, q):
        t, rr = divmod(r, 64)
        return blk_bytes + t * 64 * 4 * rec + ((p * 64 + rr) * 4 + q) * 8

    for r in (0, 1, 63, 64, 127):
        for g in range(groups):
            t, rr = divmod(r, 64)
            off = (t * groups + g) * 1024 + rr * 16
            assert np.array_equal(packed[off:off + 16], blocks[0, r, g])
            s = g // 4
            assert packed[word(r, s // 8, g % 4) + s % 8] == scales[0, r, g]
        # bytes of steps past the last group are zero
        for q in range(4):
            for s in range(rec):
                if 4 * s + q >= groups:
                    assert packed[word(r, s // 8, q) + s % 8] == 0
    # every scale byte is accounted for: the scale area is exactly the words above
    seen = np.zeros(rows * 4 * rec, dtype=bool)
    for r in range(rows):
        for q in range(4):
            for s in range(rec):
                seen[word(r, s // 8, q) + s % 8 - blk_bytes] = True
    assert seen.all()


def test_synth_fill_matches_host_generator(gpu):
    n = 4099
    for seed in (0, 4, 1000 + 4, 2**63 + 5):
        raw = ops.synth_fill(torch.empty(n, dtype=torch.uint8, device=gpu), seed, 0).cpu().numpy()
        assert np.array_equal(raw, synth.random_bytes(seed, n))
        ints = ops.synth_fill(torch.empty(n, dtype=torch.uint8, device=gpu), seed, 1, 118, 124).cpu().numpy()
        assert np.array_equal(ints, synth.random_ints(seed, n, 118, 124).astype(np.uint8))
