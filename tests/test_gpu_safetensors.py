"""The shard reader's device copy (klc_st_copy_rows_to_device) on the GPU.

Expected bytes are the host rows read from the same mapping (pinned against
the safetensors library on the CPU); the device copy must match them byte for
byte whether the range fits one staging half or wraps both halves many times.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from klcquant_amd import _native
from klcquant_amd.safetensors_shard import SafetensorShard

pytestmark = pytest.mark.gpu

safetensors_torch = pytest.importorskip("safetensors.torch")


@pytest.fixture(scope="module")
def shard_path(tmp_path_factory):
    g = torch.Generator().manual_seed(5)
    tensors = {
        # 3 rows of 6.0 MB: one row spans two 4 MiB staging halves
        "big.blocks": torch.randint(0, 256, (3, 6_000_000), generator=g, dtype=torch.uint8),
        "odd.bf16": torch.randn(7, 50_001, generator=g).to(torch.bfloat16),
        "tiny.u8": torch.arange(5, dtype=torch.uint8).reshape(5, 1),
    }
    path = tmp_path_factory.mktemp("st") / "shard.safetensors"
    safetensors_torch.save_file(tensors, str(path))
    return path


@pytest.mark.parametrize("name,first,count", [("big.blocks", 0, 3), ("big.blocks", 1, 1), ("odd.bf16", 2, 5),
                                              ("tiny.u8", 4, 1), ("tiny.u8", 5, 0)])
def test_copy_rows_to_device_matches_host_rows(gpu, shard_path, name, first, count):
    with SafetensorShard(shard_path) as shard:
        want = shard.read_rows(name, first, count)
        side = torch.cuda.Stream(gpu)
        got = shard.copy_rows_to_device(name, first, count, gpu, side)
        torch.cuda.synchronize(gpu)
        assert got.device.type == "cuda" and got.dtype == want.dtype and got.shape == want.shape
        assert torch.equal(got.cpu().view(torch.uint8), want.view(torch.uint8))


def test_minimal_staging_wraps_many_times(gpu, shard_path):
    """8 KiB of staging: the 700 KB range takes 171 alternating chunks."""
    with SafetensorShard(shard_path) as shard:
        want = shard.read_rows("odd.bf16", 0, 7).view(torch.uint8).reshape(-1)
        staging = torch.empty(8192, dtype=torch.uint8, pin_memory=True)
        dst = torch.full((want.numel() + 64,), 0xA5, dtype=torch.uint8, device=gpu)
        stream = torch.cuda.current_stream(gpu)
        _native.call("klc_st_copy_rows_to_device", shard._h(), b"odd.bf16", 0, 7,
                     ctypes.c_void_p(staging.data_ptr()), staging.numel(), ctypes.c_void_p(dst.data_ptr() + 32),
                     ctypes.c_void_p(stream.cuda_stream))
        host = dst.cpu()
        assert torch.equal(host[32:32 + want.numel()], want)
        assert (host[:32] == 0xA5).all() and (host[32 + want.numel():] == 0xA5).all()


def test_small_staging_is_rejected(gpu, shard_path):
    with SafetensorShard(shard_path) as shard:
        staging = torch.empty(4096, dtype=torch.uint8, pin_memory=True)
        dst = torch.empty(16, dtype=torch.uint8, device=gpu)
        with pytest.raises(_native.KlcError) as exc:
            _native.call("klc_st_copy_rows_to_device", shard._h(), b"tiny.u8", 0, 5,
                         ctypes.c_void_p(staging.data_ptr()), staging.numel(), ctypes.c_void_p(dst.data_ptr()),
                         ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream))
        assert exc.value.status == -1
        assert np.array_equal(shard.read_rows("tiny.u8", 0, 5).numpy().ravel(), np.arange(5))


@pytest.mark.parametrize("staging_bytes", [8192, 5 << 20, 64 << 20])
def test_batch_matches_host_rows(gpu, shard_path, staging_bytes):
    """Several ranges (one empty) through one slot ring of the given size."""
    reqs = [("big.blocks", 1, 2), ("tiny.u8", 0, 0), ("odd.bf16", 3, 4), ("tiny.u8", 2, 3), ("big.blocks", 0, 1)]
    with SafetensorShard(shard_path) as shard:
        want = [shard.read_rows(*r) for r in reqs]
        outs = [torch.full((w.numel() * w.element_size() + 64,), 0x5A, dtype=torch.uint8, device=gpu) for w in want]
        n = len(reqs)
        names = (ctypes.c_char_p * n)(*(r[0].encode() for r in reqs))
        firsts = (ctypes.c_int64 * n)(*(r[1] for r in reqs))
        counts = (ctypes.c_int64 * n)(*(r[2] for r in reqs))
        dsts = (ctypes.c_void_p * n)(*(o.data_ptr() + 32 for o in outs))
        staging = torch.empty(staging_bytes, dtype=torch.uint8, pin_memory=True)
        stream = torch.cuda.current_stream(gpu)
        _native.call("klc_st_copy_rows_batch", shard._h(), n, names, firsts, counts, dsts,
                     ctypes.c_void_p(staging.data_ptr()), staging_bytes, ctypes.c_void_p(stream.cuda_stream))
        for w, o in zip(want, outs):
            host = o.cpu()
            nb = w.numel() * w.element_size()
            assert torch.equal(host[32:32 + nb], w.reshape(-1).view(torch.uint8))
            assert (host[:32] == 0x5A).all() and (host[32 + nb:] == 0x5A).all()
        # the Python batch allocates on the side stream and returns in request order
        side = torch.cuda.Stream(gpu)
        got = shard.copy_rows_batch(reqs, gpu, side)
        torch.cuda.synchronize(gpu)
        for w, g in zip(want, got):
            assert g.shape == w.shape and torch.equal(g.cpu().view(torch.uint8), w.view(torch.uint8))


@pytest.fixture(scope="module")
def mxfp4_shard(tmp_path_factory):
    g = torch.Generator().manual_seed(9)
    tensors = {
        # 3 experts of 3200 rows (50 tiles) x 90 groups: the gpt-oss group count
        "l.gate_up_proj_blocks": torch.randint(0, 256, (3, 3200, 90, 16), generator=g, dtype=torch.uint8),
        "l.gate_up_proj_scales": torch.randint(100, 140, (3, 3200, 90), generator=g, dtype=torch.uint8),
        # 22 groups: the scale record is padded (6 steps -> 8)
        "l.down_proj_blocks": torch.randint(0, 256, (2, 128, 22, 16), generator=g, dtype=torch.uint8),
        "l.down_proj_scales": torch.randint(100, 140, (2, 128, 22), generator=g, dtype=torch.uint8),
        "l.bad_rows_blocks": torch.zeros((1, 96, 4, 16), dtype=torch.uint8),
        "l.bad_rows_scales": torch.zeros((1, 96, 4), dtype=torch.uint8),
        "l.f16": torch.zeros((1, 64, 4), dtype=torch.float16),
    }
    path = tmp_path_factory.mktemp("mx") / "mx.safetensors"
    safetensors_torch.save_file(tensors, str(path))
    return path, tensors


def _expected_packed(tensors, proj, e, gpu):
    from klcquant_amd import ops

    b = tensors[f"l.{proj}_blocks"][e:e + 1].to(gpu)
    s = tensors[f"l.{proj}_scales"][e:e + 1].to(gpu)
    return ops.mxfp4_pack(b, s)[0]


@pytest.mark.parametrize("proj,e", [("gate_up_proj", 0), ("gate_up_proj", 2), ("down_proj", 1)])
def test_load_mxfp4_packed_matches_pack(gpu, mxfp4_shard, proj, e):
    path, tensors = mxfp4_shard
    with SafetensorShard(path) as shard:
        side = torch.cuda.Stream(gpu)
        packed, rows, groups = shard.load_mxfp4_packed(f"l.{proj}_blocks", f"l.{proj}_scales", e, gpu, side)
        torch.cuda.synchronize(gpu)
        assert (rows, groups) == tuple(tensors[f"l.{proj}_scales"].shape[1:])
        assert torch.equal(packed, _expected_packed(tensors, proj, e, gpu))


@pytest.mark.parametrize("tiles_staged", [2, 3, 7])
def test_load_mxfp4_packed_small_staging_wraps(gpu, mxfp4_shard, tiles_staged):
    """Staging for 2, 3 or 7 tiles: two slots of 1, 1 or 3 tiles, so the 50
    tiles take 50, 50 or 17 chunks; a canary past the packed bytes stays intact."""
    from klcquant_amd import ops

    path, tensors = mxfp4_shard
    tile_bytes = 64 * 90 * 17
    nbytes = tiles_staged * tile_bytes
    with SafetensorShard(path) as shard:
        staging = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
        size = ops.packed_bytes(3200, 90)
        out = torch.full((size + 256,), 0x3C, dtype=torch.uint8, device=gpu)
        stream = torch.cuda.current_stream(gpu)
        _native.call("klc_st_load_mxfp4_packed", shard._h(), b"l.gate_up_proj_blocks", b"l.gate_up_proj_scales", 1,
                     ctypes.c_void_p(staging.data_ptr()), nbytes, ctypes.c_void_p(out.data_ptr()),
                     ctypes.c_void_p(stream.cuda_stream))
        torch.cuda.synchronize(gpu)
        assert torch.equal(out[:size], _expected_packed(tensors, "gate_up_proj", 1, gpu))
        assert (out[size:] == 0x3C).all()


def test_load_mxfp4_packed_rejects_bad_inputs(gpu, mxfp4_shard):
    path, _ = mxfp4_shard
    with SafetensorShard(path) as shard:
        staging = torch.empty(1 << 20, dtype=torch.uint8, pin_memory=True)
        pageable = torch.empty(1 << 20, dtype=torch.uint8)
        out = torch.empty(1 << 20, dtype=torch.uint8, device=gpu)
        stream = ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)

        def call(blocks, scales, e, nbytes=1 << 20, buf=staging, dst=out.data_ptr()):
            with pytest.raises(_native.KlcError) as exc:
                _native.call("klc_st_load_mxfp4_packed", shard._h(), blocks, scales, e,
                             ctypes.c_void_p(buf.data_ptr()), nbytes, ctypes.c_void_p(dst), stream)
            return exc.value.status

        assert call(b"l.down_proj_blocks", b"l.down_proj_scales", 2) == -2  # expert out of range
        assert call(b"l.down_proj_blocks", b"l.down_proj_scales", -1) == -2
        assert call(b"l.bad_rows_blocks", b"l.bad_rows_scales", 0) == -2  # 96 rows
        assert call(b"l.down_proj_blocks", b"l.gate_up_proj_scales", 0) == -2  # shapes differ
        assert call(b"l.f16", b"l.down_proj_scales", 0) == -2  # not U8 blocks
        assert call(b"l.missing", b"l.down_proj_scales", 0) == -1
        assert call(b"l.down_proj_blocks", b"l.down_proj_scales", 0, nbytes=64 * 22 * 17) == -1  # one tile only
        assert call(b"l.down_proj_blocks", b"l.down_proj_scales", 0, buf=pageable) == -1  # not pinned
        assert torch.cuda.synchronize(gpu) is None  # the refusal leaves no HIP error behind
        from klcquant_amd import ops
        ops.mxfp4_pack(torch.zeros((1, 64, 1, 16), dtype=torch.uint8, device=gpu),
                       torch.zeros((1, 64, 1), dtype=torch.uint8, device=gpu))
        assert call(b"l.down_proj_blocks", b"l.down_proj_scales", 0, dst=out.data_ptr() + 8) == -1  # misaligned
        with pytest.raises(ValueError):
            shard.load_mxfp4_packed("l.down_proj_blocks", "l.gate_up_proj_scales", 0, gpu)


def test_async_loads_share_one_ring(gpu, mxfp4_shard):
    """Loads that return before their packs finish: the ring carries over
    between calls (three experts through a 3-tile staging), a change of slot
    layout (90 -> 22 groups) waits for the old slots, and a staged copy after
    them waits for every pack before it reuses the buffer."""
    from klcquant_amd import ops

    path, tensors = mxfp4_shard
    nbytes = 3 * 64 * 90 * 17
    with SafetensorShard(path) as shard:
        staging = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
        side = torch.cuda.Stream(gpu)
        h = ctypes.c_void_p(staging.data_ptr())
        outs = []
        for proj, e in [("gate_up_proj", 0), ("gate_up_proj", 1), ("gate_up_proj", 2), ("down_proj", 0),
                        ("down_proj", 1)]:
            rows, groups = tensors[f"l.{proj}_scales"].shape[1:]
            out = torch.empty(ops.packed_bytes(rows, groups), dtype=torch.uint8, device=gpu)
            _native.call("klc_st_load_mxfp4_packed", shard._h(), f"l.{proj}_blocks".encode(),
                         f"l.{proj}_scales".encode(), e, h, nbytes, ctypes.c_void_p(out.data_ptr()),
                         ctypes.c_void_p(side.cuda_stream))
            outs.append((proj, e, out))
        # a staged copy through the same buffer waits for the packs still reading it
        got = shard.copy_rows_batch([("l.down_proj_blocks", 1, 1)], gpu, side)[0]
        side.synchronize()
        for proj, e, out in outs:
            assert torch.equal(out, _expected_packed(tensors, proj, e, gpu)), (proj, e)
        assert torch.equal(got.cpu(), tensors["l.down_proj_blocks"][1:2])
        _native.call("klc_st_staging_wait", h)
        _native.call("klc_st_staging_release", h)
        _native.call("klc_st_staging_release", h)  # nothing left: still fine
        # the Python wrapper without waiting, then an ordinary stream wait
        packed, _, _ = shard.load_mxfp4_packed("l.gate_up_proj_blocks", "l.gate_up_proj_scales", 2, gpu, side,
                                               wait=False)
        torch.cuda.current_stream(gpu).wait_stream(side)
        assert torch.equal(packed, _expected_packed(tensors, "gate_up_proj", 2, gpu))
