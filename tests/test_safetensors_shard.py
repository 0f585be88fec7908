"""The native safetensors shard reader (klc_st_*), on the CPU.

The format is pinned twice: files written by the safetensors library are read
back and compared with its own ``safe_open`` slices, and a file assembled here
byte by byte (8-byte little-endian header length, JSON header with
``__metadata__``, data section) is read back against the bytes placed in it,
so a wrong header offset or row stride fails either way.  Malformed files and
bad row ranges must raise, not read out of bounds.
"""

from __future__ import annotations

import ctypes
import json
import struct

import numpy as np
import pytest
import torch

from klcquant_amd import _native
from klcquant_amd.safetensors_shard import SafetensorShard

safetensors_torch = pytest.importorskip("safetensors.torch")
from safetensors import safe_open  # noqa: E402


def _tensors(seed: int = 0) -> dict[str, torch.Tensor]:
    g = torch.Generator().manual_seed(seed)
    return {
        "model.layers.0.mlp.experts.gate_up_proj_blocks": torch.randint(0, 256, (4, 6, 3, 16), generator=g,
                                                                        dtype=torch.uint8),
        "model.layers.0.mlp.experts.gate_up_proj_scales": torch.randint(0, 256, (4, 6, 3), generator=g,
                                                                        dtype=torch.uint8),
        "model.layers.0.mlp.experts.gate_up_proj_bias": torch.randn(4, 12, generator=g).to(torch.bfloat16),
        "weights.f32": torch.randn(5, 3, 2, generator=g),
        "counts.i64": torch.arange(7, dtype=torch.int64) * 1_000_000_007,
        "empty.rows": torch.zeros(0, 4, dtype=torch.float16),
        "name with \"quotes\" and ä中\U0001f600": torch.arange(6, dtype=torch.int32).reshape(3, 2),
    }


@pytest.fixture()
def shard_file(tmp_path):
    tensors = _tensors()
    path = tmp_path / "model-00001-of-00001.safetensors"
    safetensors_torch.save_file(tensors, str(path), metadata={"format": "pt", "note": "{[nested]}"})
    return path, tensors


def test_info_matches_the_library(shard_file):
    path, tensors = shard_file
    with SafetensorShard(path) as shard, safe_open(str(path), framework="pt") as ref:
        for name, t in tensors.items():
            dtype, shape, off, nbytes = shard.info(name)
            assert shape == tuple(t.shape)
            assert nbytes == t.numel() * t.element_size()
            assert dtype == {torch.uint8: "U8", torch.bfloat16: "BF16", torch.float32: "F32",
                             torch.int64: "I64", torch.float16: "F16", torch.int32: "I32"}[t.dtype]
            raw = np.fromfile(path, dtype=np.uint8, count=nbytes, offset=off)
            assert raw.tobytes() == t.contiguous().view(torch.uint8).numpy().tobytes()
            assert torch.equal(ref.get_tensor(name), t)


def test_every_row_range_matches_safe_open(shard_file):
    path, tensors = shard_file
    with SafetensorShard(path) as shard, safe_open(str(path), framework="pt") as ref:
        for name, t in tensors.items():
            rows = t.shape[0]
            for first in range(rows + 1):
                for count in range(rows - first + 1):
                    got = shard.read_rows(name, first, count)
                    want = ref.get_slice(name)[first:first + count]
                    assert got.dtype == want.dtype and got.shape == want.shape, (name, first, count)
                    assert torch.equal(got.view(torch.uint8) if got.numel() else got,
                                       want.contiguous().view(torch.uint8) if want.numel() else want)


def _handmade(tmp_path, header: dict | bytes, data: bytes, declared_len: int | None = None):
    h = header if isinstance(header, bytes) else json.dumps(header).encode()
    n = len(h) if declared_len is None else declared_len
    path = tmp_path / "hand.safetensors"
    path.write_bytes(struct.pack("<Q", n) + h + data)
    return path


def test_handmade_file_offsets_and_strides(tmp_path):
    # two tensors stored in reverse order in the data section, padded header
    a = np.arange(3 * 4, dtype=np.uint8).reshape(3, 4) + 100
    b = (np.arange(2 * 3, dtype=np.int16).reshape(2, 3) * -7)
    data = b.tobytes() + a.tobytes()
    header = {
        "__metadata__": {"k": "v"},
        "a": {"dtype": "U8", "shape": [3, 4], "data_offsets": [b.nbytes, b.nbytes + a.nbytes]},
        "b": {"dtype": "I16", "shape": [2, 3], "data_offsets": [0, b.nbytes]},
    }
    h = json.dumps(header, indent=1).encode() + b"   "
    path = _handmade(tmp_path, h, data)
    with SafetensorShard(path) as shard:
        assert shard.info("a") == ("U8", (3, 4), 8 + len(h) + b.nbytes, a.nbytes)
        assert shard.info("b") == ("I16", (2, 3), 8 + len(h), b.nbytes)
        assert np.array_equal(shard.read_rows("a", 1, 2).numpy(), a[1:3])
        assert np.array_equal(shard.read_rows("b", 1, 1).numpy(), b[1:2])
        assert np.array_equal(shard.read_rows("a", 0, 3).numpy(), a)


def _err(fn, *args):
    with pytest.raises(_native.KlcError) as exc:
        fn(*args)
    return exc.value


def test_bad_names_and_row_ranges(shard_file):
    path, _ = shard_file
    name = "model.layers.0.mlp.experts.gate_up_proj_blocks"
    with SafetensorShard(path) as shard:
        assert _err(shard.info, "missing").status == -1
        assert _err(shard.read_rows, "missing", 0, 1).status == -1
        assert _err(shard.read_rows, name, 3, 2).status == -2
        assert _err(shard.read_rows, name, -1, 1).status == -2
        assert _err(shard.read_rows, name, 4, 1).status == -2
        assert shard.read_rows(name, 4, 0).shape == (0, 6, 3, 16)


@pytest.mark.parametrize("case", ["short", "header_past_end", "not_json", "bad_offsets", "size_mismatch",
                                  "missing_field", "truncated_data", "deep_metadata"])
def test_malformed_files_are_rejected(tmp_path, case):
    ok = {"t": {"dtype": "F32", "shape": [2, 2], "data_offsets": [0, 16]}}
    data = bytes(16)
    if case == "short":
        path = tmp_path / "short.safetensors"
        path.write_bytes(b"\x01\x02")
    elif case == "header_past_end":
        path = _handmade(tmp_path, ok, data, declared_len=10_000)
    elif case == "not_json":
        path = _handmade(tmp_path, b'{"t": {"dtype": "F32", "shape": [2, 2], "data_offsets": [0, 16]', data)
    elif case == "bad_offsets":
        path = _handmade(tmp_path, {"t": {"dtype": "F32", "shape": [2, 2], "data_offsets": [16, 0]}}, data)
    elif case == "size_mismatch":
        path = _handmade(tmp_path, {"t": {"dtype": "F32", "shape": [2, 3], "data_offsets": [0, 16]}}, data)
    elif case == "missing_field":
        path = _handmade(tmp_path, {"t": {"dtype": "F32", "data_offsets": [0, 16]}}, data)
    elif case == "truncated_data":
        path = _handmade(tmp_path, ok, data[:12])
    else:
        deep = {}
        for _ in range(100):
            deep = {"x": deep}
        path = _handmade(tmp_path, {"__metadata__": deep, **ok}, data)
    assert _err(SafetensorShard, path).status == -2


def test_unknown_dtype_rows_are_refused(tmp_path):
    """A dtype whose element size the reader does not know (sub-byte or new
    formats) is listed but never sliced by rows."""
    path = _handmade(tmp_path, {"f4": {"dtype": "F4", "shape": [4, 2], "data_offsets": [0, 4]}}, bytes(4))
    with SafetensorShard(path) as shard:
        assert shard.info("f4") == ("F4", (4, 2), 8 + len(json.dumps({"f4": {"dtype": "F4", "shape": [4, 2],
                                                                        "data_offsets": [0, 4]}}).encode()), 4)
        buf = (ctypes.c_uint8 * 4)()
        assert _err(_native.call, "klc_st_read_rows", shard._h(), b"f4", 0, 1, ctypes.addressof(buf)).status == -3


def test_missing_file_is_an_argument_error(tmp_path):
    assert _err(SafetensorShard, tmp_path / "absent.safetensors").status == -1


def test_closed_shard_refuses_reads(shard_file):
    path, _ = shard_file
    shard = SafetensorShard(path)
    shard.close()
    shard.close()
    with pytest.raises(ValueError):
        shard.info("weights.f32")


def test_large_ranges_and_concurrent_readers(tmp_path):
    """Ranges above the per-thread slice size are read by the thread pool;
    several Python threads share one shard and the pool."""
    from concurrent.futures import ThreadPoolExecutor

    g = torch.Generator().manual_seed(3)
    big = torch.randint(0, 256, (6, 3_000_001), generator=g, dtype=torch.uint8)
    path = tmp_path / "big.safetensors"
    safetensors_torch.save_file({"big": big}, str(path))
    with SafetensorShard(path) as shard:
        assert torch.equal(shard.read_rows("big", 0, 6), big)

        def one(i):
            first, count = i % 6, 1 + (i % (6 - i % 6))
            return torch.equal(shard.read_rows("big", first, count), big[first:first + count])

        with ThreadPoolExecutor(max_workers=4) as ex:
            assert all(ex.map(one, range(24)))


def test_pool_jobs_of_alternating_slice_counts_run_each_slice_once(tmp_path):
    """Back-to-back reads alternate between few and many pool slices (a job
    with more slices than the one before is where a worker still holding the
    old job could claim a slice of the new one); every read must come back
    whole, and no call may hang."""
    g = torch.Generator().manual_seed(5)
    rows = torch.randint(0, 256, (16, 1 << 20), generator=g, dtype=torch.uint8)  # 1 MiB rows
    path = tmp_path / "rows.safetensors"
    safetensors_torch.save_file({"rows": rows}, str(path))
    with SafetensorShard(path) as shard:
        for i in range(600):
            first, count = (i * 7) % 8, (1, 8, 2, 6, 1, 3)[i % 6]  # 1 MiB .. 8 MiB: 8 .. 64 slices
            got = shard.read_rows("rows", first, count)
            assert torch.equal(got, rows[first:first + count]), i


def test_forked_child_reads_without_the_pool(tmp_path):
    import os
    import signal

    big = torch.arange(4 * 1_000_000, dtype=torch.int32).reshape(4, -1)
    path = tmp_path / "fork.safetensors"
    safetensors_torch.save_file({"big": big}, str(path))
    with SafetensorShard(path) as shard:
        assert torch.equal(shard.read_rows("big", 1, 3), big[1:])  # the pool exists before the fork
        pid = os.fork()
        if pid == 0:  # numpy only: torch's OpenMP pool does not survive a fork
            signal.alarm(20)
            ok = np.array_equal(shard.read_rows("big", 0, 4).numpy(), big.numpy())
            os._exit(0 if ok else 1)
        _, status = os.waitpid(pid, 0)
        assert os.WIFEXITED(status) and os.WEXITSTATUS(status) == 0


def test_file_truncated_after_open_is_an_error(tmp_path):
    t = torch.arange(4 * 100_000, dtype=torch.int32).reshape(4, -1)
    path = tmp_path / "trunc.safetensors"
    safetensors_torch.save_file({"t": t}, str(path))
    with SafetensorShard(path) as shard:
        os_size = path.stat().st_size
        with open(path, "r+b") as fh:
            fh.truncate(os_size - 200_000)
        assert torch.equal(shard.read_rows("t", 0, 2), t[:2])
        assert _err(shard.read_rows, "t", 2, 2).status == -1
