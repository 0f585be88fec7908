"""Native reader for one safetensors shard (klc_st_* in libklcmoe.so).

The shard is opened and its header parsed once; an expert's slice of a
``[E, ...]`` tensor is a contiguous byte range along dimension 0, read with
pread by a small thread pool into host memory (``read_rows``) or into a ring
of pinned staging slots and from there to device memory
(``copy_rows_to_device``, ``copy_rows_batch``).
This replaces the per-miss ``safe_open(...).get_slice(name)[expert]`` ->
``pin_memory()`` -> ``.to(device)`` chain of mxfp4_expert.py:478-525.
"""

from __future__ import annotations

import ctypes
import functools
import threading
from pathlib import Path

import torch

from . import _native, ops

_DTYPES = {
    "U8": torch.uint8, "I8": torch.int8, "BOOL": torch.bool, "F8_E4M3": torch.float8_e4m3fn,
    "F8_E5M2": torch.float8_e5m2, "BF16": torch.bfloat16, "F16": torch.float16, "I16": torch.int16,
    "U16": torch.uint16, "F32": torch.float32, "I32": torch.int32, "U32": torch.uint32,
    "F64": torch.float64, "I64": torch.int64, "U64": torch.uint64,
}

#: Pinned staging per thread: a ring of four 8 MiB slots, so reading later
#: slots from the page cache overlaps the PCIe transfers of earlier ones.
STAGING_BYTES = 32 << 20

@functools.lru_cache(maxsize=64)
def _packed_bytes(rows: int, groups: int) -> int:
    return ops.packed_bytes(rows, groups)


class _Staging:
    """A thread's pinned staging buffer.  Packs enqueued by asynchronous
    loads may still read it, so it is released through the library (which
    waits for them) before torch may reuse the memory."""

    def __init__(self) -> None:
        self.buf = torch.empty(STAGING_BYTES, dtype=torch.uint8, pin_memory=True)

    def __del__(self) -> None:
        try:
            _native.call("klc_st_staging_release", ctypes.c_void_p(self.buf.data_ptr()))
        except Exception:
            pass


_staging = threading.local()


def _thread_staging() -> torch.Tensor:
    owner = getattr(_staging, "owner", None)
    if owner is None:
        owner = _Staging()
        _staging.owner = owner
    return owner.buf


class SafetensorShard:
    """One open shard; lookups are read-only, so threads may share it."""

    def __init__(self, path: str | Path) -> None:
        self.path = Path(path)
        handle = ctypes.c_void_p()
        _native.call("klc_st_open", str(self.path).encode(), ctypes.byref(handle))
        self._handle = handle
        self._info: dict[str, tuple[str, tuple[int, ...], int, int]] = {}

    def close(self) -> None:
        if self._handle is not None and self._handle.value:
            _native.call("klc_st_close", self._handle)
        self._handle = None

    def __enter__(self) -> "SafetensorShard":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass

    def _h(self) -> ctypes.c_void_p:
        if self._handle is None:
            raise ValueError(f"{self.path} is closed")
        return self._handle

    def info(self, name: str) -> tuple[str, tuple[int, ...], int, int]:
        """``(dtype, shape, absolute data offset, nbytes)`` of a tensor."""
        cached = self._info.get(name)
        if cached is not None and self._handle is not None:
            return cached
        dtype = ctypes.create_string_buffer(16)
        shape = (ctypes.c_int64 * 8)()
        ndim = ctypes.c_int()
        off = ctypes.c_int64()
        nbytes = ctypes.c_int64()
        _native.call("klc_st_tensor_info", self._h(), name.encode(), dtype, shape, ctypes.byref(ndim),
                     ctypes.byref(off), ctypes.byref(nbytes))
        result = (dtype.value.decode(), tuple(int(shape[i]) for i in range(ndim.value)), off.value, nbytes.value)
        self._info[name] = result
        return result

    def _row_slice(self, name: str, first: int, count: int) -> tuple[torch.dtype, tuple[int, ...]]:
        dtype, shape, _, _ = self.info(name)
        if dtype not in _DTYPES:
            raise ValueError(f"{self.path}: tensor '{name}' has unsupported dtype {dtype}")
        if not shape:
            raise ValueError(f"{self.path}: tensor '{name}' is a scalar")
        return _DTYPES[dtype], (int(count),) + shape[1:]

    def read_rows(self, name: str, first: int, count: int = 1) -> torch.Tensor:
        """Rows ``[first, first + count)`` along dimension 0 as a host tensor."""
        tdtype, shape = self._row_slice(name, first, count)
        out = torch.empty(shape, dtype=tdtype)
        _native.call("klc_st_read_rows", self._h(), name.encode(), int(first), int(count),
                     ctypes.c_void_p(out.data_ptr()))
        return out

    def copy_rows_to_device(self, name: str, first: int, count: int, device: torch.device,
                            stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        """Rows ``[first, first + count)`` as a device tensor allocated on ``stream``.

        Returns once the copy has completed (the staging buffer is reused).
        """
        return self.copy_rows_batch([(name, first, count)], device, stream)[0]

    def copy_rows_batch(self, requests: list[tuple[str, int, int]], device: torch.device,
                        stream: torch.cuda.Stream | None = None) -> list[torch.Tensor]:
        """Several ``(name, first, count)`` row ranges as device tensors, in one
        staged copy (one wait at the end); the tensors are allocated on ``stream``."""
        device = torch.device(device)
        stream = stream if stream is not None else torch.cuda.current_stream(device)
        slices = [self._row_slice(name, first, count) for name, first, count in requests]
        with torch.cuda.stream(stream):
            outs = [torch.empty(shape, dtype=tdtype, device=device) for tdtype, shape in slices]
        n = len(requests)
        names = (ctypes.c_char_p * n)(*(name.encode() for name, _, _ in requests))
        firsts = (ctypes.c_int64 * n)(*(int(first) for _, first, _ in requests))
        counts = (ctypes.c_int64 * n)(*(int(count) for _, _, count in requests))
        dsts = (ctypes.c_void_p * n)(*(out.data_ptr() for out in outs))
        staging = _thread_staging()
        _native.call("klc_st_copy_rows_batch", self._h(), n, names, firsts, counts, dsts,
                     ctypes.c_void_p(staging.data_ptr()), staging.numel(), ctypes.c_void_p(stream.cuda_stream))
        return outs

    def load_mxfp4_packed(self, blocks_name: str, scales_name: str, expert: int, device: torch.device,
                          stream: torch.cuda.Stream | None = None, wait: bool = True) -> tuple[torch.Tensor, int, int]:
        """One expert's MXFP4 projection, read from the shard straight into the
        packed row-tile layout on the device: ``(packed, rows, groups)``.

        Chunks of 64-row tiles are read into this thread's pinned staging and
        packed by a kernel on ``stream`` that reads the staging over PCIe (the
        packed tensor is allocated on ``stream``; a caller that uses it on
        another stream records that stream on it).  With ``wait`` the call
        returns once the packed matrix is complete; without it, once the last
        pack is enqueued (work on ``stream`` then sees the finished matrix, and
        the next load from this thread overlaps the packs still running).
        """
        device = torch.device(device)
        stream = stream if stream is not None else torch.cuda.current_stream(device)
        b_dtype, b_shape, _, _ = self.info(blocks_name)
        s_dtype, s_shape, _, _ = self.info(scales_name)
        if b_dtype != "U8" or s_dtype != "U8" or len(b_shape) != 4 or tuple(b_shape[:-1]) != tuple(s_shape):
            raise ValueError(f"MXFP4 block/scale shape mismatch: blocks.shape={b_shape[1:]} "
                             f"scales.shape={s_shape[1:]} ({b_dtype}/{s_dtype})")
        rows, groups = int(b_shape[1]), int(b_shape[2])
        staging = _thread_staging()
        # allocated on `stream`, the stream that writes it: the caching
        # allocator then hands out only memory whose earlier users are done
        # in that stream's order (or recorded by record_stream)
        with torch.cuda.stream(stream):
            packed = torch.empty(_packed_bytes(rows, groups), dtype=torch.uint8, device=device)
        _native.call("klc_st_load_mxfp4_packed", self._h(), blocks_name.encode(), scales_name.encode(), int(expert),
                     ctypes.c_void_p(staging.data_ptr()), staging.numel(), ctypes.c_void_p(packed.data_ptr()),
                     ctypes.c_void_p(stream.cuda_stream))
        if wait:
            _native.call("klc_st_staging_wait", ctypes.c_void_p(staging.data_ptr()))
        return packed, rows, groups
