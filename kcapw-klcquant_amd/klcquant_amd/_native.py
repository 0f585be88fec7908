"""ctypes binding of ``libklcmoe.so`` (the C ABI declared in include/klc_moe.h).

The library is loaded once, from this package directory.  There is no
fallback: if the library is missing or fails to load, every entry point raises
``KlcLibraryError``.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libklcmoe.so"

KLC_OK = 0
KLC_ERR_ARGUMENT = -1
KLC_ERR_SHAPE = -2
KLC_ERR_UNSUPPORTED = -3
KLC_ERR_HIP = -4

DTYPE_BF16 = 0
DTYPE_F16 = 1
DTYPE_F32 = 2

PRECISION_FP32 = 0
PRECISION_BF16 = 1

LAYER_EVENTS = 7  # KLC_LAYER_EVENTS
PATH_AUTO, PATH_GEMV, PATH_GEMM, PATH_FUSED = 0, 1, 2, 3  # KLC_PATH_*
DISPATCH_MAX_PAIRS = 2097152  # KLC_DISPATCH_MAX_PAIRS
LAYER_MAX_TOKENS = 65535  # KLC_LAYER_MAX_TOKENS

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_F32 = ctypes.c_float
_U64 = ctypes.c_uint64

# name -> (restype, argtypes); the order matches include/klc_moe.h
SIGNATURES: dict[str, tuple] = {
    "klc_last_error": (ctypes.c_char_p, []),
    "klc_abi_version": (_I32, []),
    "klc_mxfp4_dequant": (_I32, [_P, _P, _P, _I64, _I64, _I64, _I32, _P]),
    "klc_mxfp4_packed_bytes": (_I64, [_I64, _I64]),
    "klc_mxfp4_pack": (_I32, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "klc_mxfp4_dequant_packed": (_I32, [_P, _P, _I64, _I64, _I64, _I32, _P]),
    "klc_moe_router_logits": (_I32, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "klc_moe_topk_softmax": (_I32, [_P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "klc_moe_softmax_weights": (_I32, [_P, _P, _I64, _I64, _P]),
    "klc_moe_dispatch": (_I32, [_P, _I64, _I64, _P, _P, _P, _P, _P, _P]),
    "klc_moe_units_size": (_I64, [_I64, _I64]),
    "klc_moe_gate_up": (_I32, [_P, _P, _P, _I64, _I64, _I64, _P, _P, _P, _I64, _I64, _F32, _I32, _P, _P, _P]),
    "klc_moe_down": (_I32, [_P, _P, _P, _I64, _I64, _P, _P, _P, _I64, _I64, _I32, _P, _P]),
    "klc_moe_gemm_gate_up": (_I32, [_P, _P, _P, _I64, _I64, _I64, _P, _P, _P, _I64, _I64, _F32, _I32, _P, _P, _P]),
    "klc_moe_gemm_down": (_I32, [_P, _P, _P, _I64, _I64, _P, _P, _P, _I64, _I64, _I32, _P, _P]),
    "klc_moe_combine": (_I32, [_P, _P, _P, _I64, _I64, _I64, _P, _P]),
    "klc_rms_norm": (_I32, [_P, _P, _P, _I64, _I64, _F32, _P]),
    "klc_moe_bias_combine": (_I32, [_P, _P, _P, _I64, _I64, _I64, _P, _P]),
    "klc_moe_pair_norms": (_I32, [_P, _P, _I64, _I64, _I64, _P, _P]),
    "klc_moe_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64, _I64]),
    "klc_moe_layer_path": (_I32, [_I64, _I64, _I64, _I64, _I64, _I32, _P]),
    "klc_moe_layer_status_offset": (_I64, [_I64, _I64, _I64, _I64, _I64]),
    "klc_moe_layer": (_I32, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F32, _I32, _I32, _P, _I64,
                             _P, _P, _P, _P, _P, _P]),
    "klc_moe_route": (_I32, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F32, _I32, _I32, _P, _I64,
                             _P, _P, _P, _P, _P, _P]),
    "klc_moe_route_readback": (_I32, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F32, _I32, _I32, _P,
                                      _I64, _P, _P, _P, _P, _P, ctypes.c_uint32, _P]),
    "klc_moe_select": (_I32, [_P, _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _P, _P, _P]),
    "klc_moe_experts": (_I32, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F32, _I32, _I32, _P, _I64,
                               _P, _P, _P, _P]),
    "klc_moe_layer_static_scratch": (_I32, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F32, _I32,
                                            _I32, _P, _P, _P, _P, _P, _P]),
    "klc_st_open": (_I32, [ctypes.c_char_p, _P]),
    "klc_st_close": (_I32, [_P]),
    "klc_st_tensor_info": (_I32, [_P, ctypes.c_char_p, _P, _P, _P, _P, _P]),
    "klc_st_read_rows": (_I32, [_P, ctypes.c_char_p, _I64, _I64, _P]),
    "klc_st_copy_rows_to_device": (_I32, [_P, ctypes.c_char_p, _I64, _I64, _P, _I64, _P, _P]),
    "klc_st_copy_rows_batch": (_I32, [_P, _I32, _P, _P, _P, _P, _P, _I64, _P]),
    "klc_st_load_mxfp4_packed": (_I32, [_P, ctypes.c_char_p, ctypes.c_char_p, _I64, _P, _I64, _P, _P]),
    "klc_st_staging_wait": (_I32, [_P]),
    "klc_st_staging_release": (_I32, [_P]),
    "klc_lm_head_workspace_bytes": (_I64, [_I64]),
    "klc_lm_head_logits": (_I32, [_P, _P, _P, _I64, _I64, _P, _I64, _P, _P, _P]),
    "klc_rope_append": (_I32, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _P]),
    "klc_attn_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    "klc_attn_decode": (_I32, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _P, _I64, _P, _P]),
    "klc_synth_fill": (_I32, [_P, _I64, _U64, _I32, _I32, _I32, _P]),
}


class KlcLibraryError(RuntimeError):
    """The HIP library is missing, stale or failed to load."""


class KlcError(RuntimeError):
    """A C-ABI call returned an error status."""

    def __init__(self, func: str, status: int, message: str):
        super().__init__(f"{func} failed ({status}): {message}")
        self.func = func
        self.status = status
        self.message = message


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Loads (once) and returns the library with typed entry points."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        p = Path(path) if path else LIB_PATH
        if not p.exists():
            raise KlcLibraryError(
                f"{p} is missing: build it with `python -m klcquant_amd._build` (hipcc, gfx950); "
                "the MoE path has no CPU fallback")
        try:
            lib = ctypes.CDLL(str(p))
        except OSError as exc:  # pragma: no cover - depends on the host
            raise KlcLibraryError(f"cannot load {p}: {exc}") from exc
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        return lib


def last_error() -> str:
    return load().klc_last_error().decode("utf-8", "replace")


def call(name: str, *args) -> int:
    """Calls ``name``; raises :class:`KlcError` on a negative status."""
    fn = getattr(load(), name)
    rc = fn(*args)
    if rc < 0:
        raise KlcError(name, int(rc), last_error())
    return int(rc)
