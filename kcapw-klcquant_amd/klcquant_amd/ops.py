"""Tensor-level wrappers over the C ABI (device tensors in, device tensors out).

Every function validates shapes, dtypes, devices and contiguity on the host,
then enqueues HIP work on the current torch stream of the tensors' device and
returns without synchronising.  There is no CPU path: CPU tensors are
rejected.
"""

from __future__ import annotations

import ctypes
import math
from typing import NamedTuple

import torch

from . import _native as nat

_DTYPE_CODES = {torch.bfloat16: nat.DTYPE_BF16, torch.float16: nat.DTYPE_F16, torch.float32: nat.DTYPE_F32}
PRECISIONS = {"fp32": nat.PRECISION_FP32, "bf16": nat.PRECISION_BF16}


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _check_gpu(name: str, t: torch.Tensor, dtype: torch.dtype | None = None, ndim: int | None = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on a GPU device (the MoE path has no CPU implementation), got {t.device}")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name} must have {ndim} dims, got shape {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _same_device(*ts: torch.Tensor) -> torch.device:
    dev = ts[0].device
    for t in ts[1:]:
        if t is not None and t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


# ---- MXFP4 -------------------------------------------------------------------

def _mxfp4_shapes(blocks: torch.Tensor, scales: torch.Tensor) -> tuple[int, int, int, bool]:
    if blocks.dim() < 3 or blocks.shape[:-1] != scales.shape:
        # same message as mxfp4_expert.py:368-369
        raise ValueError(f"MXFP4 block/scale shape mismatch: blocks.shape={blocks.shape} scales.shape={scales.shape}")
    if blocks.shape[-1] != 16:
        raise ValueError(f"MXFP4 blocks must pack 16 bytes per group, got shape {tuple(blocks.shape)}")
    single = blocks.dim() == 3
    n_mat = 1 if single else math.prod(blocks.shape[:-3])
    return n_mat, int(blocks.shape[-3]), int(blocks.shape[-2]), single


def mxfp4_dequant(blocks: torch.Tensor, scales: torch.Tensor, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """``[..., out, G, 16]`` + ``[..., out, G]`` -> ``[..., G * 32, out]`` in ``dtype``."""
    n_mat, out_dim, groups, single = _mxfp4_shapes(blocks, scales)
    if dtype not in _DTYPE_CODES:
        raise TypeError(f"unsupported dequant dtype {dtype}")
    blocks = blocks.contiguous() if blocks.dtype == torch.uint8 else blocks.to(torch.uint8).contiguous()
    scales = scales.contiguous() if scales.dtype == torch.uint8 else scales.to(torch.uint8).contiguous()
    _check_gpu("blocks", blocks, torch.uint8)
    _check_gpu("scales", scales, torch.uint8)
    dev = _same_device(blocks, scales)
    out = torch.empty((*blocks.shape[:-3], groups * 32, out_dim), dtype=dtype, device=dev)
    nat.call("klc_mxfp4_dequant", _ptr(blocks), _ptr(scales), _ptr(out), n_mat, out_dim, groups,
             _DTYPE_CODES[dtype], _stream(dev))
    return out


def packed_bytes(out_dim: int, groups: int) -> int:
    return nat.call("klc_mxfp4_packed_bytes", out_dim, groups)


def mxfp4_pack(blocks: torch.Tensor, scales: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Checkpoint layout -> row-tile layout; returns uint8 ``[n, packed_bytes]``."""
    n_mat, out_dim, groups, _ = _mxfp4_shapes(blocks, scales)
    _check_gpu("blocks", blocks, torch.uint8)
    _check_gpu("scales", scales, torch.uint8)
    dev = _same_device(blocks, scales)
    nbytes = packed_bytes(out_dim, groups)
    if out is None:
        out = torch.empty((n_mat, nbytes), dtype=torch.uint8, device=dev)
    else:
        _check_gpu("out", out, torch.uint8)
        if out.numel() != n_mat * nbytes:
            raise ValueError(f"out holds {out.numel()} bytes, need {n_mat * nbytes}")
    nat.call("klc_mxfp4_pack", _ptr(blocks), _ptr(scales), _ptr(out), n_mat, out_dim, groups, _stream(dev))
    return out


def mxfp4_dequant_packed(packed: torch.Tensor, out_dim: int, groups: int,
                         dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Row-tile packed ``[n, bytes]`` (or ``[bytes]``) -> ``[n, G * 32, out]`` (or ``[G * 32, out]``)."""
    _check_gpu("packed", packed, torch.uint8)
    nbytes = packed_bytes(out_dim, groups)
    if packed.numel() % nbytes:
        raise ValueError(f"packed holds {packed.numel()} bytes, not a multiple of {nbytes}")
    n_mat = packed.numel() // nbytes
    shape = (groups * 32, out_dim) if packed.dim() == 1 else (n_mat, groups * 32, out_dim)
    out = torch.empty(shape, dtype=dtype, device=packed.device)
    nat.call("klc_mxfp4_dequant_packed", _ptr(packed), _ptr(out), n_mat, out_dim, groups, _DTYPE_CODES[dtype],
             _stream(packed.device))
    return out


# ---- Router --------------------------------------------------------------------

def router_logits(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, want_f32: bool = False):
    """bf16 ``x [B, H]``, ``weight [E, H]``, ``bias [E]`` -> bf16 logits ``[B, E]`` (and fp32 x)."""
    _check_gpu("hidden", x, torch.bfloat16, 2)
    _check_gpu("router weight", weight, torch.bfloat16, 2)
    _check_gpu("router bias", bias, torch.bfloat16, 1)
    dev = _same_device(x, weight, bias)
    n_tok, hidden = x.shape
    n_exp = weight.shape[0]
    if weight.shape[1] != hidden or bias.shape[0] != n_exp:
        raise ValueError(f"router shapes mismatch: x {tuple(x.shape)}, weight {tuple(weight.shape)}, bias {tuple(bias.shape)}")
    logits = torch.empty((n_tok, n_exp), dtype=torch.bfloat16, device=dev)
    x_f32 = torch.empty((n_tok, hidden), dtype=torch.float32, device=dev) if want_f32 else None
    nat.call("klc_moe_router_logits", _ptr(x), _ptr(weight), _ptr(bias), _ptr(logits), _ptr(x_f32), n_tok, hidden,
             n_exp, _stream(dev))
    return (logits, x_f32) if want_f32 else logits


def topk_softmax(logits: torch.Tensor, k: int):
    """bf16 logits ``[B, E]`` -> (int32 ids ``[B, k]``, fp32 values, bf16 weights)."""
    _check_gpu("logits", logits, torch.bfloat16, 2)
    n_tok, n_exp = logits.shape
    dev = logits.device
    ids = torch.empty((n_tok, k), dtype=torch.int32, device=dev)
    values = torch.empty((n_tok, k), dtype=torch.float32, device=dev)
    weights = torch.empty((n_tok, k), dtype=torch.bfloat16, device=dev)
    nat.call("klc_moe_topk_softmax", _ptr(logits), _ptr(ids), _ptr(values), _ptr(weights), n_tok, n_exp, k,
             _stream(dev))
    return ids, values, weights


def softmax_weights(values: torch.Tensor) -> torch.Tensor:
    """fp32 scores ``[B, k]`` -> bf16 softmax weights ``[B, k]``."""
    _check_gpu("values", values, torch.float32, 2)
    weights = torch.empty(values.shape, dtype=torch.bfloat16, device=values.device)
    nat.call("klc_moe_softmax_weights", _ptr(values), _ptr(weights), values.shape[0], values.shape[1],
             _stream(values.device))
    return weights


class Dispatch(NamedTuple):
    """klc_moe_dispatch outputs: expert offsets ``[E + 1]``, pairs sorted by expert
    ``[P]``, active experts ``[E]`` (-1 padded), their count ``[1]`` and the GEMV
    work units (``units[0]``/``units[1]`` = gate_up/down unit counts, then the lists)."""

    offsets: torch.Tensor
    sorted_pairs: torch.Tensor
    active: torch.Tensor
    n_active: torch.Tensor
    units: torch.Tensor
    n_experts: int


def max_tokens_per_call(k: int) -> int:
    """Tokens of top-``k`` routing that one dispatch / layer call takes."""
    return min(nat.LAYER_MAX_TOKENS, nat.DISPATCH_MAX_PAIRS // max(1, int(k)))


def dispatch(ids: torch.Tensor, n_experts: int) -> Dispatch:
    """int32 ids ``[B, k]`` -> :class:`Dispatch`."""
    _check_gpu("ids", ids, torch.int32)
    dev = ids.device
    n_pairs = ids.numel()
    offsets = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    sorted_pairs = torch.empty(n_pairs, dtype=torch.int32, device=dev)
    active = torch.empty(n_experts, dtype=torch.int32, device=dev)
    n_active = torch.empty(1, dtype=torch.int32, device=dev)
    units = torch.empty(nat.call("klc_moe_units_size", n_pairs, n_experts), dtype=torch.int32, device=dev)
    nat.call("klc_moe_dispatch", _ptr(ids), n_pairs, n_experts, _ptr(offsets), _ptr(sorted_pairs), _ptr(active),
             _ptr(n_active), _ptr(units), _stream(dev))
    return Dispatch(offsets, sorted_pairs, active, n_active, units, n_experts)


# ---- Experts --------------------------------------------------------------------

def pointer_table(mats: list[torch.Tensor] | torch.Tensor, device: torch.device) -> torch.Tensor:
    """Device int64 table of matrix base addresses (one per expert)."""
    if isinstance(mats, torch.Tensor):
        base = mats.data_ptr()
        stride = mats.stride(0) * mats.element_size()
        addrs = [base + i * stride for i in range(mats.shape[0])]
    else:
        addrs = [m.data_ptr() for m in mats]
    return torch.tensor(addrs, dtype=torch.int64).to(device)


def gate_up(table: torch.Tensor, bias: torch.Tensor, x: torch.Tensor, k: int, disp: Dispatch, hidden: int,
            inter: int, limit: float = 7.0, precision: str = "fp32", want_raw: bool = False, gemm: bool = False):
    """Returns the down input as bf16 hi/lo planes ``[2, B * k, I]`` (and the float32 SwiGLU output).

    ``gemm`` selects the grouped GEMM (klc_moe_gemm_gate_up) instead of the GEMV.
    """
    _check_gpu("hidden", x, torch.bfloat16, 2)
    dev = x.device
    n_tok = x.shape[0]
    split = torch.empty((2, n_tok * k, inter), dtype=torch.bfloat16, device=dev)
    raw = torch.empty((n_tok * k, inter), dtype=torch.float32, device=dev) if want_raw else None
    nat.call("klc_moe_gemm_gate_up" if gemm else "klc_moe_gate_up", _ptr(table), _ptr(bias), _ptr(x), n_tok, k,
             disp.n_experts, _ptr(disp.offsets), _ptr(disp.sorted_pairs), _ptr(disp.units), hidden, inter,
             float(limit), PRECISIONS[precision], _ptr(split), _ptr(raw), _stream(dev))
    return (split, raw) if want_raw else split


def down(table: torch.Tensor, bias: torch.Tensor, gated_split: torch.Tensor, disp: Dispatch, hidden: int, inter: int,
         precision: str = "fp32", gemm: bool = False) -> torch.Tensor:
    """float32 expert outputs ``[P, H]`` (``gemm``: klc_moe_gemm_down instead of the GEMV)."""
    _check_gpu("gated_split", gated_split, torch.bfloat16, 3)
    dev = gated_split.device
    n_pairs = gated_split.shape[1]
    eo = torch.empty((n_pairs, hidden), dtype=torch.float32, device=dev)
    nat.call("klc_moe_gemm_down" if gemm else "klc_moe_down", _ptr(table), _ptr(bias), _ptr(gated_split), n_pairs,
             disp.n_experts, _ptr(disp.offsets), _ptr(disp.sorted_pairs), _ptr(disp.units), hidden, inter,
             PRECISIONS[precision], _ptr(eo), _stream(dev))
    return eo


def combine(expert_out: torch.Tensor, weights: torch.Tensor, n_tokens: int, k: int,
            residual: torch.Tensor | None = None) -> torch.Tensor:
    """bf16 weighted sum of the k expert outputs per token (+ ``residual`` if given)."""
    _check_gpu("expert_out", expert_out, torch.float32)
    _check_gpu("weights", weights, torch.bfloat16)
    hidden = expert_out.shape[-1]
    if residual is not None:
        _check_gpu("residual", residual, torch.bfloat16, 2)
        if tuple(residual.shape) != (n_tokens, hidden):
            raise ValueError(f"residual shape {tuple(residual.shape)} != ({n_tokens}, {hidden})")
    out = torch.empty((n_tokens, hidden), dtype=torch.bfloat16, device=expert_out.device)
    nat.call("klc_moe_combine", _ptr(expert_out), _ptr(weights), _ptr(residual), n_tokens, k, hidden, _ptr(out),
             _stream(expert_out.device))
    return out


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-5, out: torch.Tensor | None = None):
    """bf16 ``x [B, H]`` -> ``x * rsqrt(mean(x^2) + eps).to(bf16) * weight`` (klc_rms_norm)."""
    _check_gpu("x", x, torch.bfloat16, 2)
    _check_gpu("weight", weight, torch.bfloat16, 1)
    if weight.shape[0] != x.shape[1]:
        raise ValueError(f"norm weight of {weight.shape[0]} for hidden {x.shape[1]}")
    if out is None:
        out = torch.empty_like(x)
    nat.call("klc_rms_norm", _ptr(x), _ptr(weight), _ptr(out), x.shape[0], x.shape[1], float(eps), _stream(x.device))
    return out


def bias_combine(down_bias: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
    _check_gpu("down_bias", down_bias, torch.bfloat16, 2)
    _check_gpu("ids", ids, torch.int32, 2)
    _check_gpu("weights", weights, torch.bfloat16, 2)
    n_tok, k = ids.shape
    hidden = down_bias.shape[1]
    out = torch.empty((n_tok, hidden), dtype=torch.bfloat16, device=ids.device)
    nat.call("klc_moe_bias_combine", _ptr(down_bias), _ptr(ids), _ptr(weights), n_tok, k, hidden, _ptr(out),
             _stream(ids.device))
    return out


def pair_norms(gated: torch.Tensor, expert_out: torch.Tensor) -> torch.Tensor:
    _check_gpu("gated", gated, torch.float32, 2)
    _check_gpu("expert_out", expert_out, torch.float32, 2)
    norms = torch.empty((gated.shape[0], 2), dtype=torch.float32, device=gated.device)
    nat.call("klc_moe_pair_norms", _ptr(gated), _ptr(expert_out), gated.shape[0], gated.shape[1],
             expert_out.shape[1], _ptr(norms), _stream(gated.device))
    return norms


def workspace_bytes(n_tokens: int, hidden: int, inter: int, n_experts: int, k: int) -> int:
    return nat.call("klc_moe_workspace_bytes", n_tokens, hidden, inter, n_experts, k)


def synth_fill(dst: torch.Tensor, seed: int, mode: int = 0, lo: int = 0, hi: int = 255) -> torch.Tensor:
    """Fills a uint8 device tensor from the SplitMix64 stream (see klcquant_amd.synth)."""
    _check_gpu("dst", dst, torch.uint8)
    nat.call("klc_synth_fill", _ptr(dst), dst.numel(), ctypes.c_uint64(seed & ((1 << 64) - 1)), mode, lo, hi,
             _stream(dst.device))
    return dst
