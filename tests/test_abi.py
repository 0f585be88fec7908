"""The C-ABI library: loads, exports every symbol in include/klc_moe.h, checks
arguments on the host.  No call here reaches a kernel launch."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from klcquant_amd import _native as nat

HEADER = Path(__file__).resolve().parents[1] / "include" / "klc_moe.h"


def header_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(klc_\w+)\s*\(", text, flags=re.M)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = nat.load()
    names = header_functions()
    assert "klc_moe_layer" in names and "klc_mxfp4_dequant" in names
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(nat.SIGNATURES), "ctypes table and header disagree"


def test_abi_version_matches_header():
    m = re.search(r"#define KLC_ABI_VERSION (\d+)", HEADER.read_text())
    assert nat.load().klc_abi_version() == int(m.group(1))


def test_status_codes_match_header():
    text = HEADER.read_text()
    for name, value in [("KLC_ERR_ARGUMENT", nat.KLC_ERR_ARGUMENT), ("KLC_ERR_SHAPE", nat.KLC_ERR_SHAPE),
                        ("KLC_ERR_UNSUPPORTED", nat.KLC_ERR_UNSUPPORTED), ("KLC_ERR_HIP", nat.KLC_ERR_HIP),
                        ("KLC_DTYPE_BF16", nat.DTYPE_BF16), ("KLC_DTYPE_F16", nat.DTYPE_F16),
                        ("KLC_DTYPE_F32", nat.DTYPE_F32), ("KLC_PRECISION_FP32", nat.PRECISION_FP32),
                        ("KLC_PRECISION_BF16", nat.PRECISION_BF16), ("KLC_LAYER_EVENTS", nat.LAYER_EVENTS),
                        ("KLC_DISPATCH_MAX_PAIRS", nat.DISPATCH_MAX_PAIRS),
                        ("KLC_LAYER_MAX_TOKENS", nat.LAYER_MAX_TOKENS)]:
        m = re.search(rf"#define {name} \(?(-?\d+)\)?", text)
        assert m and int(m.group(1)) == value, name


def test_packed_sizes():
    lib = nat.load()
    # 5760 rows x 90 groups: blocks 90 tiles x 90 KiB, scale records of 24 bytes per (row, quarter)
    assert lib.klc_mxfp4_packed_bytes(5760, 90) == 90 * 90 * 1024 + 5760 * 4 * 24
    assert lib.klc_mxfp4_packed_bytes(64, 1) == 1024 + 64 * 4 * 8
    assert lib.klc_mxfp4_packed_bytes(100, 90) == nat.KLC_ERR_SHAPE
    assert "multiple of 64" in nat.last_error()
    assert lib.klc_mxfp4_packed_bytes(0, 90) == nat.KLC_ERR_ARGUMENT


def test_argument_errors_before_any_launch():
    with pytest.raises(nat.KlcError) as ei:
        nat.call("klc_mxfp4_dequant", None, None, None, 1, 64, 2, nat.DTYPE_BF16, None)
    assert ei.value.status == nat.KLC_ERR_ARGUMENT and "null pointer" in ei.value.message
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    with pytest.raises(nat.KlcError) as ei:
        nat.call("klc_moe_topk_softmax", fake, fake, fake, fake, 4, 8, 9, None)
    assert ei.value.status == nat.KLC_ERR_SHAPE
    with pytest.raises(nat.KlcError) as ei:
        nat.call("klc_moe_dispatch", fake, 16, 300, fake, fake, fake, fake, fake, None)
    assert ei.value.status == nat.KLC_ERR_UNSUPPORTED
    with pytest.raises(nat.KlcError) as ei:
        nat.call("klc_moe_router_logits", fake, fake, fake, fake, None, 2, 100, 8, None)
    assert ei.value.status == nat.KLC_ERR_SHAPE
    with pytest.raises(nat.KlcError) as ei:
        nat.call("klc_moe_gate_up", fake, fake, fake, 2, 4, 128, fake, fake, fake, 2880, 2880, 7.0, 5, fake,
                 None, None)
    assert ei.value.status == nat.KLC_ERR_ARGUMENT
    with pytest.raises(nat.KlcError) as ei:
        nat.call("klc_moe_down", fake, fake, fake, 8, 128, fake, fake, fake, 4096, 2880, 0, fake, None)
    assert ei.value.status == nat.KLC_ERR_UNSUPPORTED
    with pytest.raises(nat.KlcError) as ei:
        nat.call("klc_synth_fill", fake, 16, 1, 1, 10, 300, None)
    assert ei.value.status == nat.KLC_ERR_ARGUMENT


def test_route_entry_argument_errors():
    """klc_moe_route: its own outputs may not be NULL, and the one-launch path (which keeps no float32
    SwiGLU outputs) is refused; both before any device work."""
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    args = [fake] * 7 + [2, 2880, 2880, 128, 4, 7.0, nat.PRECISION_FP32]
    with pytest.raises(nat.KlcError) as ei:
        nat.call("klc_moe_route", *args, nat.PATH_AUTO, fake, 1 << 30, fake, fake, fake, None, fake, None)
    assert ei.value.status == nat.KLC_ERR_ARGUMENT and "null pointer" in ei.value.message
    with pytest.raises(nat.KlcError) as ei:
        nat.call("klc_moe_route", *args, nat.PATH_FUSED, fake, 1 << 30, fake, fake, fake, fake, fake, None)
    assert ei.value.status == nat.KLC_ERR_UNSUPPORTED and "float32 SwiGLU" in ei.value.message
    with pytest.raises(nat.KlcError) as ei:
        nat.call("klc_moe_route", *args, nat.PATH_AUTO, fake, 256, fake, fake, fake, fake, fake, None)
    assert ei.value.status == nat.KLC_ERR_ARGUMENT and "workspace" in ei.value.message


def test_units_size():
    lib = nat.load()
    # 256 pairs over 128 experts: gate_up (256 + 7 * 128) // 8 = 144, down (256 + 3 * 128) // 4 = 160,
    # GEMM (256 + 63 * 128) // 64 = 130
    assert lib.klc_moe_units_size(256, 128) == 4 + 144 + 160 + 130
    assert lib.klc_moe_units_size(4, 128) == 4 + 4 + 4 + 4
    assert lib.klc_moe_units_size(16, 300) == nat.KLC_ERR_UNSUPPORTED


def test_workspace_size_grows_with_tokens():
    lib = nat.load()
    a = lib.klc_moe_workspace_bytes(1, 2880, 2880, 128, 4)
    b = lib.klc_moe_workspace_bytes(64, 2880, 2880, 128, 4)
    assert 0 < a < b and a % 256 == 0 and b % 256 == 0
    assert lib.klc_moe_workspace_bytes(0, 2880, 2880, 128, 4) == nat.KLC_ERR_ARGUMENT


def test_cpu_tensors_are_rejected():
    torch = pytest.importorskip("torch")
    from klcquant_amd import ops

    x = torch.zeros((2, 64), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        ops.router_logits(x, torch.zeros((4, 64), dtype=torch.bfloat16), torch.zeros(4, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="shape mismatch"):
        ops.mxfp4_dequant(torch.zeros((4, 2, 16), dtype=torch.uint8), torch.zeros((4, 3), dtype=torch.uint8))


def test_select_and_experts_argument_errors():
    """klc_moe_select / klc_moe_experts check their arguments before any device work."""
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    with pytest.raises(nat.KlcError) as ei:
        nat.call("klc_moe_select", fake, fake, None, 2, 2880, 128, 4, fake, 1 << 30, fake, fake, None)
    assert ei.value.status == nat.KLC_ERR_ARGUMENT and "null pointer" in ei.value.message
    with pytest.raises(nat.KlcError) as ei:
        nat.call("klc_moe_select", fake, fake, fake, 2, 2880, 128, 4, fake, 64, fake, fake, None)
    assert ei.value.status == nat.KLC_ERR_ARGUMENT and "workspace" in ei.value.message
    with pytest.raises(nat.KlcError) as ei:
        nat.call("klc_moe_select", fake, fake, fake, 2, 2880, 8, 9, fake, 1 << 30, fake, fake, None)
    assert ei.value.status == nat.KLC_ERR_SHAPE
    args = [fake] * 7 + [2, 2880, 2880, 128, 4, 7.0, nat.PRECISION_FP32]
    with pytest.raises(nat.KlcError) as ei:
        nat.call("klc_moe_experts", *args, nat.PATH_FUSED, fake, 1 << 30, fake, None, None, None)
    assert ei.value.status == nat.KLC_ERR_UNSUPPORTED
    with pytest.raises(nat.KlcError) as ei:
        nat.call("klc_moe_experts", *args, nat.PATH_AUTO, fake, 1 << 30, fake, fake, None, None)
    assert ei.value.status == nat.KLC_ERR_ARGUMENT and "together" in ei.value.message


def test_route_readback_argument_errors():
    """klc_moe_route_readback: a host record and a nonzero tag are required, before any device work."""
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    head = [fake] * 7 + [1, 2880, 2880, 128, 4, 7.0, nat.PRECISION_FP32, nat.PATH_AUTO, fake, 1 << 30]
    outs = [fake] * 4
    with pytest.raises(nat.KlcError) as ei:
        nat.call("klc_moe_route_readback", *head, *outs, None, 1, fake)
    assert ei.value.status == nat.KLC_ERR_ARGUMENT and "null host record" in ei.value.message
    with pytest.raises(nat.KlcError) as ei:
        nat.call("klc_moe_route_readback", *head, *outs, fake, 0, fake)
    assert ei.value.status == nat.KLC_ERR_ARGUMENT and "tag 0" in ei.value.message
