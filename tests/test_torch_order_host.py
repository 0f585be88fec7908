"""Host build of the router's torch-order code (csrc/klc_torch_order.h).

The header is compiled for the host (hipcc, host pass only) and its
sequential libstdc++ restatement and SLEEF expf are checked against the
oracle and against torch itself.
"""

from __future__ import annotations

import ctypes
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

from oracle import torch_cpu
from oracle.numerics import f32_to_bf16

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def lib(tmp_path_factory):
    cc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(cc).exists():
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("host") / "libtorch_order_host.so"
    cmd = [cc, "-x", "hip", "--cuda-host-only", "-O2", "-std=c++17", "-shared", "-fPIC",
           f"-I{ROOT / 'kcapw-klcquant_amd' / 'csrc'}", str(ROOT / "tests" / "native" / "torch_order_host.cpp"),
           "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr
    so = ctypes.CDLL(str(out))
    so.host_torch_topk.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    so.host_sleef_expf.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
    return so


def host_topk(lib, bits: np.ndarray, k: int) -> list[int]:
    bits = np.ascontiguousarray(bits, np.uint16)
    out = np.zeros(k, np.int32)
    work = np.zeros(bits.size, np.uint32)
    lib.host_torch_topk(bits.ctypes.data, bits.size, k, out.ctypes.data, work.ctypes.data)
    return out.tolist()


def test_host_topk_equals_oracle(lib):
    rng = np.random.default_rng(31)
    for _ in range(3000):
        n = int(rng.integers(1, 600))
        k = int(rng.integers(1, min(n, 32) + 1))
        vals = rng.integers(0, int(rng.integers(1, 9)), n).astype(np.float32)
        if rng.random() < 0.2:
            vals[rng.integers(0, n, 2)] = np.nan
        bits = f32_to_bf16(vals)
        assert host_topk(lib, bits, k) == torch_cpu.topk_order(torch_cpu.order_key_bf16(bits), k), (n, k)


def test_host_topk_past_depth_limit(lib):
    from test_oracle_torch_cpu import _mcilroy_killer

    for n in (40, 100, 128, 200):
        for coarse in (1, 2, 3):
            bits = f32_to_bf16(np.floor(_mcilroy_killer(n, 3) / coarse))
            assert host_topk(lib, bits, 4) == torch_cpu.topk_order(torch_cpu.order_key_bf16(bits), 4)


def test_host_sleef_expf_equals_oracle(lib):
    rng = np.random.default_rng(32)
    x = np.concatenate([(rng.standard_normal(200000) * 30).astype(np.float32),
                        np.array([0.0, -0.0, 88.7, 89.0, -87.3, -103.9, -104.0, -104.1, 99.9, 100.0, 100.1,
                                  np.inf, -np.inf], np.float32)])
    y = np.zeros_like(x)
    lib.host_sleef_expf(x.ctypes.data, y.ctypes.data, x.size)
    want = torch_cpu.sleef_expf_u10(x)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))
