"""Shared test setup.

``-m "not gpu"`` tests run anywhere (oracle pinning, host logic, C-ABI
exports).  ``-m gpu`` tests need an MI355X and the built HIP library; they
fail (not skip) when either is missing.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_ROOT = ROOT / "kcapw-klcquant_amd"
for p in (str(ROOT), str(PKG_ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    from klcquant_amd import _native

    _native.load()  # raises if libklcmoe.so is missing
    return torch.device("cuda:0")


def bf16_tensor(bits: np.ndarray, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).view(torch.bfloat16).to(device)


def bf16_bits(t) -> np.ndarray:
    import torch

    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
