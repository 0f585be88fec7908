"""Every gfx950 kernel of the library runs without scratch (private) memory.

Scratch on these kernels means spilled registers or a register array the
compiler could not keep in registers: both cost a memory round trip per
access inside the hot loops.  The check compiles each source with the
compiler's per-kernel resource remarks (no GPU needed).
"""

from __future__ import annotations

import re
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

from klcquant_amd import _build

REMARK = re.compile(r"remark: +(Function Name|ScratchSize \[bytes/lane\]): (\S+)")


def kernel_scratch(src) -> dict[str, int]:
    cmd = [_build.hipcc(), *_build.HIPCC_FLAGS, "--cuda-device-only", "-c", str(src), "-o", "/dev/null",
           "-Rpass-analysis=kernel-resource-usage"]
    proc = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert proc.returncode == 0, proc.stderr[-2000:]
    out, name = {}, None
    for key, value in REMARK.findall(proc.stderr):
        if key == "Function Name":
            name = value
        else:
            out[name] = int(value)
    return out


def test_no_kernel_uses_scratch():
    try:
        _build.hipcc()
    except RuntimeError:
        pytest.skip("hipcc is not installed")
    srcs = _build.sources()
    with ThreadPoolExecutor(max_workers=8) as pool:
        results = list(pool.map(kernel_scratch, srcs))
    kernels = {f"{src.name}:{k}": v for src, res in zip(srcs, results) for k, v in res.items()}
    assert len(kernels) >= 20
    assert {k: v for k, v in kernels.items() if v} == {}
