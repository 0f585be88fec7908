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


DMA = re.compile(r"^\s*buffer_load\w*\s.*\slds\s*$")
VMEM = re.compile(r"^\s*(buffer_load|global_load|flat_load|buffer_store|global_store|global_atomic|buffer_atomic)")
WAIT = re.compile(r"^\s*s_waitcnt vmcnt\((\d+)\)")


def dma_waits(asm: str) -> list[tuple[str, int, int]]:
    """For each kernel that stages rows by buffer-to-LDS DMA: (kernel, vmcnt of the wait before its first
    s_barrier after the last DMA, vector memory operations issued between that DMA and the wait)."""
    out = []
    for body in re.split(r"\n(?=_Z[^\n]*:\s*;\s*@)", asm):
        name = body.split(":", 1)[0]
        lines = body.split("\n")
        last, count = None, 0
        for i, line in enumerate(lines):
            if DMA.match(line):
                last, count = i, 0
                continue
            if last is None:
                continue
            if VMEM.match(line):
                count += 1
            m = WAIT.match(line)
            if m and i + 1 < len(lines) and "s_barrier" in lines[i + 1]:
                out.append((name, int(m.group(1)), count))
                break
    return out


def test_lds_dma_waits_cover_every_dma():
    """The decode GEMVs stage activation rows by buffer-to-LDS DMA ahead of the weight ring and wait with an
    explicit vmcnt that lets exactly the ring's loads stay in flight.  vmcnt counts in issue order, so the
    wait covers every DMA only if exactly that many vector memory operations follow the last DMA; a load the
    compiler placed between them, or moved past the wait, would leave a DMA unwaited (a race on LDS)."""
    try:
        cc = _build.hipcc()
    except RuntimeError:
        pytest.skip("hipcc is not installed")
    src = _build.CSRC / "klc_experts.hip"
    cmd = [cc, *_build.HIPCC_FLAGS, "--cuda-device-only", "-S", str(src), "-o", "-"]
    proc = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert proc.returncode == 0, proc.stderr[-2000:]
    waits = dma_waits(proc.stdout)
    assert len(waits) >= 24  # 16 GEMV instantiations + 8 single-token gate_up and 8 down+combine
    assert [w for w in waits if w[1] != w[2]] == []
