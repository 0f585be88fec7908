"""Builds the HIP library ``libklcmoe.so`` for gfx950 with hipcc.

The library is built in-tree next to this file so that it travels with the
source tree; objects go to ``kcapw-klcquant_amd/_build``.  Run as
``python -m klcquant_amd._build`` (from ``kcapw-klcquant_amd``) or call
:func:`build_library`.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT = PKG_DIR.parent
CSRC = ROOT / "csrc"
INCLUDE = ROOT.parent / "include"
BUILD_DIR = ROOT / "_build"
LIB_NAME = "libklcmoe.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = "gfx950"

# Packed-FP32 VALU instructions are kept out of the code objects on purpose.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the KLC MoE library needs ROCm's hipcc to build")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path, cc: str) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [cc, *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (proc.stderr or "").splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build_library(verbose: bool = True) -> Path:
    """Compiles every ``csrc/*.hip`` for gfx950 and links ``libklcmoe.so``."""
    cc = hipcc()
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(srcs), max(1, (os.cpu_count() or 2) // 2), 8)
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(lambda s: _compile(s, cc), srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources")
    return LIB_PATH


def build_single(src: Path, out: Path, verbose: bool = True) -> Path:
    """Compiles one self-contained ``.hip`` file into its own shared library
    (the measurement libraries under ``tests/native``)."""
    cc = hipcc()
    tmp = out.with_suffix(".so.tmp")
    cmd = [cc, *HIPCC_FLAGS, "-shared", "-o", str(tmp), str(src)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{proc.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build_library()
