"""Build the gfx950 kernel library `deciax_amd/libdeciax_hip.so` with hipcc.

Run as `python -m deciax_amd.build` (or through `__graft_entry__.build()`).
The library is built in-tree so it travels with the source tree; it holds the
HIP kernels and the C ABI declared in `include/deciax_hip.h`.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
LIB = PKG / "libdeciax_hip.so"
SOURCES = ("abi.hip", "gemm.hip", "attention.hip", "rowwise.hip", "head.hip")
ARCH = "gfx950"

# Packed-fp32 VALU forms stay disabled in every device compile.
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the deciax_amd kernels need ROCm's hipcc")


def _compile(src: str, objdir: Path) -> Path:
    obj = objdir / (Path(src).stem + ".o")
    cmd = [hipcc(), *FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every kernel source and link the shared library (always rebuilds)."""
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), 4)) as pool:
        objs = list(pool.map(lambda s: _compile(s, objdir), SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build()
