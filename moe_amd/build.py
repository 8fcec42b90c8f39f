"""Builds the HIP C-ABI library ``moe_amd/_moe_amd.so`` for gfx950 in-tree.

``python -m moe_amd.build`` (or ``__graft_entry__.build()``) compiles every
source under ``moe_amd/csrc`` with hipcc in parallel and links one shared
library.  No GPU is needed: hipcc cross-compiles the gfx950 code objects.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "_moe_amd.so"
ARCH = os.environ.get("MOE_AMD_ARCH", "gfx950")

# Packed-fp32 VALU forms stay disabled in every HIP translation unit.
HIPFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def sources() -> list[Path]:
    return sorted([*CSRC.glob("*.hip"), *CSRC.glob("*.cpp")])


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile and link the library; returns its path.  Always rebuilds."""
    hipcc = _hipcc()
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    srcs = sources()
    deps = [*srcs, *CSRC.glob("*.h"), PKG.parent / "include" / "moe_amd.h"]
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 16)

    def compile_one(src: Path) -> Path:
        obj = objdir / (src.name + ".o")
        cmd = [hipcc, *HIPFLAGS, "-c", str(src), "-o", str(obj)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
        if verbose and res.stderr.strip():
            print(res.stderr, file=sys.stderr)
        return obj

    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, OUT)
    _ = deps
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
