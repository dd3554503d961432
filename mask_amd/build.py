"""Build the gfx950 shared library ``libmask_srbcrs.so`` in-tree with hipcc.

Usage: ``python -m mask_amd.build`` (or ``mask_amd.build.build()``).
The library is placed next to this file so that it travels with the source
tree; nothing is installed.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
ROOT = PKG.parent
LIB = PKG / "libmask_srbcrs.so"
ARCH = "gfx950"

# gfx950 device flags.  Packed-FP32 instruction selection is disabled: the
# kernels are written against scalar FP32 / MFMA only.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the gfx950 backend cannot be built")


def _run(cmd):
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature
    out = "\n".join(l for l in res.stdout.splitlines() if "packed-fp32-ops" not in l and l.strip())
    if res.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{out}")
    return out


def build(verbose: bool = False) -> Path:
    hipcc = _hipcc()
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    objs = []
    for src in ("srbcrs_kernels.hip", "srbcrs_capi.cpp"):
        obj = objdir / (src.rsplit(".", 1)[0] + ".o")
        cmd = [hipcc, *DEVICE_FLAGS, f"-I{ROOT / 'include'}", "-x", "hip", "-c", str(CSRC / src), "-o", str(obj)]
        out = _run(cmd)
        if verbose and out:
            print(out)
        objs.append(str(obj))
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *objs, "-lpthread"])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
