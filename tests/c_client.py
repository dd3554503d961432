"""Build helper for the plain-C client of the C ABI (tests/c/)."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
SRC = ROOT / "tests" / "c" / "srbcrs_c_client.c"
ROCM = Path("/opt/rocm")


def compile_client(out: Path) -> Path:
    """gcc -std=c99 against include/srbcrs.h, libmask_srbcrs.so and libamdhip64."""
    gcc = shutil.which("gcc")
    if gcc is None:
        raise RuntimeError("gcc not found")
    lib_dir = ROOT / "mask_amd"
    cmd = [gcc, "-std=c99", "-O1", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
           f"-I{ROOT / 'include'}", f"-I{ROCM / 'include'}", str(SRC), "-o", str(out),
           f"-L{lib_dir}", "-lmask_srbcrs", f"-Wl,-rpath,{lib_dir}", f"-L{ROCM / 'lib'}", "-lamdhip64",
           f"-Wl,-rpath,{ROCM / 'lib'}", "-lm"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return out
