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
    """Compile the library and the emitter's default operators (in parallel)."""
    from concurrent.futures import ThreadPoolExecutor
    hipcc = _hipcc()
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)

    def compile_obj(src):
        obj = objdir / (src.rsplit(".", 1)[0] + ".o")
        out = _run([hipcc, *DEVICE_FLAGS, f"-I{ROOT / 'include'}", "-x", "hip", "-c", str(CSRC / src), "-o", str(obj)])
        if verbose and out:
            print(out)
        return str(obj)

    with ThreadPoolExecutor(max_workers=8) as ex:
        gen = [ex.submit(build_generated_one, bm, bk, lds) for bm, bk, lds in GENERATED_SHAPES]
        objs = list(ex.map(compile_obj, SOURCES))
        for f in gen:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *objs, "-lpthread"])
    os.replace(tmp, LIB)
    return LIB


# translation units of the library, the slowest (the spmm_stream instantiations) first
SOURCES = ("srbcrs_merged.hip", "srbcrs_nzsweep.hip", "srbcrs_stream_compact.hip", "srbcrs_stream_compact_tasks.hip", "srbcrs_stream_dense.hip",
           "srbcrs_stream_dense_tasks.hip", "srbcrs_kernels.hip", "srbcrs_capi.cpp", "srbcrs_pack.cpp",
           "srbcrs_convert.hip", "srbcrs_compact.hip", "srbcrs_probe.hip")
GENERATED = PKG / "generated"
# (block rows, block columns, B materialized in shared memory / LDS)
GENERATED_SHAPES = ((16, 8, False), (32, 32, False), (16, 8, True))


def build_generated_one(bm: int, bk: int, lds: bool = False) -> str:
    """Emit and compile an operator of the HIP emitter for one SR-BCRS block
    shape into mask_amd/generated/: the default strategy, or (lds) one that
    stages B in LDS with direct-to-LDS loads (b_array_ref_mode
    "global_load_lds")."""
    from .backend_registry import sr_bcrs_spec
    from .emitter import lower_format_operator
    strategy = ({"tensor_placement": {"materialize_b_array_ref_to_smem": True, "b_array_ref_mode": "global_load_lds"}}
                if lds else None)
    name = f"sr_bcrs_{bm}x{bk}{'_lds' if lds else ''}"
    work = PKG / "_build" / "generated" / name
    return lower_format_operator(format_obj=sr_bcrs_spec(bm, bk), codegen_format_name="SR_BCRS",
                                 operator_path=GENERATED / f"{name}.so", ir_dir=work / "ir",
                                 strategy_dir=work / "strategy", strategy_decision=strategy)["operator_path"]


SANITIZE_DIR = PKG / "_build" / "sanitize"
SANITIZE_LIB = SANITIZE_DIR / "libmask_srbcrs_sanitize.so"
# host-pass only: each -fsanitize goes right after -Xarch_host (GPU code is
# not instrumented)
SANITIZE_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                  "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer",
                  "-Xarch_host", "-g"]


def build_sanitized() -> Path:
    """The same library with AddressSanitizer and UndefinedBehaviorSanitizer
    in its host code (converter, packings, row orders, schedules, plan
    bookkeeping), for CPU tests: tests/sanitize_host.sh loads it in place of
    the product library."""
    from concurrent.futures import ThreadPoolExecutor
    hipcc = _hipcc()
    SANITIZE_DIR.mkdir(parents=True, exist_ok=True)

    def compile_obj(src):
        obj = SANITIZE_DIR / (src.rsplit(".", 1)[0] + ".o")
        _run([hipcc, *DEVICE_FLAGS, *SANITIZE_FLAGS, f"-I{ROOT / 'include'}", "-x", "hip", "-c", str(CSRC / src),
              "-o", str(obj)])
        return str(obj)

    with ThreadPoolExecutor(max_workers=8) as ex:
        objs = list(ex.map(compile_obj, SOURCES))
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-shared-libasan", "-fsanitize=address,undefined",
          "-o", str(SANITIZE_LIB), *objs, "-lpthread"])
    return SANITIZE_LIB


# Decomposition builds: the same library with one part of the SpMM's work taken
# out, for timing only.  Their results are wrong on purpose: srbcrs_version()
# names the experiment and mask_amd._capi refuses to load such a build unless
# MASK_AMD_ALLOW_EXPERIMENT=1 (set only by the timing runs that load it
# through MASK_AMD_SRBCRS_LIB).
EXPERIMENTS = {
    "no_a": "SRBCRS_EXPERIMENT_NO_A",                  # A fragments (dense or compact) not loaded
    "no_b": "SRBCRS_EXPERIMENT_NO_B",                  # B rows not gathered
    "no_mfma": "SRBCRS_EXPERIMENT_NO_MFMA",            # one VALU FMA per MFMA instead
    "plain_c_store": "SRBCRS_EXPERIMENT_PLAIN_C_STORE",  # C written with plain (not nontemporal) stores
    "gather_only": "SRBCRS_EXPERIMENT_NO_A SRBCRS_EXPERIMENT_NO_MFMA",   # B gathers and C stores only
    "mfma_only": "SRBCRS_EXPERIMENT_NO_A SRBCRS_EXPERIMENT_NO_B",        # MFMAs, indices and C stores only
    "b_hit_quarter": "SRBCRS_EXPERIMENT_B_HIT_MASK=3",  # every 4th unit gathers B row 0 (a cache hit)
    "b_hit_half": "SRBCRS_EXPERIMENT_B_HIT_MASK=1",     # every 2nd unit gathers B row 0
    "b_skip_two_thirds": "SRBCRS_EXPERIMENT_B_SKIP=3",  # only every 3rd unit gathers B (register ring)
    "lds_pad_40k": "SRBCRS_EXPERIMENT_LDS_PAD=40960",    # 40 KB of unused LDS per workgroup: at most 4 per CU
    "merged_pin": "SRBCRS_MERGED_SCHED_PIN",            # merged grid: loads pinned in source order (sched_barrier)
    "merged_vec_idx": "SRBCRS_MERGED_VEC_IDX",          # merged grid: each lane loads its B-row index pair
    "nz_no_lds": "SRBCRS_EXPERIMENT_NZ_NO_LDS",         # nonzero sweep: gathers, values summed in registers
    "nz_no_b": "SRBCRS_EXPERIMENT_NZ_NO_B",             # nonzero sweep: LDS read-add-writes, no B gathers
    "nz_no_pin": "SRBCRS_NZ_NO_PIN",                    # nonzero sweep: no sched_barrier between loads and adds
    "nz_plain_c_store": "SRBCRS_NZ_PLAIN_C_STORE",      # nonzero sweep: C written with plain stores
}


def build_experiment(name: str) -> Path:
    """mask_amd/experiments/libmask_srbcrs_<name>.so with the macros of
    EXPERIMENTS[name] defined (objects under mask_amd/_build)."""
    from concurrent.futures import ThreadPoolExecutor
    macros = [f"-D{m}" if "=" in m else f"-D{m}=1" for m in EXPERIMENTS[name].split()]
    macros.append(f"-DSRBCRS_EXPERIMENT_TAG={name}")   # stamps srbcrs_version(); the loader refuses it
    hipcc = _hipcc()
    out_dir = PKG / "_build" / "experiments" / name
    out_dir.mkdir(parents=True, exist_ok=True)

    def compile_obj(src):
        obj = out_dir / (src.rsplit(".", 1)[0] + ".o")
        _run([hipcc, *DEVICE_FLAGS, *macros, f"-I{ROOT / 'include'}", "-x", "hip", "-c", str(CSRC / src),
              "-o", str(obj)])
        return str(obj)

    with ThreadPoolExecutor(max_workers=8) as ex:
        objs = list(ex.map(compile_obj, SOURCES))
    lib_dir = PKG / "experiments"
    lib_dir.mkdir(exist_ok=True)
    lib = lib_dir / f"libmask_srbcrs_{name}.so"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(lib), *objs, "-lpthread"])
    return lib


if __name__ == "__main__":
    if "--experiment" in sys.argv:
        print(build_experiment(sys.argv[sys.argv.index("--experiment") + 1]))
    elif "--sanitize" in sys.argv:
        print(build_sanitized())
    else:
        print(build(verbose="-v" in sys.argv))
