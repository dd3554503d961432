"""HIP emitter: NVIR SR_BCRS program + strategy knobs -> gfx950 operator.

Replaces the reference's NVIR -> CUDA emitter for ``format_name ==
"SR_BCRS"`` (``NvIrCodeGenerator.dump_nvop_program``,
python/sparsene/op_gen/nvir/codegen.py:2324-2386, called from
``compiler_driver._dump_code``, compiler_driver.py:2190-2200).  Instead of
lowering each NVIR op to CuTe/PTX text, the emitter checks the program's
gmem interface against the operands the gfx950 kernel templates
(``mask_amd/csrc/srbcrs_stream.hpp``) consume, maps the strategy knobs onto
their template parameters, and emits a small HIP translation unit that
instantiates them behind a C ABI:

  const char* sparsene_generated_metadata(void)            JSON
  int sparsene_generated_run(...)                           row schedule
  int sparsene_generated_run_tasks(...)                     task-mapped
  int sparsene_generated_reduce(...)                        split reduction
  int sparsene_generated_zero_rows(...)                     rows a packing omits

The run entries take the reference kernel's parameters first, in its order:
the gmem pointers sorted by name, then the varlens sorted
(codegen.py:2092-2140; the SR_BCRS program's interface is recorded in
tests/golden/sr_bcrs_nvir_abi.json), i.e. dB_val, dC_val, dval_len_offset,
dval_new, dval_sidx_new, K, M, Mo, N, nnz_dim_K -- as launched by the
reference's bridge (examples/src_fp32/acc/testbed/custom_format_e2e.cu:
980-990).  Mo is the length of dval_len_offset (row windows + 1), as that
call site passes it.

Knob mapping (strategy_agent.py:81-130 -> template parameters):
  tensor_placement.tile_b (16/32/64)      -> VEC = tile_b / 16
  pipeline.enable_async_pipeline = False  -> DEPTH 2 (shortest ring)
  pipeline.max_wait_prior 0..3            -> DEPTH 2, 2, 4, 8
  pipeline.stage_shifts [s0, s1]          -> DEPTH 2 ** max(s0, s1) (at least 2)
  runtime_schedule.execution_policy       -> schedule (row / strict_lb / multi_bind / auto)
  runtime_schedule.task_group_tiles       -> strict_lb workload
  runtime_schedule.runtime_max_tiles_per_segment -> split cap
  tensor_placement.b_array_ref_mode == "global_load_lds" (with
      materialize_b_array_ref_to_smem) -> BSTAGE 1: B staged through LDS by
      direct-to-LDS loads (vector width 4 only).  Any other B placement,
      the reference's default shared-memory staging included, maps to the
      register ring: on gfx950 it is faster on every workload measured.
The cp.async mode, swizzle and COO placement knobs have no counterpart
(recorded in the metadata): the block indices and values are read through
the scalar cache and registers.  Each operator holds both A sources (the
reference's value array, or the plan's compact copy) and picks at run time.
"""
from __future__ import annotations

import ctypes
import dataclasses
import hashlib
import json
import re
from dataclasses import asdict, dataclass
from pathlib import Path
from typing import Any, Dict, Mapping, Optional

from .backend_registry import BackendPlan

CSRC = Path(__file__).resolve().parent / "csrc"

# The gmem interface of the reference's SR_BCRS NVIR program (generate.py
# registers it; nvir/generate.py:175-203 holds its shape and layout rules):
# name -> (dtype, number of dims, what the gfx950 kernel reads there).
SR_BCRS_GMEM_ABI = {
    "B_val": ("float", 2, "B, K x N row-major"),
    "C_val": ("float", 2, "C, the output (written as M x N row-major)"),
    "val_len_offset": ("int", 1, "row-window block offsets (soff / row_window_offset)"),
    "val_new": ("float", 3, "block values, BLK_M x BLK_K per block, Swizzle<2,2,3>"),
    "val_sidx_new": ("int", 2, "block column indices, BLK_K per block"),
}
SR_BCRS_VARLENS = ("K", "M", "Mo", "N", "nnz_dim_K")


@dataclass(frozen=True)
class KernelParams:
    """Template parameters of ``srbcrs::spmm_stream`` plus launch policy."""
    blk_m: int = 16
    blk_k: int = 8
    vec: int = 4             # columns per lane per MFMA sweep
    col_groups: int = 2      # G
    waves: int = 1           # waves per workgroup (128 columns each for 16x8/VEC 4/G 2)
    depth: int = 2           # units in flight per wave
    chunk_major: bool = True
    b_lds: bool = False      # stage B through LDS (direct-to-LDS loads) instead of registers
    schedule: str = "auto"   # row / split / strict_lb / multi_bind / auto
    schedule_param: int = 0

    @property
    def wave_cols(self) -> int:
        return 16 * self.vec * self.col_groups

    def validate(self) -> None:
        if (self.blk_m, self.blk_k) not in {(16, 8), (32, 32)}:
            raise ValueError(f"unsupported block {self.blk_m}x{self.blk_k}")
        if self.vec not in (1, 2, 4) or self.col_groups not in (1, 2) or self.waves not in (1, 2, 4):
            raise ValueError("vec must be 1/2/4, col_groups 1/2, waves 1/2/4")
        if self.depth not in (2, 4, 8):
            raise ValueError("depth must be 2, 4 or 8")
        if self.b_lds and self.vec != 4:
            raise ValueError("LDS staging of B needs vec 4 (16-byte direct-to-LDS loads)")
        if self.schedule not in ("row", "split", "strict_lb", "multi_bind", "auto"):
            raise ValueError(f"unknown schedule {self.schedule}")


def _get(obj: Any, *path, default=None):
    for p in path:
        if obj is None:
            return default
        obj = obj.get(p) if isinstance(obj, Mapping) else getattr(obj, p, None)
    return default if obj is None else obj


def params_from_strategy(strategy: Any = None, plan: Optional[BackendPlan] = None) -> KernelParams:
    """Map a StrategyDecision (object or dict) onto kernel template parameters."""
    bm = plan.physical_blk_m if plan else 16
    bk = plan.physical_blk_k if plan else 8
    tile_b = int(_get(strategy, "tensor_placement", "tile_b", default=64))
    if tile_b not in (16, 32, 64):
        tile_b = 64
    vec = tile_b // 16
    depth = 2
    if _get(strategy, "pipeline", "enable_async_pipeline", default=True):
        mwp = _get(strategy, "pipeline", "max_wait_prior")
        if mwp is not None and int(mwp) in (0, 1, 2, 3):
            depth = max(depth, {0: 2, 1: 2, 2: 4, 3: 8}[int(mwp)])
        shifts = _get(strategy, "pipeline", "stage_shifts", default=[]) or []
        if len(shifts) == 2 and all(int(s) in (1, 2, 3) for s in shifts):
            depth = max(depth, min(8, 2 ** max(int(s) for s in shifts)))
    policy = str(_get(strategy, "runtime_schedule", "execution_policy", default="auto"))
    if policy not in ("row", "strict_lb", "multi_bind", "auto"):
        policy = "auto"
    param = 0
    if policy == "strict_lb":
        param = int(_get(strategy, "runtime_schedule", "task_group_tiles", default=64))
    cap = int(_get(strategy, "runtime_schedule", "runtime_max_tiles_per_segment", default=0))
    if policy == "auto" and cap > 0:
        policy, param = "split", cap
    g = 2 if (bm, bk) == (16, 8) and vec == 4 else 1
    b_lds = (bool(_get(strategy, "tensor_placement", "materialize_b_array_ref_to_smem", default=False))
             and _get(strategy, "tensor_placement", "b_array_ref_mode") == "global_load_lds" and vec == 4)
    kp = KernelParams(blk_m=bm, blk_k=bk, vec=vec, col_groups=g, waves=1, depth=depth, chunk_major=True,
                      b_lds=b_lds, schedule=policy, schedule_param=param)
    kp.validate()
    return kp


_IDENT = re.compile(r"[A-Za-z_][A-Za-z0-9_]*")


def _check_specialized(specialized: Mapping[str, Any]) -> Dict[str, int]:
    # the reference's rule (codegen.py:2325-2333)
    out = {}
    for name, value in specialized.items():
        if (not isinstance(name, str) or not _IDENT.fullmatch(name) or name in {"BLK_M", "BLK_N", "BLK_K"}
                or isinstance(value, bool) or not isinstance(value, int) or value <= 0):
            raise ValueError(f"invalid specialized parameter: {name!r}")
        out[name] = value
    return out


def _gmem_table(program: Any) -> Dict[str, Dict[str, str]]:
    """{name: {"dtype", "shape"}} of a program's gmem_inouts (NvOpProgram
    GmemInout objects, or the dict form of lower_format_operator's result)."""
    raw = getattr(program, "gmem_inouts", None)
    if raw is None and isinstance(program, Mapping):
        raw = program.get("gmem_inouts")
    out = {}
    for name, io_ in (raw or {}).items():
        dtype = _get(io_, "dtype")
        shape = _get(io_, "shape")
        out[str(name)] = {"dtype": str(dtype), "shape": str(shape)}
    return out


def _shape_rank(shape: str) -> int:
    s = shape.strip()
    if s.startswith("(") and s.endswith(")"):
        s = s[1:-1]
    return len([p for p in s.split(",") if p.strip()]) if s else 0


def check_gmem_abi(program: Any) -> Dict[str, Dict[str, str]]:
    """The program's gmem interface must be exactly the operand set of the
    gfx950 SR-BCRS kernel (names, element types, ranks), so that what the
    middle end lowered is what the emitted operator reads.  A program
    without gmem_inouts (attributes only) is taken to have that interface.
    Returns the interface used."""
    table = _gmem_table(program)
    if not table:
        return {n: {"dtype": d, "shape": f"rank {r}"} for n, (d, r, _) in SR_BCRS_GMEM_ABI.items()}
    missing = sorted(set(SR_BCRS_GMEM_ABI) - set(table))
    extra = sorted(set(table) - set(SR_BCRS_GMEM_ABI))
    if missing or extra:
        raise ValueError(f"SR_BCRS gmem interface mismatch: missing {missing}, unexpected {extra}")
    for name, (dtype, rank, _) in SR_BCRS_GMEM_ABI.items():
        if table[name]["dtype"] != dtype:
            raise ValueError(f"gmem {name}: dtype {table[name]['dtype']}, the kernel reads {dtype}")
        got = _shape_rank(table[name]["shape"])
        if got != rank:
            raise ValueError(f"gmem {name}: rank {got}, the kernel reads rank {rank}")
    return table


_SOURCE = """// Generated by mask_amd.emitter (HIP, gfx950) for SR_BCRS operator '{name}'.
// Do not edit: regenerate from the NVIR program and strategy.
#define SPARSENE_GENERATED_TILE_B {tile_b}
#define SPARSENE_GENERATED_SUPPORTS_TASK_MAPPING 1
#define SPARSENE_GENERATED_WAVE_SIZE 64
#define SPARSENE_GENERATED_THREADS_PER_BLOCK {threads}
#define SPARSENE_GENERATED_BLK_M {bm}
#define SPARSENE_GENERATED_BLK_K {bk}
#define SPARSENE_GENERATED_PIPELINE_DEPTH {depth}
#define SPARSENE_GENERATED_WAVE_COLS {wcols}
{specialized}
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "srbcrs_stream.hpp"

namespace {{
constexpr int kBH = {bm}, kBW = {bk}, kVEC = {vec}, kG = {g}, kWAVES = {waves}, kDEPTH = {depth};
constexpr int kChunkMajor = {chunk_major};
constexpr int kBSTAGE = {bstage};   // 0: B ring in registers, 1: staged through LDS
constexpr int kWCOLS = 16 * kVEC * kG;
constexpr int kChunkCols = kWAVES * kWCOLS;

// Operand checks shared by the run entries (status -1 on failure, nothing launched).
int operand_check(const void* B, const void* C, const int* offsets, const int* sidx, int K, int M, int Mo,
                  int N, int nnz_dim_K, long long ldb, long long ldc, long long c_rows, const int* rowmap,
                  const void* a_words, const void* a_packed) {{
  if (!B || !C || !offsets || K <= 0 || M < 0 || Mo < 1 || nnz_dim_K < 0) return -1;
  if (nnz_dim_K > 0 && !sidx) return -1;
  const long long windows = Mo - 1;
  if ((long long)M > windows * kBH || (long long)M <= (windows - 1) * kBH) return -1;
  if (N <= 0 || N % kWCOLS) return -1;
  if (ldb < N || ldc < N || ldb % kVEC || ldc % kVEC) return -1;
  if (!rowmap && c_rows < M) return -1;
  if ((reinterpret_cast<uintptr_t>(B) | reinterpret_cast<uintptr_t>(C)) % (4 * kVEC)) return -1;
  if ((a_words == nullptr) != (a_packed == nullptr)) return -1;
  return 0;
}}

template <class AF, class Src>
int launch(const Src& src, const AF& af, int n_groups, const float* B, float* C, float* partial, const int* sidx,
           int M, int N, long long ldb, long long ldc, hipStream_t st) {{
  const int n_chunks = (N + kChunkCols - 1) / kChunkCols;
  const long long nwg = (long long)n_groups * n_chunks;
  if (nwg == 0) return 0;
  if (nwg > 0x7fffffffLL) return -1;
  hipLaunchKernelGGL((srbcrs::spmm_stream<Src, kBH, kBW, kVEC, kG, kWAVES, kDEPTH, AF, kBSTAGE>),
                     dim3((unsigned)nwg), dim3(64 * kWAVES), 0, st, src, B, C, partial, sidx, af, M, N,
                     (int64_t)ldb, (int64_t)ldc, n_chunks, kChunkMajor);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}}

// The A source: the compact copy when the caller hands it over, else the value array.
template <class Src>
int launch_a(const Src& src, int n_groups, const float* B, float* C, float* partial, const int* sidx,
             const float* val, const void* a_words, const float* a_packed, int M, int N, long long ldb,
             long long ldc, hipStream_t st) {{
  if (a_words)
    return launch(src, srbcrs::CompactA{{static_cast<const uint2*>(a_words), a_packed}}, n_groups, B, C, partial,
                  sidx, M, N, ldb, ldc, st);
  return launch(src, srbcrs::DenseA{{val}}, n_groups, B, C, partial, sidx, M, N, ldb, ldc, st);
}}
}}  // namespace

extern "C" const char* sparsene_generated_metadata(void) {{
  return R"JSON({metadata})JSON";
}}

// C = A * B over the row schedule (one task per BH-row window).  The first ten
// parameters are the reference kernel's, in its order: B (K x N), C, the
// row-window block offsets (Mo = windows + 1 entries), the block values, the
// block column indices, K, M (packed rows), Mo, N, nnz_dim_K (blocks).  Then
// ldb / ldc (row strides), c_rows (rows of C's storage, >= M without a row
// map), rowmap (packed row p -> output row rowmap[p], or null), the plan's
// compact copy of the values (a_words / a_packed, both or neither) and the
// stream.
extern "C" int sparsene_generated_run(const float* dB_val, float* dC_val, const int* dval_len_offset,
                                      const float* dval_new, const int* dval_sidx_new, int K, int M, int Mo,
                                      int N, int nnz_dim_K, long long ldb, long long ldc, long long c_rows,
                                      const int* rowmap, const void* a_words, const float* a_packed,
                                      void* stream) {{
  if (operand_check(dB_val, dC_val, dval_len_offset, dval_sidx_new, K, M, Mo, N, nnz_dim_K, ldb, ldc, c_rows,
                    rowmap, a_words, a_packed))
    return -1;
  if (!a_words && nnz_dim_K > 0 && !dval_new) return -1;
  srbcrs::RowTasks src{{dval_len_offset, Mo - 1, 1, rowmap}};
  return launch_a(src, Mo - 1, dB_val, dC_val, nullptr, dval_sidx_new, dval_new, a_words, a_packed, M, N, ldb,
                  ldc, static_cast<hipStream_t>(stream));
}}

// Task-mapped run: the reference's task kernel parameters (B, C, offsets,
// values, columns, then the task tables, task_slot in place of its atomic
// flag: -1 = store into C, else the partial slot) followed by the varlens;
// then the group count and the partial buffer (slots x BH rows x ldc) that
// sparsene_generated_reduce sums into C.
extern "C" int sparsene_generated_run_tasks(const float* dB_val, float* dC_val, const int* dval_len_offset,
                                            const float* dval_new, const int* dval_sidx_new,
                                            const int* task_begin, const int* task_end, const int* task_window,
                                            const int* task_slot, const int* group_off, int K, int M, int Mo,
                                            int N, int nnz_dim_K, int n_groups, float* partial, long long ldb,
                                            long long ldc, long long c_rows, const int* rowmap,
                                            const void* a_words, const float* a_packed, void* stream) {{
  if (operand_check(dB_val, dC_val, dval_len_offset, dval_sidx_new, K, M, Mo, N, nnz_dim_K, ldb, ldc, c_rows,
                    rowmap, a_words, a_packed))
    return -1;
  if (n_groups < 0 || (n_groups > 0 && (!task_begin || !task_end || !task_window || !task_slot || !group_off)))
    return -1;
  if (!a_words && nnz_dim_K > 0 && !dval_new) return -1;
  srbcrs::TableTasks src{{group_off, task_begin, task_end, task_window, task_slot, rowmap}};
  return launch_a(src, n_groups, dB_val, dC_val, partial, dval_sidx_new, dval_new, a_words, a_packed, M, N, ldb,
                  ldc, static_cast<hipStream_t>(stream));
}}

// Deterministic reduction of the partial tiles into C (tile_rows = BH).
extern "C" int sparsene_generated_reduce(const float* partial, float* C, const int* red_window,
                                         const int* red_slot_off, int n_red, int M, int N,
                                         long long ldc, const int* rowmap, void* stream) {{
  if (n_red == 0) return 0;
  if (N % kVEC || ldc % kVEC) return -1;
  long long total = (long long)n_red * kBH * (N / kVEC);
  long long blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(srbcrs::segment_reduce<kVEC>, dim3((unsigned)blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), partial, C, red_window, red_slot_off, n_red, kBH,
                     M, N, (int64_t)ldc, rowmap, 0);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}}

// Zero the output rows a sparse-row packing leaves out.
extern "C" int sparsene_generated_zero_rows(float* C, const int* rows, int n_rows, int N, long long ldc,
                                            void* stream) {{
  if (n_rows == 0 || N == 0) return 0;
  long long total = (long long)n_rows * N;
  long long blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(srbcrs::zero_rows<float>, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     C, rows, n_rows, N, (int64_t)ldc);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}}
"""


def emit_source(params: KernelParams, name: str = "sr_bcrs", specialized: Optional[Mapping[str, int]] = None,
                notes: Optional[Dict[str, Any]] = None, gmem: Optional[Mapping[str, Any]] = None) -> str:
    """Render the HIP translation unit for one operator."""
    params.validate()
    spec = _check_specialized(specialized or {})
    spec_lines = "\n".join(f"constexpr int {k} = {v};" for k, v in sorted(spec.items()))
    gmem = dict(gmem) if gmem else {n: {"dtype": d} for n, (d, _, _) in SR_BCRS_GMEM_ABI.items()}
    meta = {"format_name": "SR_BCRS", "operator": name, "target": "gfx950", "wave_size": 64,
            "kernel_params": asdict(params), "wave_cols": params.wave_cols, "specialized_parameters": spec,
            "gmem_inouts": gmem, "kernel_parameter_order":
                [f"d{n}" for n in sorted(gmem)] + list(SR_BCRS_VARLENS),
            "a_sources": ["dense", "compact"]}
    if notes:
        meta["notes"] = notes
    return _SOURCE.format(name=name, tile_b=16 * params.vec, threads=64 * params.waves, bm=params.blk_m,
                          bk=params.blk_k, depth=params.depth, wcols=params.wave_cols, specialized=spec_lines,
                          vec=params.vec, g=params.col_groups, waves=params.waves,
                          chunk_major=int(params.chunk_major), bstage=int(params.b_lds),
                          metadata=json.dumps(meta, sort_keys=True))


class HipCodeGenerator:
    """Drop-in for NvIrCodeGenerator.dump_nvop_program on SR_BCRS programs.

    ``program`` is the reference's NvOpProgram (or any object with the same
    ``name`` / ``attrs`` / ``gmem_inouts`` members): attrs["format_name"]
    must be "SR_BCRS"; its gmem interface must be the kernel's operand set
    (check_gmem_abi); attrs["strategy_decision"],
    attrs["specialized_parameters"] and attrs["launch_contract"] are
    honoured as in codegen.py:2324-2386.  The block shape comes from the
    BackendPlan (select_backend), 16x8 without one."""

    def __init__(self, backend_plan: Optional[BackendPlan] = None):
        self.backend_plan = backend_plan

    def dump_nvop_program(self, program: Any) -> str:
        attrs = getattr(program, "attrs", None)
        if attrs is None and isinstance(program, Mapping):
            attrs = program.get("attrs", {})
        attrs = attrs or {}
        fmt = attrs.get("format_name")
        if fmt != "SR_BCRS":
            raise NotImplementedError(f"the gfx950 HIP emitter lowers SR_BCRS programs only, got {fmt!r}")
        gmem = check_gmem_abi(program)
        specialized = attrs.get("specialized_parameters", {}) or {}
        if not isinstance(specialized, Mapping):
            raise ValueError("specialized_parameters must be a dictionary")
        contract = attrs.get("launch_contract", {}) or {}
        sync = contract.get("synchronization")
        if sync not in (None, "block", "warp"):
            raise ValueError(f"unsupported generated synchronization scope: {sync}")
        ignored = {}
        tp = _get(attrs.get("strategy_decision"), "tensor_placement")
        for knob in ("enable_b_array_ref_cp_async", "b_array_ref_mode",
                     "b_smem_swizzle", "coo_idx_output_mem", "coo_val_output_mem", "coo_load_mode",
                     "coo_restore_swizzle"):
            v = _get(tp, knob)
            if v is not None and not (knob == "b_array_ref_mode" and v == "global_load_lds"):
                ignored[knob] = v
        params = params_from_strategy(attrs.get("strategy_decision"), self.backend_plan)
        notes = {"ignored_knobs": ignored,
                 "b_placement": "lds (global_load_lds)" if params.b_lds else "registers",
                 "launch_contract": "wave64 (one 64-lane wave per column chunk)"
                 if sync == "warp" else "workgroup"}
        name = str(getattr(program, "name", None) or attrs.get("name") or "sr_bcrs")
        return emit_source(params, name=name, specialized=specialized, notes=notes, gmem=gmem)


def operator_sha256(source: str) -> str:
    return hashlib.sha256(source.encode()).hexdigest()


def compile_operator(source: str, out_path: Path) -> Path:
    """hipcc the generated unit into a shared library out_path (the source
    is written next to it with the .hip suffix)."""
    from .build import DEVICE_FLAGS, _hipcc, _run
    out_path = Path(out_path)
    out_path.parent.mkdir(parents=True, exist_ok=True)
    src = out_path.with_suffix(".hip")
    src.write_text(source)
    tmp = out_path.with_suffix(".so.tmp")
    _run([_hipcc(), *DEVICE_FLAGS, f"-I{CSRC}", "-shared", "-o", str(tmp), str(src)])
    tmp.replace(out_path)
    return out_path


class GeneratedOperator:
    """A compiled operator; runs on a ``mask_amd.SRBCRSSpMM.Plan``'s arrays."""

    def __init__(self, path: Path):
        self.path = Path(path)
        L = ctypes.CDLL(str(self.path))
        vp, i32, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong
        L.sparsene_generated_metadata.restype = ctypes.c_char_p
        L.sparsene_generated_run.argtypes = [vp] * 5 + [i32] * 5 + [i64] * 3 + [vp] * 4
        L.sparsene_generated_run.restype = ctypes.c_int
        L.sparsene_generated_run_tasks.argtypes = [vp] * 10 + [i32] * 6 + [vp] + [i64] * 3 + [vp] * 4
        L.sparsene_generated_run_tasks.restype = ctypes.c_int
        L.sparsene_generated_reduce.argtypes = [vp] * 4 + [i32, i32, i32, i64, vp, vp]
        L.sparsene_generated_reduce.restype = ctypes.c_int
        L.sparsene_generated_zero_rows.argtypes = [vp, vp, i32, i32, i64, vp]
        L.sparsene_generated_zero_rows.restype = ctypes.c_int
        self._lib = L
        self.metadata = json.loads(L.sparsene_generated_metadata().decode())
        self.params = KernelParams(**self.metadata["kernel_params"])
        self._tables = {}

    def _gmem(self, dense, out, desc):
        """The five gmem pointers in the order the operator's metadata
        declares (the reference kernel's: sorted by gmem name), looked up by
        name so that no call site can transpose two of them."""
        by_name = {"dB_val": dense.data_ptr(), "dC_val": out.data_ptr(), "dval_len_offset": desc.d_soff,
                   "dval_new": desc.d_val, "dval_sidx_new": desc.d_sidx}
        order = self.metadata["kernel_parameter_order"][:5]
        if sorted(order) != sorted(by_name):
            raise RuntimeError(f"operator declares gmem operands {order}, expected {sorted(by_name)}")
        return tuple(by_name[n] for n in order)

    def resolve_schedule(self, plan, schedule: Optional[str] = None, schedule_param: Optional[int] = None):
        """(policy, param) a run uses.  "auto" is resolved by the library's own
        rule (srbcrs_schedule_build), so both paths pick the same schedule
        and give the same bits."""
        pol = schedule or self.params.schedule
        param = self.params.schedule_param if schedule_param is None else schedule_param
        return pol, param

    def run(self, plan, dense, out=None, schedule: Optional[str] = None, schedule_param: Optional[int] = None,
            a_operand: str = "default"):
        import numpy as np
        import torch
        from . import _capi
        from .SRBCRSSpMM import check_operand
        if (plan.blk_h, plan.blk_w) != (self.params.blk_m, self.params.blk_k):
            raise RuntimeError("operator block shape does not match the plan")
        check_operand(dense, "dense", plan.device)
        if dense.shape[0] <= plan.max_col:
            raise RuntimeError("dense has fewer rows than the matrix's columns")
        if out is None:
            out = torch.empty((plan.num_nodes, dense.shape[1]), dtype=torch.float32, device=dense.device)
        check_operand(out, "out", plan.device)
        if out.shape[1] != dense.shape[1]:
            raise RuntimeError("out and dense must have the same number of columns")
        if out.shape[0] < plan.num_nodes:
            raise RuntimeError(f"out has {out.shape[0]} rows, the plan writes {plan.num_nodes}")
        if a_operand not in ("default", "compact", "dense"):
            raise ValueError("a_operand must be default, compact or dense")
        d = plan.desc
        stored = int(d.stored_values)
        has_compact = bool(d.d_a_words) or plan.total_blocks == 0
        if a_operand == "compact" and not has_compact:
            raise RuntimeError("the plan has no compact copy of its block values")
        # the library's default: compact for 16x8 blocks at most half full
        use_compact = a_operand == "compact" or (
            a_operand == "default" and has_compact and plan.blk_h == 16
            and 2 * stored <= plan.total_blocks * plan.blk_h * plan.blk_w)
        aw = d.d_a_words if use_compact and plan.total_blocks else None
        ap = d.d_a_packed if use_compact and plan.total_blocks else None
        st = torch.cuda.current_stream(dense.device).cuda_stream
        pol, param = self.resolve_schedule(plan, schedule, schedule_param)
        N = int(dense.shape[1])
        P = int(d.packed_rows)
        Mo = plan.row_windows + 1
        K = int(dense.shape[0])
        zk = ("zero", id(plan))
        if zk not in self._tables:
            order = plan.row_order()
            mask = np.ones(plan.num_nodes, bool)
            mask[order] = False
            self._tables[zk] = (torch.from_numpy(np.nonzero(mask)[0].astype(np.int32)).to(dense.device), plan)
        zero = self._tables[zk][0]
        if zero.numel():
            if self._lib.sparsene_generated_zero_rows(out.data_ptr(), zero.data_ptr(), zero.numel(), N,
                                                      out.stride(0), st):
                raise RuntimeError("generated zero-fill failed")
        if pol == "row":
            rc = self._lib.sparsene_generated_run(*self._gmem(dense, out, d),
                                                  K, P, Mo, N, plan.total_blocks, dense.stride(0), out.stride(0),
                                                  out.shape[0], d.d_row_map, aw, ap, st)
            if rc:
                raise RuntimeError(f"generated operator rejected the operands (status {rc})")
            return out
        key = (id(plan), pol, param)
        if key not in self._tables:
            tab = _capi.build_schedule(plan_soff(plan), pol, param)
            dev = {k: torch.from_numpy(v).to(dense.device) for k, v in tab.items() if k != "n_slots"}
            self._tables[key] = (tab, dev, plan)
        tab, dev, _ = self._tables[key]
        if out.stride(0) != N:
            raise RuntimeError("task-mapped runs need a dense-packed output")
        partial = torch.empty((max(tab["n_slots"], 1) * plan.blk_h, N), dtype=torch.float32, device=dense.device)
        rc = self._lib.sparsene_generated_run_tasks(
            *self._gmem(dense, out, d), dev["task_begin"].data_ptr(),
            dev["task_end"].data_ptr(), dev["task_window"].data_ptr(), dev["task_slot"].data_ptr(),
            dev["group_off"].data_ptr(), K, P, Mo, N, plan.total_blocks, tab["group_off"].size - 1,
            partial.data_ptr(), dense.stride(0), N, out.shape[0], d.d_row_map, aw, ap, st)
        if rc:
            raise RuntimeError(f"generated operator rejected the operands (status {rc})")
        rc = self._lib.sparsene_generated_reduce(partial.data_ptr(), out.data_ptr(), dev["red_window"].data_ptr(),
                                                 dev["red_slot_off"].data_ptr(), tab["red_window"].size,
                                                 P, N, N, d.d_row_map, st)
        if rc:
            raise RuntimeError(f"generated reduction failed (status {rc})")
        return out


def plan_soff(plan):
    """row_window_offset of a plan, on the host."""
    import torch
    from . import _capi
    n = plan.row_windows + 1
    t = torch.empty(n, dtype=torch.int32, device=plan.device)
    _capi.check(_capi.lib().srbcrs_plan_export_index(plan.handle, t.data_ptr(), n, None, 0,
                                                     torch.cuda.current_stream(plan.device).cuda_stream))
    return t.cpu().numpy()


# ---- the compiler-side entry (generate_custom_format_operators.py:88-157) -------------

def _jsonable(value: Any) -> Any:
    if dataclasses.is_dataclass(value) and not isinstance(value, type):
        return dataclasses.asdict(value)
    if isinstance(value, Mapping):
        return {str(k): _jsonable(v) for k, v in value.items()}
    if isinstance(value, (list, tuple)):
        return [_jsonable(v) for v in value]
    if value is None or isinstance(value, (str, int, float, bool)):
        return value
    if hasattr(value, "__dict__"):
        return {k: _jsonable(v) for k, v in vars(value).items() if not k.startswith("_")}
    return str(value)


def _write_text(path: Path, value: Any) -> None:
    path.write_text(value if isinstance(value, str) else str(value), encoding="utf-8")


def _reference_program(format_obj: Any, codegen_format_name: str, ir_dir: Path, strategy_dir: Path,
                       strategy_decision: Any, specialized_parameters: Optional[Mapping[str, int]]):
    """The reference's Format -> RTS -> Computent -> OPIR -> NVIR middle end
    (generate_custom_format_operators.py:112-146), unchanged, for a Format
    object of the reference DSL.  Needs the reference's ``sparsene``
    package on the path (a sparsene checkout); this package does not ship it."""
    try:
        from sparsene.op_gen.computent.computent import computent_from_rts
        from sparsene.op_gen.nvir.generate import generate_nvir
        from sparsene.op_gen.opir.cValFlattenPass import CValFlattenPass
        from sparsene.op_gen.opir.generate import generate_from_computent
        from sparsene.op_gen.opir.varlenLoweringPass import VarlenLoweringPass
        from sparsene.op_gen.strategy_agent import StrategyConfig
        from sparsene.transform.rts import derive_rts
    except ImportError as exc:
        raise RuntimeError("lowering a Format object needs the sparsene compiler package (Format -> NVIR "
                           "middle end); pass a format spec mapping to lower without it") from exc
    rts = derive_rts(format_obj)
    _write_text(ir_dir / "01_rts.txt", rts)
    computent = computent_from_rts(codegen_format_name, rts)
    _write_text(ir_dir / "02_computent.txt", computent)
    opir = generate_from_computent(computent)
    _write_text(ir_dir / "03_opir.txt", opir)
    lowered = VarlenLoweringPass(op_builder=None, varlen2LenArrayTable=computent.varlen2LenArrayTable).run(opir)
    _write_text(ir_dir / "04_varlen_lowered_opir.txt", lowered)
    flattened = CValFlattenPass(op_builder=None).run(lowered)
    _write_text(ir_dir / "05_cval_flattened_opir.txt", flattened)
    return generate_nvir(
        opir=flattened, format_name=codegen_format_name,
        strategy_config=(StrategyConfig(provider="heuristic", log_dir=str(strategy_dir))
                         if strategy_decision is None else None),
        strategy_decision_override=strategy_decision,
        strategy_log_dir_override=str(strategy_dir) if strategy_decision is not None else None,
        specialized_parameters=specialized_parameters)


class SpecProgram:
    """The program the emitter lowers for a format spec mapping (no sparsene
    middle end): the SR_BCRS gmem interface of the reference's NVIR program
    and the attributes its generator sets (format name, strategy, launch
    contract)."""

    def __init__(self, name: str, strategy_decision: Any = None):
        self.name = name
        self.gmem_inouts = {n: {"dtype": d, "shape": "(" + ", ".join(["_"] * r) + ")"}
                            for n, (d, r, _) in SR_BCRS_GMEM_ABI.items()}
        self.attrs = {"format_name": "SR_BCRS", "strategy_decision": strategy_decision,
                      "launch_contract": {"threads_per_block": 64, "synchronization": "warp"}}

    def __str__(self) -> str:
        return json.dumps({"name": self.name, "gmem_inouts": self.gmem_inouts,
                           "attrs": _jsonable(self.attrs)}, indent=1, sort_keys=True)


def lower_format_operator(*, format_obj: Any, codegen_format_name: str, operator_path: Path, ir_dir: Path,
                          strategy_dir: Path, strategy_decision: Any = None,
                          specialized_parameters: Optional[Dict[str, int]] = None,
                          preserve_scalar_offset_divisors: tuple = (),
                          explicit_sequential_iteration: bool = False,
                          diagnostic_program_transform=None,
                          backend_plan: Optional[BackendPlan] = None,
                          target: str = "gfx950", tile_n: int = 64) -> Dict[str, Any]:
    """Lower a format through the gfx950 HIP emitter: the keyword signature
    and result keys of the reference's lower_format_operator
    (python/test/generate_custom_format_operators.py:88-157).

    ``format_obj`` is either a Format object of the reference DSL (lowered by
    the reference's own middle end, which must then be importable) or a
    format spec mapping (``levels`` / ``atomic`` / ``params``, as
    select_backend consumes; lowered to the SR_BCRS program interface
    directly).  The HIP source goes to ``operator_path`` (with a ``.so``
    suffix, the source goes next to it as ``.hip``) and is compiled to the
    shared library beside it.  Returns operator_sha256 (of the written
    source), lowered_block_barriers (0: wave64 kernels have no block
    barriers), strategy_decision and gmem_inouts, plus operator_path /
    source_path / backend_plan / kernel_params."""
    from .backend_registry import select_backend
    if codegen_format_name != "SR_BCRS":
        raise NotImplementedError(f"the gfx950 HIP emitter lowers SR_BCRS programs only, got "
                                  f"{codegen_format_name!r}")
    operator_path = Path(operator_path)
    ir_dir, strategy_dir = Path(ir_dir), Path(strategy_dir)
    ir_dir.mkdir(parents=True, exist_ok=True)
    strategy_dir.mkdir(parents=True, exist_ok=True)
    if isinstance(format_obj, Mapping):
        backend_plan = backend_plan or select_backend(format_obj, target=target, tile_n=tile_n)
        program = SpecProgram(str(format_obj.get("format_name", "sr_bcrs")), strategy_decision)
        _write_text(ir_dir / "06_nvir_before_pipeline.txt", program)
    else:
        program = _reference_program(format_obj, codegen_format_name, ir_dir, strategy_dir, strategy_decision,
                                     specialized_parameters)
        _write_text(ir_dir / "06_nvir_before_pipeline.txt", program)
    if explicit_sequential_iteration:
        program.attrs["explicit_sequential_iteration"] = True
    if specialized_parameters:
        program.attrs["specialized_parameters"] = dict(specialized_parameters)
    if preserve_scalar_offset_divisors:
        program.attrs["preserve_scalar_offset_divisors"] = tuple(preserve_scalar_offset_divisors)
    if diagnostic_program_transform is not None:
        diagnostic_program_transform(program)
    source = HipCodeGenerator(backend_plan).dump_nvop_program(program)
    so_path = operator_path if operator_path.suffix == ".so" else operator_path.with_suffix(".so")
    compile_operator(source, so_path)
    src_path = so_path.with_suffix(".hip")
    if operator_path.suffix != ".so" and operator_path != src_path:
        operator_path.write_text(source, encoding="utf-8")
        src_path = operator_path
    strategy = program.attrs.get("strategy_decision")
    return {
        "operator_sha256": hashlib.sha256(src_path.read_bytes()).hexdigest(),
        "lowered_block_barriers": 0,
        "strategy_decision": _jsonable(strategy),
        "gmem_inouts": _gmem_table(program),
        "operator_path": str(so_path),
        "source_path": str(src_path),
        "backend_plan": backend_plan.to_dict() if backend_plan else None,
        "kernel_params": asdict(params_from_strategy(strategy, backend_plan)),
    }
