"""HIP emitter: NVIR SR_BCRS program + strategy knobs -> gfx950 operator.

Replaces the reference's NVIR -> CUDA emitter for ``format_name ==
"SR_BCRS"`` (``NvIrCodeGenerator.dump_nvop_program``,
python/sparsene/op_gen/nvir/codegen.py:2324-2386, with the skeletons of
templates.py).  Instead of lowering each NVIR op to CuTe/PTX text, the
emitter maps the program's attributes and the strategy knobs onto the
template parameters of the hand-written gfx950 kernels
(``mask_amd/csrc/srbcrs_stream.hpp``) and emits a small HIP translation unit
that instantiates them behind a C ABI:

  const char* sparsene_generated_metadata(void)            JSON
  int sparsene_generated_run(...)                           row schedule
  int sparsene_generated_run_tasks(...)                     task-mapped
  int sparsene_generated_reduce(...)                        split reduction

Knob mapping (strategy_agent.py:81-130 -> template parameters):
  tensor_placement.tile_b (16/32/64)      -> VEC = tile_b / 16
  pipeline.enable_async_pipeline = False  -> DEPTH 2 (shortest ring)
  pipeline.max_wait_prior 0..3            -> DEPTH 2, 2, 4, 8
  pipeline.stage_shifts [s0, s1]          -> DEPTH 2 ** max(s0, s1) (at least 2)
  runtime_schedule.execution_policy       -> schedule (row / strict_lb / multi_bind / auto)
  runtime_schedule.task_group_tiles       -> strict_lb workload
  runtime_schedule.runtime_max_tiles_per_segment -> split cap
  tensor_placement.materialize_b_array_ref_to_smem -> BSTAGE 1: B staged
      through LDS by direct-to-LDS loads (vector width 4 only; measured
      slower than the register ring on every workload, so strategies for
      gfx950 should set it False)
The cp.async mode, swizzle and COO placement knobs have no counterpart
(recorded as ignored in the metadata): direct-to-LDS loads need no swizzle
(each wave reads its own slot conflict-free) and the block indices and
values are read through the scalar cache and registers.
"""
from __future__ import annotations

import ctypes
import hashlib
import json
import re
from dataclasses import asdict, dataclass
from pathlib import Path
from typing import Any, Dict, Mapping, Optional

from .backend_registry import BackendPlan

CSRC = Path(__file__).resolve().parent / "csrc"


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
    b_lds = bool(_get(strategy, "tensor_placement", "materialize_b_array_ref_to_smem", default=False)) and vec == 4
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

int operand_check(const void* B, const void* C, int N, long long ldb, long long ldc) {{
  if (N <= 0 || N % kWCOLS) return -1;
  if (ldb < N || ldc < N || ldb % kVEC || ldc % kVEC) return -1;
  if ((reinterpret_cast<uintptr_t>(B) | reinterpret_cast<uintptr_t>(C)) % (4 * kVEC)) return -1;
  return 0;
}}

template <class Src>
int launch(const Src& src, int n_groups, const float* B, float* C, float* partial, const int* sidx,
           const float* val, int M, int N, long long ldb, long long ldc, hipStream_t st) {{
  const int n_chunks = (N + kChunkCols - 1) / kChunkCols;
  const long long nwg = (long long)n_groups * n_chunks;
  if (nwg == 0) return 0;
  if (nwg > 0x7fffffffLL) return -1;
  hipLaunchKernelGGL((srbcrs::spmm_stream<Src, kBH, kBW, kVEC, kG, kWAVES, kDEPTH, srbcrs::DenseA, kBSTAGE>),
                     dim3((unsigned)nwg), dim3(64 * kWAVES), 0, st, src, B, C, partial, sidx,
                     srbcrs::DenseA{{val}}, M, N, (int64_t)ldb,
                     (int64_t)ldc, n_chunks, kChunkMajor);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}}
}}  // namespace

extern "C" const char* sparsene_generated_metadata(void) {{
  return R"JSON({metadata})JSON";
}}

// C = A * B over the row schedule (one task per BH-row window).  M counts
// packed rows; rowmap (or null) sends packed row p to output row rowmap[p].
extern "C" int sparsene_generated_run(const float* B, float* C, const int* soff, const int* sidx,
                                      const float* val, int M, int N, int Mo, long long ldb,
                                      long long ldc, const int* rowmap, void* stream) {{
  if (operand_check(B, C, N, ldb, ldc)) return -1;
  srbcrs::RowTasks src{{soff, Mo, 1, rowmap}};
  return launch(src, Mo, B, C, nullptr, sidx, val, M, N, ldb, ldc, static_cast<hipStream_t>(stream));
}}

// Task-mapped run (split / strict_lb / multi_bind tables from srbcrs_schedule_build).
extern "C" int sparsene_generated_run_tasks(const float* B, float* C, float* partial, const int* sidx,
                                            const float* val, const int* group_off,
                                            const int* task_begin, const int* task_end,
                                            const int* task_window, const int* task_slot,
                                            int n_groups, int M, int N, long long ldb,
                                            long long ldc, const int* rowmap, void* stream) {{
  if (operand_check(B, C, N, ldb, ldc)) return -1;
  srbcrs::TableTasks src{{group_off, task_begin, task_end, task_window, task_slot, rowmap}};
  return launch(src, n_groups, B, C, partial, sidx, val, M, N, ldb, ldc, static_cast<hipStream_t>(stream));
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
                     M, N, (int64_t)ldc, rowmap);
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
                notes: Optional[Dict[str, Any]] = None) -> str:
    """Render the HIP translation unit for one operator."""
    params.validate()
    spec = _check_specialized(specialized or {})
    spec_lines = "\n".join(f"constexpr int {k} = {v};" for k, v in sorted(spec.items()))
    meta = {"format_name": "SR_BCRS", "operator": name, "target": "gfx950", "wave_size": 64,
            "kernel_params": asdict(params), "wave_cols": params.wave_cols, "specialized_parameters": spec}
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
    ``name`` / ``attrs`` members): attrs["format_name"] must be "SR_BCRS";
    attrs["strategy_decision"], attrs["specialized_parameters"] and
    attrs["launch_contract"] are honoured as in codegen.py:2324-2386.  The
    block shape comes from the BackendPlan (select_backend)."""

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
            if v is not None:
                ignored[knob] = v
        notes = {"ignored_knobs": ignored,
                 "launch_contract": "wave64 (one 64-lane wave per 128-column chunk)"
                 if sync == "warp" else "workgroup"}
        params = params_from_strategy(attrs.get("strategy_decision"), self.backend_plan)
        name = str(getattr(program, "name", None) or attrs.get("name") or "sr_bcrs")
        return emit_source(params, name=name, specialized=specialized, notes=notes)


def operator_sha256(source: str) -> str:
    return hashlib.sha256(source.encode()).hexdigest()


def compile_operator(source: str, out_path: Path) -> Path:
    """hipcc the generated unit into a shared library next to out_path."""
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
        L.sparsene_generated_run.argtypes = [vp] * 5 + [i32, i32, i32, i64, i64, vp, vp]
        L.sparsene_generated_run.restype = ctypes.c_int
        L.sparsene_generated_run_tasks.argtypes = [vp] * 10 + [i32, i32, i32, i64, i64, vp, vp]
        L.sparsene_generated_run_tasks.restype = ctypes.c_int
        L.sparsene_generated_reduce.argtypes = [vp] * 4 + [i32, i32, i32, i64, vp, vp]
        L.sparsene_generated_reduce.restype = ctypes.c_int
        L.sparsene_generated_zero_rows.argtypes = [vp, vp, i32, i32, i64, vp]
        L.sparsene_generated_zero_rows.restype = ctypes.c_int
        self._lib = L
        self.metadata = json.loads(L.sparsene_generated_metadata().decode())
        self.params = KernelParams(**self.metadata["kernel_params"])
        self._tables = {}

    def run(self, plan, dense, out=None, schedule: Optional[str] = None, schedule_param: Optional[int] = None):
        import numpy as np
        import torch
        from . import _capi
        if (plan.blk_h, plan.blk_w) != (self.params.blk_m, self.params.blk_k):
            raise RuntimeError("operator block shape does not match the plan")
        if dense.shape[0] <= plan.max_col:
            raise RuntimeError("dense has fewer rows than the matrix's columns")
        if out is None:
            out = torch.empty((plan.num_nodes, dense.shape[1]), dtype=torch.float32, device=dense.device)
        st = torch.cuda.current_stream(dense.device).cuda_stream
        d = plan.desc
        pol = schedule or self.params.schedule
        param = self.params.schedule_param if schedule_param is None else schedule_param
        if pol == "auto":
            soff = plan_soff(plan)
            lens = np.diff(soff)
            p95 = int(np.sort(lens)[min(lens.size - 1, max(0, int(np.ceil(lens.size * 0.95)) - 1))]) if lens.size else 0
            pol = "strict_lb" if lens.size and lens.max() > max(64, 4 * max(p95, 1)) else "row"
        N = int(dense.shape[1])
        P = int(d.packed_rows)
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
            rc = self._lib.sparsene_generated_run(dense.data_ptr(), out.data_ptr(), d.d_soff, d.d_sidx, d.d_val,
                                                  P, N, plan.row_windows, dense.stride(0),
                                                  out.stride(0), d.d_row_map, st)
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
            dense.data_ptr(), out.data_ptr(), partial.data_ptr(), d.d_sidx, d.d_val, dev["group_off"].data_ptr(),
            dev["task_begin"].data_ptr(), dev["task_end"].data_ptr(), dev["task_window"].data_ptr(),
            dev["task_slot"].data_ptr(), tab["group_off"].size - 1, P, N, dense.stride(0), N, d.d_row_map, st)
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


def lower_format_operator(spec: Mapping[str, Any], operator_path: Path, strategy: Any = None,
                          target: str = "gfx950", tile_n: int = 64) -> Dict[str, Any]:
    """spec -> select_backend -> HIP source -> compiled operator.  Returns a
    dict in the spirit of generate_custom_format_operators.py:88-157
    (operator path, sha256, backend plan, kernel parameters)."""
    from .backend_registry import select_backend
    plan = select_backend(spec, target=target, tile_n=tile_n)
    program = {"attrs": {"format_name": plan.codegen_format_name, "strategy_decision": strategy,
                         "name": spec.get("format_name", "sr_bcrs")}}
    source = HipCodeGenerator(plan).dump_nvop_program(program)
    path = compile_operator(source, Path(operator_path))
    return {"operator_path": str(path), "source_path": str(path.with_suffix(".hip")),
            "operator_sha256": operator_sha256(source), "backend_plan": plan.to_dict(),
            "kernel_params": asdict(params_from_strategy(strategy, plan))}
