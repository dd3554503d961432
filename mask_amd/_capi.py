"""ctypes binding of ``libmask_srbcrs.so`` (declarations: include/srbcrs.h).

The library is built in-tree by ``mask_amd.build``.  Loading never falls back
to anything else: a missing library raises, so a GPU run cannot silently take
a non-HIP path.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

import os as _os

# MASK_AMD_SRBCRS_LIB selects another build of the same library (the host
# sanitizer build of mask_amd.build --sanitize); default: the in-tree one.
LIB_PATH = Path(_os.environ.get("MASK_AMD_SRBCRS_LIB") or Path(__file__).resolve().parent / "libmask_srbcrs.so")
# Decomposition builds (mask_amd.build --experiment) leave out part of the
# SpMM's work on purpose and stamp srbcrs_version() with "+experiment:<name>".
# The loader refuses such a library unless this variable is "1" (timing runs
# of those builds only).
ALLOW_EXPERIMENT_ENV = "MASK_AMD_ALLOW_EXPERIMENT"

SRBCRS_OK = 0
SRBCRS_EINVAL = -1
SRBCRS_EHIP = -2
SRBCRS_ENOMEM = -3
SRBCRS_ESTATE = -4
SRBCRS_TUNE_NONZERO_SWEEP = 1

# Every symbol include/srbcrs.h declares (checked by the CPU test suite).
EXPORTS = (
    "srbcrs_last_error", "srbcrs_version",
    "srbcrs_convert_count", "srbcrs_convert_fill",
    "srbcrs_plan_create", "srbcrs_plan_destroy", "srbcrs_plan_get", "srbcrs_plan_write_edges",
    "srbcrs_plan_export_index", "srbcrs_plan_export_values",
    "srbcrs_schedule_build", "srbcrs_schedule_info", "srbcrs_schedule_export", "srbcrs_schedule_destroy",
    "srbcrs_plan_set_schedule", "srbcrs_run", "srbcrs_run_ex", "srbcrs_csr_spmm",
    "srbcrs_row_order", "srbcrs_pack_count", "srbcrs_pack_fill", "srbcrs_plan_create_ex", "srbcrs_plan_row_order",
    "srbcrs_plan_tune", "srbcrs_plan_tune_ex", "srbcrs_shard_windows", "srbcrs_run_noalloc", "srbcrs_noalloc_scratch_floats",
    "srbcrs_plan_trim",
)

_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_f32p = ctypes.POINTER(ctypes.c_float)
_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64


class PlanDesc(ctypes.Structure):
    _fields_ = [
        ("num_nodes", ctypes.c_int32),
        ("blk_h", ctypes.c_int32),
        ("blk_w", ctypes.c_int32),
        ("row_windows", ctypes.c_int32),
        ("max_col", ctypes.c_int32),
        ("device", ctypes.c_int32),
        ("nnz", ctypes.c_int64),
        ("total_blocks", ctypes.c_int64),
        ("d_soff", ctypes.c_void_p),
        ("d_sidx", ctypes.c_void_p),
        ("d_val", ctypes.c_void_p),
        ("packed_rows", ctypes.c_int64),
        ("d_row_map", ctypes.c_void_p),
        ("packing", ctypes.c_int32),
        ("dup_policy", ctypes.c_int32),
        ("stored_values", ctypes.c_int64),
        ("d_a_words", ctypes.c_void_p),
        ("d_a_packed", ctypes.c_void_p),
    ]


class PackOpts(ctypes.Structure):
    _fields_ = [("blk_h", ctypes.c_int32), ("blk_w", ctypes.c_int32), ("packing", ctypes.c_int32),
                ("dup_policy", ctypes.c_int32), ("row_order", ctypes.c_int32), ("order", ctypes.c_void_p),
                ("order_len", ctypes.c_int32), ("K", ctypes.c_int32)]


ORDERS = {"identity": 0, "row_rcm": 1, "first_col_sort": 2, "jaccard_greedy": 3, "sparse_rows": 4, "explicit": 5}
PACKINGS = {"column_condensed_dense": 0, "active_fixed_blocks_dense": 1}
DUPS = {"last": 0, "sum": 1}


class RunOpts(ctypes.Structure):
    _fields_ = [("depth", ctypes.c_int32), ("tile_b", ctypes.c_int32), ("wg_cols", ctypes.c_int32),
                ("grid_order", ctypes.c_int32), ("windows_per_wave", ctypes.c_int32),
                ("a_operand", ctypes.c_int32), ("b_stage", ctypes.c_int32), ("epilogue", ctypes.c_int32)]


A_OPERANDS = {"default": 0, "compact": 1, "dense": 2}
B_STAGES = {"default": 0, "registers": 1, "lds": 2}
EPILOGUE_NONE, EPILOGUE_RELU = 0, 1   # srbcrs_run_opts.epilogue


class SrbcrsError(RuntimeError):
    """A failing status from the C ABI; the message is srbcrs_last_error()."""

    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH.name} is not built; run `python -m mask_amd.build` (hipcc, gfx950). "
            "There is no non-HIP fallback.")
    L = ctypes.CDLL(str(LIB_PATH))
    sig = {
        "srbcrs_last_error": ([], ctypes.c_char_p),
        "srbcrs_version": ([], ctypes.c_char_p),
        "srbcrs_convert_count": ([_vp, _vp, _i32, _i64, _i32, _i32, _vp, _i64p], ctypes.c_int),
        "srbcrs_convert_fill": ([_vp, _vp, _vp, _i32, _i64, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp],
                                ctypes.c_int),
        "srbcrs_plan_create": ([_vp, _vp, _vp, _i32, _i64, _i32, _i32, _i32, _vp, ctypes.POINTER(_vp)],
                               ctypes.c_int),
        "srbcrs_plan_destroy": ([_vp], None),
        "srbcrs_plan_get": ([_vp, ctypes.POINTER(PlanDesc)], ctypes.c_int),
        "srbcrs_plan_write_edges": ([_vp, _vp, _i64, _vp, _i64, _vp, _i64, _vp], ctypes.c_int),
        "srbcrs_plan_export_index": ([_vp, _vp, _i64, _vp, _i64, _vp], ctypes.c_int),
        "srbcrs_plan_export_values": ([_vp, _vp, _i64, _vp], ctypes.c_int),
        "srbcrs_schedule_build": ([_vp, _i32, ctypes.c_char_p, _i32, ctypes.POINTER(_vp)], ctypes.c_int),
        "srbcrs_schedule_info": ([_vp, _i32p, _i32p, _i32p, _i32p], ctypes.c_int),
        "srbcrs_schedule_export": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp], ctypes.c_int),
        "srbcrs_schedule_destroy": ([_vp], None),
        "srbcrs_plan_set_schedule": ([_vp, ctypes.c_char_p, _i32], ctypes.c_int),
        "srbcrs_run": ([_vp, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp], ctypes.c_int),
        "srbcrs_run_ex": ([_vp, _vp, _i64, _i64, _i64, _vp, _i64, _i64, ctypes.POINTER(RunOpts), _vp],
                          ctypes.c_int),
        "srbcrs_row_order": ([_vp, _vp, _i32, _i64, _i32, _i32, _vp, _i32p], ctypes.c_int),
        "srbcrs_pack_count": ([_vp, _vp, _i32, _i64, ctypes.POINTER(PackOpts), _vp, _i64p], ctypes.c_int),
        "srbcrs_pack_fill": ([_vp, _vp, _vp, _i32, _i64, ctypes.POINTER(PackOpts), _vp, _vp, _vp], ctypes.c_int),
        "srbcrs_plan_create_ex": ([_vp, _vp, _vp, _i32, _i64, ctypes.POINTER(PackOpts), _i32, _vp,
                                   ctypes.POINTER(_vp)], ctypes.c_int),
        "srbcrs_plan_row_order": ([_vp, _vp, _i32, _i32p], ctypes.c_int),
        "srbcrs_shard_windows": ([_vp, _i32, _i32, _vp], ctypes.c_int),
        "srbcrs_plan_tune": ([_vp, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i32, ctypes.POINTER(RunOpts), _vp],
                             ctypes.c_int),
        "srbcrs_plan_tune_ex": ([_vp, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i32, _i32, ctypes.POINTER(RunOpts),
                                 _vp], ctypes.c_int),
        "srbcrs_csr_spmm": ([_vp, _vp, _vp, _i32, _i64, _i32, _vp, _i64, _i64, _i64, _vp, _i64, _vp],
                            ctypes.c_int),
        "srbcrs_run_noalloc": ([_vp, _vp, _i64, _i64, _i64, _vp, _i64, _i64, ctypes.POINTER(RunOpts), _vp],
                               ctypes.c_int),
        "srbcrs_noalloc_scratch_floats": ([], ctypes.c_size_t),
        "srbcrs_plan_trim": ([_vp, _vp], ctypes.c_int),
    }
    for name, (args, res) in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res
    check_not_experiment(L.srbcrs_version().decode(), LIB_PATH)
    _lib = L
    return L


def check_not_experiment(version: str, path) -> None:
    """Refuse a decomposition build (results wrong on purpose) unless the
    caller opted in through MASK_AMD_ALLOW_EXPERIMENT=1."""
    if "+experiment:" in version and _os.environ.get(ALLOW_EXPERIMENT_ENV) != "1":
        raise RuntimeError(
            f"{path} is a decomposition build ({version}): its SpMM results are wrong on purpose. "
            f"Set {ALLOW_EXPERIMENT_ENV}=1 only to time it.")


def check(code: int) -> None:
    if code != SRBCRS_OK:
        msg = lib().srbcrs_last_error().decode(errors="replace")
        raise SrbcrsError(code, msg)


def ptr(a) -> int:
    """Raw address of a numpy array or torch tensor (None -> NULL)."""
    if a is None:
        return None
    if isinstance(a, np.ndarray):
        return a.ctypes.data
    return a.data_ptr()


# ---- host helpers (no GPU involved) ---------------------------------------

def convert_host(rowptr, colind, values, num_nodes: int, blk_h: int = 16, blk_w: int = 8) -> dict:
    """CSR -> SR-BCRS on the host through the library's converter."""
    L = lib()
    rowptr = np.ascontiguousarray(rowptr, dtype=np.int32)
    colind = np.ascontiguousarray(colind, dtype=np.int32)
    values = np.ascontiguousarray(values, dtype=np.float32)
    nnz = int(colind.shape[0])
    mo = (num_nodes + blk_h - 1) // blk_h
    soff = np.zeros(mo + 1, dtype=np.int32)
    total = ctypes.c_int64(0)
    check(L.srbcrs_convert_count(ptr(rowptr), ptr(colind), num_nodes, nnz, blk_h, blk_w, ptr(soff),
                                 ctypes.byref(total)))
    t = int(total.value)
    sidx = np.zeros(max(t * blk_w, 1), dtype=np.int32)
    val = np.zeros(max(t * blk_h * blk_w, 1), dtype=np.float32)
    bp = np.zeros(max(mo, 1), dtype=np.int32)
    e2r = np.zeros(max(nnz, 1), dtype=np.int32)
    e2c = np.zeros(max(nnz, 1), dtype=np.int32)
    check(L.srbcrs_convert_fill(ptr(rowptr), ptr(colind), ptr(values), num_nodes, nnz, blk_h, blk_w, ptr(soff),
                                ptr(sidx), ptr(val), ptr(bp), ptr(e2r), ptr(e2c)))
    return dict(soff=soff, sidx=sidx[: t * blk_w], val=val[: t * blk_h * blk_w], block_partition=bp[:mo],
                edge_to_row=e2r[:nnz], edge_to_col=e2c[:nnz], total=t)


def shard_windows(soff, n_shards: int) -> np.ndarray:
    """Balanced contiguous window ranges (see srbcrs_shard_windows)."""
    soff = np.ascontiguousarray(soff, dtype=np.int32)
    bounds = np.zeros(int(n_shards) + 1, np.int32)
    check(lib().srbcrs_shard_windows(ptr(soff), soff.shape[0] - 1, int(n_shards), ptr(bounds)))
    return bounds


def build_schedule(soff, policy: str, param: int = 0) -> dict:
    """Host schedule tables (see srbcrs_schedule_build in include/srbcrs.h)."""
    L = lib()
    soff = np.ascontiguousarray(soff, dtype=np.int32)
    h = ctypes.c_void_p()
    check(L.srbcrs_schedule_build(ptr(soff), soff.shape[0] - 1, policy.encode(), int(param), ctypes.byref(h)))
    try:
        ng, nt, ns, nr = (ctypes.c_int32() for _ in range(4))
        check(L.srbcrs_schedule_info(h, ctypes.byref(ng), ctypes.byref(nt), ctypes.byref(ns), ctypes.byref(nr)))
        out = dict(group_off=np.zeros(ng.value + 1, np.int32), task_begin=np.zeros(nt.value, np.int32),
                   task_end=np.zeros(nt.value, np.int32), task_window=np.zeros(nt.value, np.int32),
                   task_slot=np.zeros(nt.value, np.int32), red_window=np.zeros(nr.value, np.int32),
                   red_slot_off=np.zeros(nr.value + 1, np.int32))
        check(L.srbcrs_schedule_export(h, *(ptr(out[k]) for k in ("group_off", "task_begin", "task_end",
                                                                   "task_window", "task_slot", "red_window",
                                                                   "red_slot_off"))))
        out["n_slots"] = ns.value
        return out
    finally:
        L.srbcrs_schedule_destroy(h)


def row_order_host(rowptr, colind, num_nodes: int, K: int, method: str) -> np.ndarray:
    """The library's row order (new -> original) for `method`."""
    L = lib()
    rowptr = np.ascontiguousarray(rowptr, dtype=np.int32)
    colind = np.ascontiguousarray(colind, dtype=np.int32)
    out = np.zeros(max(num_nodes, 1), dtype=np.int32)
    n = ctypes.c_int32(0)
    check(L.srbcrs_row_order(ptr(rowptr), ptr(colind), num_nodes, int(colind.shape[0]), int(K), ORDERS[method],
                             ptr(out), ctypes.byref(n)))
    return out[: n.value].copy()


def pack_host(rowptr, colind, values, num_nodes: int, K: int, order=None, blk_h: int = 16, blk_w: int = 8,
              packing: str = "column_condensed_dense", dup: str = "sum") -> dict:
    """The library's packer with an explicit (or identity) row order."""
    L = lib()
    rowptr = np.ascontiguousarray(rowptr, dtype=np.int32)
    colind = np.ascontiguousarray(colind, dtype=np.int32)
    values = np.ascontiguousarray(values, dtype=np.float32)
    o = PackOpts(blk_h, blk_w, PACKINGS[packing], DUPS[dup], 0, None, 0, int(K))
    rows = num_nodes
    if order is not None:
        order = np.ascontiguousarray(order, dtype=np.int32)
        o.row_order, o.order, o.order_len = ORDERS["explicit"], order.ctypes.data, order.shape[0]
        rows = order.shape[0]
    nnz = int(colind.shape[0])
    soff = np.zeros((rows + blk_h - 1) // blk_h + 1, dtype=np.int32)
    total = ctypes.c_int64(0)
    check(L.srbcrs_pack_count(ptr(rowptr), ptr(colind), num_nodes, nnz, ctypes.byref(o), ptr(soff),
                              ctypes.byref(total)))
    t = total.value
    sidx = np.zeros(max(t * blk_w, 1), dtype=np.int32)
    val = np.zeros(max(t * blk_h * blk_w, 1), dtype=np.float32)
    check(L.srbcrs_pack_fill(ptr(rowptr), ptr(colind), ptr(values), num_nodes, nnz, ctypes.byref(o), ptr(soff),
                             ptr(sidx), ptr(val)))
    return dict(soff=soff, sidx=sidx[: t * blk_w], val=val[: t * blk_h * blk_w], total=t)
