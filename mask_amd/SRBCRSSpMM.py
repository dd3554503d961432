"""Drop-in for the reference's ``SRBCRSSpMM`` torch extension module.

Same function names, argument order, return shapes and error messages as the
pybind module (examples/src_fp32/sr_bcrs/testbed/SRBCRSSpMM.cpp:194-204 and
SRBCRSSpMM_kernel.cu:172-557), backed by the gfx950 C ABI
(include/srbcrs.h) through ctypes.  Torch is used only for device memory and
the current stream.

Module state mirrors the reference's process-global cache
(SRBCRSSpMM_kernel.cu:27-45): ``preprocess_*`` creates a plan keyed by
``row_window_offset.data_ptr()`` and ``run_*`` looks it up by the same key.
"""
from __future__ import annotations

import ctypes
import os
import threading
from typing import Dict, List, Optional, Tuple

import torch

from . import _capi

Tensor = torch.Tensor

_POLICIES = ("row", "split", "strict_lb", "multi_bind", "auto")


def _check_input(t: Tensor, name: str) -> None:
    # CHECK_INPUT (SRBCRSSpMM.cpp:6-10)
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def check_operand(t: Tensor, name: str, device: torch.device) -> None:
    """A dense operand the kernels read or write through a raw pointer: a
    float32 tensor on ``device`` (a host tensor's address would reach the
    GPU), 2-D, row-major (unit column stride; any row stride >= width)."""
    if not isinstance(t, Tensor):
        raise RuntimeError(f"{name} must be a torch tensor")
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if t.device != torch.device(device):
        raise RuntimeError(f"{name} is on {t.device}, the plan on {device}")
    if t.dtype != torch.float32:
        raise RuntimeError(f"{name} must be float32")
    if t.dim() != 2 or (t.shape[1] > 1 and t.stride(1) != 1) or t.stride(0) < max(1, t.shape[1]):
        raise RuntimeError(f"{name} must be row-major 2-D")


def _stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


class Plan:
    """A device-resident SR-BCRS matrix (owns a ``srbcrs_plan``)."""

    def __init__(self, rowptr, colind, values, num_nodes: int, blk_h: int = 16, blk_w: int = 8,
                 device: Optional[torch.device] = None, packing: str = "column_condensed_dense",
                 dup: str = "last", row_order="identity", K: Optional[int] = None, convert_on: str = "device"):
        """CSR (device tensors, or host arrays) -> device-resident plan.

        The defaults are the reference's preprocess_gpu conversion.  The
        generated-operator packings take ``packing`` ("column_condensed_dense"
        / "active_fixed_blocks_dense"), ``dup`` ("last" / "sum"),
        ``row_order`` ("identity", "row_rcm", "first_col_sort",
        "jaccard_greedy", "sparse_rows", or an explicit new -> original
        sequence) and the column count ``K`` (required for fixed blocks).
        ``convert_on`` ("device" / "host") picks where a device CSR is
        converted for the canonical packing; the arrays are identical."""
        if convert_on not in ("device", "host"):
            raise ValueError("convert_on must be 'device' or 'host'")
        L = _capi.lib()
        on_dev = isinstance(rowptr, Tensor) and rowptr.is_cuda
        if on_dev:
            self.device = rowptr.device
        elif device is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        else:
            self.device = torch.device(device)
        self._keep = (rowptr, colind, values)
        nnz = int(colind.numel() if isinstance(colind, Tensor) else len(colind))
        h = ctypes.c_void_p()
        explicit = None
        if isinstance(row_order, str):
            order_code = _capi.ORDERS[row_order]
        else:
            import numpy as np
            explicit = np.ascontiguousarray(np.asarray(row_order), dtype=np.int32)
            order_code = _capi.ORDERS["explicit"]
        opts = _capi.PackOpts(int(blk_h), int(blk_w), _capi.PACKINGS[packing], _capi.DUPS[dup], order_code,
                              explicit.ctypes.data if explicit is not None else None,
                              int(explicit.shape[0]) if explicit is not None else 0, -1 if K is None else int(K))
        with torch.cuda.device(self.device):
            stream = _stream_handle(self.device) if on_dev else None
            _capi.check(L.srbcrs_plan_create_ex(_capi.ptr(rowptr), _capi.ptr(colind), _capi.ptr(values),
                                                int(num_nodes), nnz, ctypes.byref(opts),
                                                (1 if convert_on == "device" else 2) if on_dev else 0, stream,
                                                ctypes.byref(h)))
        self._h = h
        d = _capi.PlanDesc()
        _capi.check(L.srbcrs_plan_get(h, ctypes.byref(d)))
        self.desc = d
        self.num_nodes = int(num_nodes)
        self.nnz = nnz
        self.blk_h, self.blk_w = int(blk_h), int(blk_w)
        self.row_windows = int(d.row_windows)
        self.total_blocks = int(d.total_blocks)
        self.max_col = int(d.max_col)
        self.policy = ("row", 0)
        self.tuned_widths = set()   # widths srbcrs_plan_tune chose settings for (current schedule)
        self._sweep_refused = set()   # operand layouts the nonzero sweep refused (run_sweep_if_sparse)

    @property
    def handle(self):
        return self._h

    def set_schedule(self, policy: str = "row", param: int = 0) -> None:
        if (policy, param) == self.policy:
            return
        with torch.cuda.device(self.device):
            _capi.check(_capi.lib().srbcrs_plan_set_schedule(self._h, policy.encode(), int(param)))
        self.policy = (policy, param)
        self.tuned_widths = set()

    def block_fill(self) -> float:
        """nnz / (blocks * blk_h * blk_w): the stored-value density."""
        return self.nnz / max(1, self.total_blocks * self.blk_h * self.blk_w)

    def run_sweep_if_sparse(self, dense: Tensor, out: Tensor) -> bool:
        """The low-block-density dispatch of the CSR fallback (the vector
        kernel for low block density, threshold measured on an MI355X): on
        a 16x8 plan with the compact copy whose block fill is
        below SWEEP_FILL, run the nonzero sweep (grid order 5, default
        knobs) into out and return True.  The library refuses, before any
        launch, what the sweep cannot run (a split schedule, N, leading
        dimensions, alignment, B's extent); then, and on denser plans,
        return False and launch nothing.  Refusals are remembered per width
        and operand layout."""
        if self.blk_h != 16 or self.desc.stored_values < 0 or self.total_blocks == 0:
            return False
        if self.desc.stored_values >= SWEEP_FILL * self.total_blocks * self.blk_h * self.blk_w:
            return False
        key = (int(dense.shape[1]), int(dense.stride(0)), int(out.stride(0)), dense.data_ptr() % 16,
               out.data_ptr() % 16, self.policy)
        if key in self._sweep_refused:
            return False
        try:
            self.run(dense, out, grid_order=5)
        except _capi.SrbcrsError as e:
            if e.code != _capi.SRBCRS_EINVAL:
                raise
            self._sweep_refused.add(key)
            return False
        return True

    def _operands(self, dense: Tensor, out: Optional[Tensor]) -> Tensor:
        """Validate dense (and out, allocated when None) before any launch:
        float32 GPU tensors on the plan's device, 2-D with unit column
        stride, the same width, and out with at least num_nodes rows."""
        check_operand(dense, "dense", self.device)
        if out is None:
            out = torch.empty((self.num_nodes, dense.shape[1]), dtype=torch.float32, device=dense.device)
        check_operand(out, "out", self.device)
        if out.shape[1] != dense.shape[1]:
            raise RuntimeError("out and dense must have the same number of columns")
        if out.shape[0] < self.num_nodes:
            raise RuntimeError(f"out has {out.shape[0]} rows, the plan writes {self.num_nodes}")
        return out

    def run(self, dense: Tensor, out: Optional[Tensor] = None, depth: int = 0, tile_b: int = 0, wg_cols: int = 0,
            grid_order: int = 0, windows_per_wave: int = 0, a_operand: str = "default",
            b_stage: str = "default", relu: bool = False) -> Tensor:
        """out[:num_nodes] = A @ dense (relu(A @ dense) with relu=True, applied
        in the kernels' stores) on the current stream.  The keyword
        knobs are the kernel template parameters (srbcrs_run_opts; 0 =
        default; grid_order 1 = chunk-major, 2 = window-major, 3 = chunk sweep, 4 = merged
        windows ("row" schedule: windows_per_wave windows interleaved per wave), 5 = nonzero
        sweep (the vector kernel for low block density: one gather per stored value, tile_b
        values per sub-batch; its bits are the fp32 CSR product's); a_operand
        "compact" / "dense" picks the block-value copy the kernel reads; b_stage
        "registers" / "lds" where the ring holds the gathered B rows)."""
        out = self._operands(dense, out)
        opts = _capi.RunOpts(int(depth), int(tile_b), int(wg_cols), int(grid_order), int(windows_per_wave),
                             _capi.A_OPERANDS[a_operand], _capi.B_STAGES[b_stage],
                             _capi.EPILOGUE_RELU if relu else _capi.EPILOGUE_NONE)
        with torch.cuda.device(self.device):
            _capi.check(_capi.lib().srbcrs_run_ex(self._h, dense.data_ptr(), int(dense.shape[0]), int(dense.shape[1]),
                                                  int(dense.stride(0)), out.data_ptr(), int(out.stride(0)),
                                                  int(out.shape[0]), ctypes.byref(opts), _stream_handle(self.device)))
        return out

    def tune(self, dense: Tensor, out: Optional[Tensor] = None, reps: int = 3, nonzero_sweep: bool = False) -> dict:
        """Time the launch candidates for dense.shape[1] on this plan (see
        srbcrs_plan_tune) and keep the fastest for later default-knob runs
        at that width; returns the choice.  out (or a scratch tensor) is
        overwritten with A @ dense.  nonzero_sweep=True also times the
        nonzero sweep (srbcrs_plan_tune_ex, SRBCRS_TUNE_NONZERO_SWEEP),
        whose bits are the fp32 CSR product's."""
        out = self._operands(dense, out)
        best = _capi.RunOpts()
        flags = _capi.SRBCRS_TUNE_NONZERO_SWEEP if nonzero_sweep else 0
        with torch.cuda.device(self.device):
            _capi.check(_capi.lib().srbcrs_plan_tune_ex(self._h, dense.data_ptr(), int(dense.shape[0]),
                                                        int(dense.shape[1]), int(dense.stride(0)), out.data_ptr(),
                                                        int(out.stride(0)), int(out.shape[0]), int(reps), flags,
                                                        ctypes.byref(best), _stream_handle(self.device)))
        self.tuned_widths.add(int(dense.shape[1]))
        inv = {v: k for k, v in _capi.A_OPERANDS.items()}
        return {"depth": best.depth, "tile_b": best.tile_b, "wg_cols": best.wg_cols, "grid_order": best.grid_order,
                "windows_per_wave": best.windows_per_wave or 1, "a_operand": inv[best.a_operand],
                "b_stage": "lds" if best.b_stage == 2 else "registers"}

    def trim(self) -> None:
        """Free the device buffers the plan retired (srbcrs_plan_trim) after
        synchronizing the current stream; only when no captured graph of an
        earlier run will be replayed."""
        with torch.cuda.device(self.device):
            _capi.check(_capi.lib().srbcrs_plan_trim(self._h, _stream_handle(self.device)))

    def row_order(self):
        """The plan's row order (new -> original) as a numpy array."""
        import numpy as np
        out = np.zeros(max(self.num_nodes, 1), dtype=np.int32)
        n = ctypes.c_int32(0)
        _capi.check(_capi.lib().srbcrs_plan_row_order(self._h, out.ctypes.data, self.num_nodes, ctypes.byref(n)))
        return out[: n.value].copy()

    def block_values(self) -> Tensor:
        """The swizzled block values on the device (a copy)."""
        n = self.total_blocks * self.blk_h * self.blk_w
        out = torch.empty(n, dtype=torch.float32, device=self.device)
        with torch.cuda.device(self.device):
            _capi.check(_capi.lib().srbcrs_plan_export_values(self._h, out.data_ptr() if n else None, n,
                                                              _stream_handle(self.device)))
        return out

    def close(self) -> None:
        if getattr(self, "_h", None):
            _capi.lib().srbcrs_plan_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class _Entry:
    __slots__ = ("plan", "num_nodes", "num_edges", "use_16x8", "tensors", "exec_plan")

    def __init__(self, plan, num_nodes, num_edges, use_16x8, tensors):
        self.plan, self.num_nodes, self.num_edges, self.use_16x8, self.tensors = (
            plan, num_nodes, num_edges, use_16x8, tensors)
        self.exec_plan = None

    def executing_plan(self) -> "Plan":
        """The plan a run executes.  A 16x8 preprocess runs its own plan.  A
        32x32 preprocess (the base variant) keeps its 32x32 arrays -- the
        preprocess outputs -- but runs, by default, on a 16x8 plan of the same
        CSR, built on the device at the first run: the 16x8 layout pads less
        (3 % vs 6 % block fill on graphs) and was faster on every workload
        measured, full 16x8 blocks included.  SPARSENE_SRBCRS_BASE_NATIVE=1
        runs the 32x32 blocks themselves.  Either way C = A @ B within the
        fp32 gate; the bits of the two layouts differ (another summation
        order)."""
        if self.use_16x8 or os.environ.get("SPARSENE_SRBCRS_BASE_NATIVE", "0") == "1":
            return self.plan
        if self.exec_plan is None:
            rowptr, colind, values = self.tensors[:3]
            self.exec_plan = Plan(rowptr, colind, values, self.num_nodes, 16, 8)
        return self.exec_plan


_cache_mu = threading.Lock()
_cache: Dict[int, _Entry] = {}


def clear_cache() -> None:
    with _cache_mu:
        _cache.clear()


def _preprocess(colind: Tensor, rowptr: Tensor, values: Tensor, num_nodes: int, blk_h: int, blk_w: int,
                block_partition: Tensor, edge_to_col: Tensor, edge_to_row: Tensor, use_16x8: bool):
    for t, n in ((colind, "colind"), (rowptr, "rowptr"), (values, "values"), (block_partition, "block_partition"),
                 (edge_to_col, "edge_to_col"), (edge_to_row, "edge_to_row")):
        _check_input(t, n)
    if colind.dtype != torch.int32:
        raise RuntimeError("colind must be int32")
    if rowptr.dtype != torch.int32:
        raise RuntimeError("rowptr must be int32")
    if values.dtype != torch.float32:
        raise RuntimeError("values must be float32")
    if num_nodes < 1:
        raise RuntimeError("num_nodes must be positive")
    tile_m, tile_k = (16, 8) if use_16x8 else (32, 32)
    if blk_h != tile_m:
        raise RuntimeError(f"blk_h mismatch for SR-BCRS variant: expected {tile_m} got {blk_h}")
    if blk_w != tile_k:
        raise RuntimeError(f"blk_w mismatch for SR-BCRS variant: expected {tile_k} got {blk_w}")
    nnz = int(colind.numel())
    if values.numel() != nnz:
        raise RuntimeError("values length must equal colind length")
    plan = Plan(rowptr, colind, values, num_nodes, tile_m, tile_k)
    dev = colind.device
    total = plan.total_blocks
    mo = plan.row_windows
    i32 = dict(dtype=torch.int32, device=dev)
    row_window_offset = torch.empty(mo + 1, **i32)
    tcblocktile_id = torch.empty(total * tile_k, **i32)
    with torch.cuda.device(dev):
        st = _stream_handle(dev)
        _capi.check(_capi.lib().srbcrs_plan_export_index(plan.handle, row_window_offset.data_ptr(), mo + 1,
                                                         tcblocktile_id.data_ptr() if total else None,
                                                         total * tile_k, st))
        _capi.check(_capi.lib().srbcrs_plan_write_edges(plan.handle, block_partition.data_ptr(),
                                                        block_partition.numel(), edge_to_col.data_ptr(),
                                                        edge_to_col.numel(), edge_to_row.data_ptr(),
                                                        edge_to_row.numel(), st))
    tcblock_rowid = torch.zeros(total, **i32)
    tcblock_offset = torch.zeros(1, **i32)
    sparse_a_to_x_idx = torch.zeros(1, **i32)
    key = int(row_window_offset.data_ptr())
    with _cache_mu:
        # the entry keeps row_window_offset alive so the key stays unique
        _cache[key] = _Entry(plan, int(num_nodes), nnz, use_16x8,
                             (rowptr, colind, values, row_window_offset, tcblocktile_id))
    return row_window_offset, tcblock_rowid, tcblocktile_id, tcblock_offset, sparse_a_to_x_idx, total


# Block fill (stored values / (blocks * 128)) below which the nonzero sweep
# beats the tuned MFMA kernels at N = 512 on one MI355X (bench.py
# --sweep-crossover, 16 values per row, window-clustered columns; sustained ms,
# sweep / tuned MFMA): fill 0.062 0.136 / 0.213, 0.095 0.136 / 0.158, 0.137
# 0.135 / 0.121, 0.250 0.136 / 0.082.
SWEEP_FILL = 0.125


def _tile_b_for(n: int) -> int:
    """SRBCRS_TILE_B handling (SRBCRSSpMM_kernel.cu:435-475): validates the
    forced tile, else picks 64/32/16 by divisibility; 0 = none fits."""
    env = os.environ.get("SRBCRS_TILE_B")
    if env is not None:
        if env in ("64", "32", "16"):
            t = int(env)
            if n % t != 0:
                raise RuntimeError(f"SRBCRS_TILE_B={t} requires dense feature dim divisible by {t}, got {n}")
            return t
        if env != "auto":
            raise RuntimeError(f"Invalid SRBCRS_TILE_B={env}. Supported values: auto, 64, 32, 16")
    for t in (64, 32, 16):
        if n % t == 0:
            return t
    return 0


def _schedule_from_exeplan(exeplan: str) -> Optional[Tuple[str, int]]:
    """The reference ignores ``exeplan``; here "policy" or "policy:param"
    with policy in row/split/strict_lb/multi_bind selects the schedule and
    anything else is ignored.  SPARSENE_SRBCRS_SCHEDULE is the env form."""
    spec = (exeplan or "").strip() or os.environ.get("SPARSENE_SRBCRS_SCHEDULE", "").strip()
    if not spec:
        return None
    name, _, param = spec.partition(":")
    if name not in _POLICIES:
        return None
    return name, int(param) if param else 0


def _run(dense: Tensor, row_window_offset: Tensor, tcblocktile_id: Tensor, tcblock_offset: Tensor,
         sparse_a_to_x_idx: Tensor, num_nodes: int, num_edges: int, exeplan: str, use_16x8: bool) -> List[Tensor]:
    for t, n in ((dense, "dense"), (row_window_offset, "row_window_offset"), (tcblocktile_id, "tcblocktile_id"),
                 (tcblock_offset, "tcblock_offset"), (sparse_a_to_x_idx, "sparse_a_to_x_idx")):
        _check_input(t, n)
    if dense.dtype != torch.float32:
        raise RuntimeError("dense must be float32")
    if dense.dim() != 2:
        raise RuntimeError("dense must be 2-D")
    key = int(row_window_offset.data_ptr())
    with _cache_mu:
        entry = _cache.get(key)
    if entry is None:
        raise RuntimeError("run_SRBCRS cache miss. Call preprocess_gpu before run_SRBCRS.")
    if num_nodes != entry.num_nodes:
        raise RuntimeError(f"num_nodes mismatch between preprocess and run: {num_nodes} vs {entry.num_nodes}")
    if use_16x8 != entry.use_16x8:
        raise RuntimeError("SR-BCRS variant mismatch between preprocess and run")
    n = int(dense.shape[1])
    if n <= 0:
        return [torch.zeros((entry.num_nodes, 0), dtype=dense.dtype, device=dense.device)]
    tile_b = _tile_b_for(n)
    if tile_b == 0:
        raise RuntimeError(f"SR-BCRS requires dense feature dim divisible by 16/32/64, got {n}. "
                           "Please pad feature dim before run.")
    if entry.plan.total_blocks <= 0:
        raise RuntimeError("SR-BCRS has empty preprocessed blocks; CSR fallback disabled.")
    sched = _schedule_from_exeplan(exeplan)
    plan = entry.executing_plan()
    # no schedule requested: "auto" (split on heavy-tailed windows, else one task per window)
    plan.set_schedule(*(sched or ("auto", 0)))
    out = torch.empty((entry.num_nodes, n), dtype=torch.float32, device=dense.device)
    # the reference's CSR-fallback opt-in also admits the CSR product's bits
    # on the SR-BCRS path: the nonzero sweep, for low block density
    csr_ok = os.environ.get("SPARSENE_ALLOW_CSR_FALLBACK", "0") == "1"
    if os.environ.get("SPARSENE_SRBCRS_AUTOTUNE", "0") == "1" and n not in plan.tuned_widths:
        plan.tune(dense, out, nonzero_sweep=csr_ok)   # once per (width, schedule); the product lands in out
    elif n in plan.tuned_widths or not (csr_ok and plan.run_sweep_if_sparse(dense, out)):
        plan.run(dense, out)
    return [out]


# ---- the module's functions (SRBCRSSpMM.cpp:77-192) -------------------------

def preprocess_gpu(colind, rowptr, values, num_nodes, blk_h, blk_w, block_partition, edge_to_col, edge_to_row):
    """SR-BCRS preprocess base, 32x32 blocks."""
    return _preprocess(colind, rowptr, values, num_nodes, blk_h, blk_w, block_partition, edge_to_col,
                       edge_to_row, False)


def preprocess_gpu_16x8(colind, rowptr, values, num_nodes, blk_h, blk_w, block_partition, edge_to_col,
                        edge_to_row):
    """SR-BCRS preprocess 16x8."""
    return _preprocess(colind, rowptr, values, num_nodes, blk_h, blk_w, block_partition, edge_to_col,
                       edge_to_row, True)


def run_SRBCRS(dense, row_window_offset, tcblocktile_id, tcblock_offset, sparse_a_to_x_idx, num_nodes,
               num_edges, exeplan):
    return _run(dense, row_window_offset, tcblocktile_id, tcblock_offset, sparse_a_to_x_idx, num_nodes,
                num_edges, exeplan, False)


def run_SRBCRS_balance(dense, row_window_offset, tcblocktile_id, tcblock_offset, sparse_a_to_x_idx, num_nodes,
                       exeplan):
    return _run(dense, row_window_offset, tcblocktile_id, tcblock_offset, sparse_a_to_x_idx, num_nodes,
                int(sparse_a_to_x_idx.numel()), exeplan, False)


def run_SRBCRS_16x8(dense, row_window_offset, tcblocktile_id, tcblock_offset, sparse_a_to_x_idx, num_nodes,
                    num_edges, exeplan):
    return _run(dense, row_window_offset, tcblocktile_id, tcblock_offset, sparse_a_to_x_idx, num_nodes,
                num_edges, exeplan, True)


def run_SRBCRS_16x8_balance(dense, row_window_offset, tcblocktile_id, tcblock_offset, sparse_a_to_x_idx,
                            num_nodes, exeplan):
    return _run(dense, row_window_offset, tcblocktile_id, tcblock_offset, sparse_a_to_x_idx, num_nodes,
                int(sparse_a_to_x_idx.numel()), exeplan, True)


def plan_for(row_window_offset: Tensor) -> Plan:
    """The plan behind a preprocess result (for benchmarking / inspection)."""
    with _cache_mu:
        e = _cache.get(int(row_window_offset.data_ptr()))
    if e is None:
        raise RuntimeError("run_SRBCRS cache miss. Call preprocess_gpu before run_SRBCRS.")
    return e.plan


def csr_spmm(rowptr: Tensor, colind: Tensor, values: Tensor, dense: Tensor, num_rows: int,
             max_col: Optional[int] = None, out: Optional[Tensor] = None) -> Tensor:
    """CSR fallback kernel (csr_spmm_value_kernel, SRBCRSSpMM_kernel.cu:66-105)."""
    for t, n in ((rowptr, "rowptr"), (colind, "colind"), (values, "values"), (dense, "dense")):
        _check_input(t, n)
    if max_col is None:
        max_col = int(colind.max().item()) if colind.numel() else -1
    n = int(dense.shape[1])
    if out is None:
        out = torch.empty((num_rows, n), dtype=torch.float32, device=dense.device)
    with torch.cuda.device(dense.device):
        _capi.check(_capi.lib().srbcrs_csr_spmm(rowptr.data_ptr(), colind.data_ptr(), values.data_ptr(), int(num_rows),
                                                int(colind.numel()), int(max_col), dense.data_ptr(),
                                                int(dense.shape[0]), n, int(dense.stride(0)), out.data_ptr(),
                                                int(out.stride(0)), _stream_handle(dense.device)))
    return out
