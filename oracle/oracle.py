"""numpy/ctypes front of the CPU oracle (``srbcrs_oracle.c``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg, and only as the checker.  The product
package ``mask_amd`` never imports it.

Each wrapper names the reference file:line its C function restates (paths
relative to the reference root; see the C file's header for abbreviations).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle_srbcrs.so"
_lib = None

_i32p = ctypes.POINTER(ctypes.c_int32)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)


def build() -> Path:
    """Compile the oracle with gcc (no reference sources involved)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not _LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(_LIB_PATH))
    lib.oracle_swizzle.argtypes = [ctypes.c_int]
    lib.oracle_swizzle.restype = ctypes.c_int
    lib.oracle_convert_count.argtypes = [_i32p, _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _i32p]
    lib.oracle_convert_count.restype = ctypes.c_int64
    lib.oracle_convert_fill.argtypes = [_i32p, _i32p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        _i32p, _i32p, _f32p, _i32p, _i32p, _i32p]
    lib.oracle_convert_fill.restype = None
    lib.oracle_csr_spmm_f64.argtypes = [_i32p, _i32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int, _f64p, _f64p]
    lib.oracle_csr_spmm_f64.restype = None
    lib.oracle_csr_spmm_f32.argtypes = [_i32p, _i32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int, _f32p,
                                        ctypes.c_int]
    lib.oracle_csr_spmm_f32.restype = None
    lib.oracle_max_threads.argtypes = []
    lib.oracle_max_threads.restype = ctypes.c_int
    lib.oracle_strict_lb.argtypes = [ctypes.c_int, ctypes.c_int, _i32p, ctypes.c_int, _i32p, _i32p, _i32p,
                                     _i32p]
    lib.oracle_strict_lb.restype = ctypes.c_int
    lib.oracle_multi_bind.argtypes = [ctypes.c_int, _i32p, _i32p, _i32p, _i32p]
    lib.oracle_multi_bind.restype = ctypes.c_int
    lib.oracle_segment_auto.argtypes = [ctypes.c_int, _i32p, ctypes.c_int, _i32p, _i32p, _i32p, _i32p]
    lib.oracle_segment_auto.restype = ctypes.c_int
    lib.oracle_segment_reduce.argtypes = [_f32p, _f32p, _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    lib.oracle_segment_reduce.restype = None
    lib.oracle_order_first_col.argtypes = [ctypes.c_int, ctypes.c_int, _i32p, _i32p, _i32p]
    lib.oracle_order_first_col.restype = None
    lib.oracle_order_rcm.argtypes = [ctypes.c_int, ctypes.c_int, _i32p, _i32p, _i32p]
    lib.oracle_order_rcm.restype = ctypes.c_int
    lib.oracle_order_jaccard.argtypes = [ctypes.c_int, ctypes.c_int, _i32p, _i32p, _i32p]
    lib.oracle_order_jaccard.restype = None
    lib.oracle_order_sparse_rows.argtypes = [ctypes.c_int, _i32p, _i32p]
    lib.oracle_order_sparse_rows.restype = ctypes.c_int
    lib.oracle_pack_count.argtypes = [_i32p, _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _i32p,
                                      ctypes.c_int, _i32p]
    lib.oracle_pack_count.restype = ctypes.c_int64
    lib.oracle_pack_fill.argtypes = [_i32p, _i32p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     _i32p, ctypes.c_int, _i32p, _i32p, _f32p]
    lib.oracle_pack_fill.restype = None
    _lib = lib
    return lib


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def swizzle(offset: int) -> int:
    """CuTe Swizzle<2,2,3> on a block offset (cute/swizzle.hpp:55-79)."""
    return int(_load().oracle_swizzle(int(offset)))


def convert(rowptr, colind, values, num_nodes: int, blk_h: int = 16, blk_w: int = 8) -> dict:
    """CSR -> SR-BCRS as preprocess_gpu_srcfp32_srbcrs
    (SRBCRSSpMM_kernel.cu:226-282 for 16x8, :284-340 for 32x32).

    Returns soff (= row_window_offset), sidx (= tcblocktile_id), val (the
    swizzled block values), block_partition, edge_to_row, edge_to_col, total.
    """
    lib = _load()
    rowptr = np.ascontiguousarray(rowptr, dtype=np.int32)
    colind = np.ascontiguousarray(colind, dtype=np.int32)
    values = np.ascontiguousarray(values, dtype=np.float32)
    mo = (num_nodes + blk_h - 1) // blk_h
    soff = np.zeros(mo + 1, dtype=np.int32)
    total = int(lib.oracle_convert_count(_p(rowptr, _i32p), _p(colind, _i32p), num_nodes, blk_h, blk_w,
                                         _p(soff, _i32p)))
    sidx = np.zeros(total * blk_w, dtype=np.int32)
    val = np.zeros(max(total * blk_h * blk_w, 1), dtype=np.float32)
    bp = np.zeros(mo, dtype=np.int32)
    nnz = colind.shape[0]
    e2r = np.zeros(max(nnz, 1), dtype=np.int32)
    e2c = np.zeros(max(nnz, 1), dtype=np.int32)
    lib.oracle_convert_fill(_p(rowptr, _i32p), _p(colind, _i32p), _p(values, _f32p), num_nodes, blk_h, blk_w,
                            _p(soff, _i32p), _p(sidx, _i32p), _p(val, _f32p), _p(bp, _i32p), _p(e2r, _i32p),
                            _p(e2c, _i32p))
    return dict(soff=soff, sidx=sidx, val=val[: total * blk_h * blk_w], block_partition=bp,
                edge_to_row=e2r[:nnz], edge_to_col=e2c[:nnz], total=total)


def csr_spmm_f64(rowptr, colind, values, B, num_rows: int, with_abs: bool = False):
    """fp64 textbook CSR SpMM: the oracle the error bound is stated against."""
    lib = _load()
    rowptr = np.ascontiguousarray(rowptr, dtype=np.int32)
    colind = np.ascontiguousarray(colind, dtype=np.int32)
    values = np.ascontiguousarray(values, dtype=np.float32)
    B = np.ascontiguousarray(B, dtype=np.float32)
    n = B.shape[1]
    C = np.empty((num_rows, n), dtype=np.float64)
    A = np.empty((num_rows, n), dtype=np.float64) if with_abs else None
    lib.oracle_csr_spmm_f64(_p(rowptr, _i32p), _p(colind, _i32p), _p(values, _f32p), _p(B, _f32p), num_rows, n,
                            _p(C, _f64p), _p(A, _f64p) if with_abs else None)
    return (C, A) if with_abs else C


def csr_spmm_f32(rowptr, colind, values, B, num_rows: int, nthreads: int = 0):
    """fp32 CPU CSR SpMM, the math of csr_spmm_value_kernel
    (SRBCRSSpMM_kernel.cu:66-87).  The timed CPU baseline."""
    lib = _load()
    rowptr = np.ascontiguousarray(rowptr, dtype=np.int32)
    colind = np.ascontiguousarray(colind, dtype=np.int32)
    values = np.ascontiguousarray(values, dtype=np.float32)
    B = np.ascontiguousarray(B, dtype=np.float32)
    C = np.empty((num_rows, B.shape[1]), dtype=np.float32)
    lib.oracle_csr_spmm_f32(_p(rowptr, _i32p), _p(colind, _i32p), _p(values, _f32p), _p(B, _f32p), num_rows,
                            B.shape[1], _p(C, _f32p), int(nthreads))
    return C


def max_threads() -> int:
    return int(_load().oracle_max_threads())


def strict_lb(soff, workload: int = 64):
    """strict_load_balance (main_strict_lb_16x8.cu:208-256)."""
    lib = _load()
    soff = np.ascontiguousarray(soff, dtype=np.int32)
    mo = soff.shape[0] - 1
    total = int(soff[-1])
    cap = mo + total // max(workload, 1) + 3
    fb = np.zeros(cap, dtype=np.int32)
    fw = np.zeros(cap, dtype=np.int32)
    go = np.zeros(cap, dtype=np.int32)
    ng = np.zeros(1, dtype=np.int32)
    nf = lib.oracle_strict_lb(mo, total, _p(soff, _i32p), workload, _p(fb, _i32p), _p(fw, _i32p), _p(go, _i32p),
                              _p(ng, _i32p))
    return dict(frag_begin=fb[: nf + 1].copy(), frag_window=fw[:nf].copy(), group_off=go[: int(ng[0]) + 1].copy())


def multi_bind(soff):
    """multi_binding_load_balance (main_multi_bind_16x8.cu:211-270)."""
    lib = _load()
    soff = np.ascontiguousarray(soff, dtype=np.int32)
    mo = soff.shape[0] - 1
    cap = int(soff[-1]) + mo + 2
    pw = np.zeros(cap, dtype=np.int32)
    po = np.zeros(cap + 1, dtype=np.int32)
    ws = np.zeros(max(mo, 1), dtype=np.int32)
    npart = lib.oracle_multi_bind(mo, _p(soff, _i32p), _p(pw, _i32p), _p(po, _i32p), _p(ws, _i32p))
    return dict(part_window=pw[:npart].copy(), part_off=po[: npart + 1].copy(), window_split=ws[:mo].copy())


def segment_auto(soff, requested: int = 0):
    """Automatic execution segmentation (custom_format_e2e.cu:640-699)."""
    lib = _load()
    soff = np.ascontiguousarray(soff, dtype=np.int32)
    mo = soff.shape[0] - 1
    cap = int(soff[-1]) + mo + 2
    se = np.zeros(cap, dtype=np.int32)
    wo = np.zeros(mo + 1, dtype=np.int32)
    c = np.zeros(1, dtype=np.int32)
    h = np.zeros(1, dtype=np.int32)
    nseg = lib.oracle_segment_auto(mo, _p(soff, _i32p), int(requested), _p(se, _i32p), _p(wo, _i32p),
                                   _p(c, _i32p), _p(h, _i32p))
    return dict(seg_end=se[:nseg].copy(), win_seg_off=wo, cap=int(c[0]), heavy=bool(h[0]))


def segment_reduce(partial, win_seg_off, tile_rows: int, n: int):
    """reduce_tcf_segments (custom_format_e2e.cu:832-853)."""
    lib = _load()
    partial = np.ascontiguousarray(partial, dtype=np.float32)
    wso = np.ascontiguousarray(win_seg_off, dtype=np.int32)
    mo = wso.shape[0] - 1
    out = np.zeros((mo * tile_rows, n), dtype=np.float32)
    lib.oracle_segment_reduce(_p(partial, _f32p), _p(out, _f32p), _p(wso, _i32p), mo, tile_rows, n)
    return out


def row_order(rowptr, colind, m: int, k: int, method: str) -> np.ndarray:
    """Row orders new -> original (custom_format_e2e.cu:157-349, 483-488):
    "row_rcm", "first_col_sort", "jaccard_greedy", "sparse_rows", "identity"."""
    lib = _load()
    rowptr = np.ascontiguousarray(rowptr, dtype=np.int32)
    colind = np.ascontiguousarray(colind, dtype=np.int32)
    out = np.zeros(max(m, 1), dtype=np.int32)
    if method == "identity":
        return np.arange(m, dtype=np.int32)
    if method == "first_col_sort":
        lib.oracle_order_first_col(m, k, _p(rowptr, _i32p), _p(colind, _i32p), _p(out, _i32p))
    elif method == "row_rcm":
        if lib.oracle_order_rcm(m, k, _p(rowptr, _i32p), _p(colind, _i32p), _p(out, _i32p)) != 0:
            raise ValueError("row_rcm currently requires a square matrix")
    elif method == "jaccard_greedy":
        lib.oracle_order_jaccard(m, k, _p(rowptr, _i32p), _p(colind, _i32p), _p(out, _i32p))
    elif method == "sparse_rows":
        n = lib.oracle_order_sparse_rows(m, _p(rowptr, _i32p), _p(out, _i32p))
        return out[:n].copy()
    else:
        raise ValueError(method)
    return out[:m].copy()


def pack(rowptr, colind, values, k: int, order, blk_h: int = 16, blk_w: int = 8, packing: int = 0) -> dict:
    """Generated-operator packing (custom_format_e2e.cu:496-640): rows in
    `order`, duplicates summed; packing 0 = column-condensed dense, 1 =
    active fixed blocks dense."""
    lib = _load()
    rowptr = np.ascontiguousarray(rowptr, dtype=np.int32)
    colind = np.ascontiguousarray(colind, dtype=np.int32)
    values = np.ascontiguousarray(values, dtype=np.float32)
    order = np.ascontiguousarray(order, dtype=np.int32)
    P = int(order.shape[0])
    W = (P + blk_h - 1) // blk_h
    soff = np.zeros(W + 1, dtype=np.int32)
    total = int(lib.oracle_pack_count(_p(rowptr, _i32p), _p(colind, _i32p), k, blk_h, blk_w, packing,
                                      _p(order, _i32p), P, _p(soff, _i32p)))
    if total < 0:
        raise ValueError("CSR column index out of range")
    sidx = np.zeros(max(total * blk_w, 1), dtype=np.int32)
    val = np.zeros(max(total * blk_h * blk_w, 1), dtype=np.float32)
    lib.oracle_pack_fill(_p(rowptr, _i32p), _p(colind, _i32p), _p(values, _f32p), k, blk_h, blk_w, packing,
                         _p(order, _i32p), P, _p(soff, _i32p), _p(sidx, _i32p), _p(val, _f32p))
    return dict(soff=soff, sidx=sidx[: total * blk_w], val=val[: total * blk_h * blk_w], total=total)


def read_mtx_loop(path):
    """Loop restatement of mmio_allinone (examples/src/mmio_highlevel.cu:
    255-402): per-row counters, exclusive scan, then entries placed in file
    order; symmetric/hermitian off-diagonals also placed mirrored right after.
    Small files only."""
    lines = [l for l in open(path).read().splitlines()]
    banner = lines[0].split()
    field, sym = banner[3].lower(), banner[4].lower()
    body = [l for l in lines[1:] if l.strip() and not l.lstrip().startswith("%")]
    m, n, nnz = (int(x) for x in body[0].split()[:3])
    ri, ci, vv = [], [], []
    for l in body[1:1 + nnz]:
        t = l.split()
        ri.append(int(t[0]) - 1)
        ci.append(int(t[1]) - 1)
        vv.append(1.0 if field == "pattern" else float(int(t[2])) if field == "integer" else float(t[2]))
    symmetric = sym in ("symmetric", "hermitian")
    count = [0] * (m + 1)
    for i in range(nnz):
        count[ri[i]] += 1
        if symmetric and ri[i] != ci[i]:
            count[ci[i]] += 1
    start = [0] * (m + 1)
    for r in range(m):
        start[r + 1] = start[r] + count[r]
    fill = [0] * m
    col = [0] * start[m]
    val = [0.0] * start[m]
    for i in range(nnz):
        for r, c in ((ri[i], ci[i]), (ci[i], ri[i])) if symmetric and ri[i] != ci[i] else ((ri[i], ci[i]),):
            col[start[r] + fill[r]] = c
            val[start[r] + fill[r]] = vv[i]
            fill[r] += 1
    return m, n, np.array(start, np.int32), np.array(col, np.int32), np.array(val, np.float32), symmetric


def error_metrics(C, C64, absAB):
    """Gate metrics.  North star: |C - C64| <= 1e-4 * (|A||B|) elementwise and
    a relative-L2 bound; the reference's own gate |d| <= 1e-3 + 1e-3*|ref|
    (custom_format_e2e.cu:1200-1240, main_16x8.cu:63-92) is reported too."""
    C = np.asarray(C, dtype=np.float64)
    d = np.abs(C - C64)
    with np.errstate(divide="ignore", invalid="ignore"):
        ratio = np.where(absAB > 0, d / absAB, np.where(d > 0, np.inf, 0.0))
    nrm = float(np.linalg.norm(C64))
    rel_l2 = float(np.linalg.norm(C - C64) / nrm) if nrm > 0 else float(np.linalg.norm(C - C64))
    ref_gate = bool(np.all(np.isfinite(C)) and np.all(d <= 1e-3 + 1e-3 * np.abs(C64)))
    return dict(max_abs=float(d.max()) if d.size else 0.0, max_ratio=float(ratio.max()) if ratio.size else 0.0,
                rel_l2=rel_l2, ref_gate=ref_gate, finite=bool(np.all(np.isfinite(C))))
