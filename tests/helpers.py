"""Shared test helpers: small seeded CSR builders and the error gate."""
from __future__ import annotations

import numpy as np

from oracle import oracle

# Elementwise gate of the north star: |C - C64| <= TOL_ELEM * (|A||B|)_ij,
# and a relative-L2 bound for fp32 accumulation.
TOL_ELEM = 1e-4
TOL_REL_L2 = 1e-6


def random_csr(M: int, K: int, density: float, seed: int, *, unsorted: bool = False, duplicates: bool = False,
               empty_rows: float = 0.0, heavy_rows: int = 0, heavy_len: int = 0):
    """Random CSR (int32/float32).  Options: unsorted columns inside rows,
    duplicated (row, col) entries, a fraction of empty rows, a few long rows."""
    rng = np.random.default_rng(seed)
    rows = []
    for r in range(M):
        if rng.random() < empty_rows:
            rows.append(np.zeros(0, np.int64))
            continue
        n = rng.binomial(K, density)
        if r < heavy_rows:
            n = min(K, heavy_len)
        cols = rng.choice(K, size=n, replace=False) if n else np.zeros(0, np.int64)
        if duplicates and n:
            extra = rng.choice(cols, size=max(1, n // 4))
            cols = np.concatenate([cols, extra])
        if not unsorted:
            cols = np.sort(cols)
        else:
            rng.shuffle(cols)
        rows.append(cols)
    rowptr = np.zeros(M + 1, np.int64)
    rowptr[1:] = np.cumsum([len(c) for c in rows])
    colind = np.concatenate(rows).astype(np.int32) if rowptr[-1] else np.zeros(0, np.int32)
    values = rng.uniform(-1, 1, size=colind.shape[0]).astype(np.float32)
    return rowptr.astype(np.int32), colind, values


def dedupe_last(rowptr, colind, values):
    """Collapse duplicate (row, col) pairs keeping the last value: the
    conversion's last-write-wins rule restated as a CSR."""
    M = rowptr.shape[0] - 1
    rp = [0]
    cs, vs = [], []
    for r in range(M):
        d = {}
        for e in range(rowptr[r], rowptr[r + 1]):
            d[int(colind[e])] = values[e]
        for c in sorted(d):
            cs.append(c)
            vs.append(d[c])
        rp.append(len(cs))
    return np.asarray(rp, np.int32), np.asarray(cs, np.int32), np.asarray(vs, np.float32)


def gate(C, rowptr, colind, values, B, M):
    """Compare C against the fp64 oracle; returns the metrics dict."""
    C64, absAB = oracle.csr_spmm_f64(rowptr, colind, values, B, M, with_abs=True)
    return oracle.error_metrics(np.asarray(C)[:M], C64, absAB)


def assert_gate(m, rel_l2=TOL_REL_L2):
    assert m["finite"], m
    assert m["max_ratio"] <= TOL_ELEM, m
    assert m["rel_l2"] <= rel_l2, m
    assert m["ref_gate"], m


# The reference harness's value protocol (custom_format_e2e.cu:1336-1342):
# values p % 5 + 1 by CSR position, B element i = ((i % 29) - 14) / 14.
def protocol_values(nnz: int) -> np.ndarray:
    return (np.arange(nnz, dtype=np.int64) % 5 + 1).astype(np.float32)


def protocol_dense(K: int, N: int) -> np.ndarray:
    i = np.arange(K * N, dtype=np.int64)
    return ((i % 29 - 14) / 14.0).astype(np.float32).reshape(K, N)


def exact_product(rowptr, colind, values, B_int, M) -> np.ndarray:
    """A @ B in int64 (duplicates collapsed to the last value first)."""
    rp, ci, vv = dedupe_last(rowptr, colind, values)
    out = np.zeros((M, B_int.shape[1]), np.int64)
    rows = np.repeat(np.arange(M), np.diff(rp))
    np.add.at(out, rows, vv.astype(np.int64)[:, None] * B_int.astype(np.int64)[ci])
    return out
