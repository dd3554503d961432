"""MatrixMarket coordinate files -> CSR, as the reference's loader builds it.

Follows ``mmio_allinone`` (examples/src/mmio_highlevel.cu:255-402):
1-based indices become 0-based; ``pattern`` entries get value 1, ``integer``
entries their integer value, ``complex`` entries their real part; for
``symmetric`` / ``hermitian`` files every off-diagonal entry (i, j) is also
stored as (j, i).  Rows are filled in file order (for symmetric files the
mirrored entry directly follows its source entry in the mirrored row), so
columns are not sorted inside a row -- the conversion handles that.
Values are returned as float32 (the fp32 testbed's value type).
"""
from __future__ import annotations

import gzip
import io
from pathlib import Path
from typing import Tuple, Union

import numpy as np


def _open(path: Union[str, Path]):
    path = Path(path)
    if path.suffix == ".gz":
        return io.TextIOWrapper(gzip.open(path, "rb"))
    return open(path, "r")


def read_mtx(path: Union[str, Path]) -> Tuple[int, int, np.ndarray, np.ndarray, np.ndarray, bool]:
    """Returns (m, n, rowptr int32, colind int32, values float32, symmetric)."""
    with _open(path) as f:
        banner = f.readline().split()
        if len(banner) < 5 or banner[0].lower() != "%%matrixmarket" or banner[1].lower() != "matrix":
            raise ValueError("Could not process Matrix Market banner.")
        fmt, field, sym = banner[2].lower(), banner[3].lower(), banner[4].lower()
        if fmt != "coordinate":
            raise ValueError(f"only coordinate MatrixMarket files are supported, got {fmt}")
        if field not in ("real", "double", "integer", "pattern", "complex"):
            raise ValueError(f"unsupported MatrixMarket field {field}")
        line = f.readline()
        while line and line.lstrip().startswith("%"):
            line = f.readline()
        if not line:
            raise ValueError("missing size line")
        m, n, nnz = (int(x) for x in line.split()[:3])
        body = f.read()
    ncols = {"pattern": 2, "complex": 4}.get(field, 3)
    data = np.array(body.split(), dtype=np.float64) if nnz else np.zeros(0)
    if data.size < nnz * ncols:
        raise ValueError(f"expected {nnz} entries, file is truncated")
    data = data[: nnz * ncols].reshape(nnz, ncols)
    rows = data[:, 0].astype(np.int64) - 1
    cols = data[:, 1].astype(np.int64) - 1
    if nnz and (rows.min() < 0 or rows.max() >= m or cols.min() < 0 or cols.max() >= n):
        raise ValueError("MatrixMarket entry index out of range")
    if field == "pattern":
        vals = np.ones(nnz, np.float64)
    elif field == "integer":
        vals = np.trunc(data[:, 2])
    else:
        vals = data[:, 2]
    symmetric = sym in ("symmetric", "hermitian")   # skew-symmetric is read as general, as mmio_allinone does
    if symmetric:
        off = rows != cols
        # sequence: entry i -> 2i, its mirror -> 2i + 1
        r2 = np.concatenate([rows, cols[off]])
        c2 = np.concatenate([cols, rows[off]])
        v2 = np.concatenate([vals, vals[off]])
        seq = np.concatenate([2 * np.arange(nnz), 2 * np.nonzero(off)[0] + 1])
        rows, cols, vals = r2, c2, v2
    else:
        seq = np.arange(nnz)
    order = np.lexsort((seq, rows))          # by row, then file order
    counts = np.bincount(rows, minlength=m)
    rowptr = np.zeros(m + 1, np.int64)
    rowptr[1:] = np.cumsum(counts)
    return (m, n, rowptr.astype(np.int32), cols[order].astype(np.int32), vals[order].astype(np.float32),
            symmetric)


def write_mtx(path: Union[str, Path], m: int, n: int, rows, cols, vals=None, symmetric: bool = False) -> None:
    """Write a coordinate MatrixMarket file (1-based), real or pattern."""
    field = "pattern" if vals is None else "real"
    kind = "symmetric" if symmetric else "general"
    with open(path, "w") as f:
        f.write(f"%%MatrixMarket matrix coordinate {field} {kind}\n% written by mask_amd.mtx\n")
        f.write(f"{m} {n} {len(rows)}\n")
        for i in range(len(rows)):
            if vals is None:
                f.write(f"{int(rows[i]) + 1} {int(cols[i]) + 1}\n")
            else:
                f.write(f"{int(rows[i]) + 1} {int(cols[i]) + 1} {float(vals[i])!r}\n")
