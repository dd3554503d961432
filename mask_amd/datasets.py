"""Seeded synthetic SpMM workloads (numpy, host side).

The five workloads of the benchmark definition, built deterministically from
fixed seeds.  All return a CSR matrix (int32 rowptr / colind, float32 values,
columns sorted inside each row, no duplicates) plus the dense operand's
shape and distribution; ``dense()`` materialises the dense operand.

Interpretations that the workload text leaves open are recorded in
``CSRMatrix.meta``:
  * banded: block (i, j) of the 32768 x 65536 grid of 16x8 blocks lies on
    "diagonal" d when j = 2*i + d, d in [-4, 4] (the grid is twice as wide
    as tall); each such block is kept with probability 0.7;
  * R-MAT: the listed (a, b, c, d) = (0.57, 0.19, 0.19, 0.19) sums to 1.14,
    so the quadrant probabilities are the listed values over their sum.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, Optional

import numpy as np

CONFIG_SEEDS = {
    "uniform-4096": 1001,
    "uniform-65536": 1002,
    "banded-524288": 1003,
    "rmat-2^20": 1004,
    "gcn-232965": 1005,
}


@dataclass
class CSRMatrix:
    name: str
    rowptr: np.ndarray
    colind: np.ndarray
    values: np.ndarray
    M: int
    K: int
    N: int                   # dense operand width of the workload
    dense_dist: str          # "uniform" (U[-1,1]) or "normal" (N(0,1))
    seed: int
    meta: Dict = field(default_factory=dict)

    @property
    def nnz(self) -> int:
        return int(self.colind.shape[0])

    def dense(self, N: Optional[int] = None, seed: Optional[int] = None) -> np.ndarray:
        return make_dense(self.K, N or self.N, self.dense_dist, (self.seed + 7) if seed is None else seed)


def make_dense(K: int, N: int, dist: str, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    if dist == "uniform":
        return rng.uniform(-1.0, 1.0, size=(K, N)).astype(np.float32)
    if dist == "normal":
        return rng.standard_normal(size=(K, N), dtype=np.float32)
    raise ValueError(dist)


def _csr_from_coo(rows: np.ndarray, cols: np.ndarray, vals: np.ndarray, M: int):
    """Sort (row, col), build rowptr.  Input must hold no duplicates."""
    order = np.lexsort((cols, rows))
    rows, cols, vals = rows[order], cols[order], vals[order]
    rowptr = np.zeros(M + 1, dtype=np.int64)
    np.add.at(rowptr, rows + 1, 1)
    rowptr = np.cumsum(rowptr).astype(np.int32)
    return rowptr, cols.astype(np.int32), vals.astype(np.float32)


def uniform_bernoulli(M: int = 4096, K: int = 4096, p: float = 0.005, N: int = 64,
                      seed: int = CONFIG_SEEDS["uniform-4096"], name: str = "uniform-4096") -> CSRMatrix:
    """Each entry nonzero with probability p, values U[-1, 1] (row-major order)."""
    rng = np.random.default_rng(seed)
    rowptr = np.zeros(M + 1, dtype=np.int64)
    cols_l = []
    chunk = max(1, (1 << 24) // K)
    for r0 in range(0, M, chunk):
        r1 = min(M, r0 + chunk)
        mask = rng.random((r1 - r0, K)) < p
        rr, cc = np.nonzero(mask)
        rowptr[r0 + 1:r1 + 1] = np.bincount(rr, minlength=r1 - r0)
        cols_l.append(cc.astype(np.int32))
    rowptr = np.cumsum(rowptr).astype(np.int32)
    colind = np.concatenate(cols_l) if cols_l else np.zeros(0, np.int32)
    values = rng.uniform(-1.0, 1.0, size=colind.shape[0]).astype(np.float32)
    return CSRMatrix(name, rowptr, colind, values, M, K, N, "uniform", seed, dict(p=p))


def uniform_fixed_row(M: int = 65536, K: int = 65536, per_row: int = 16, N: int = 512,
                      seed: int = CONFIG_SEEDS["uniform-65536"], name: str = "uniform-65536") -> CSRMatrix:
    """Exactly `per_row` distinct uniformly random columns per row, values U[-1, 1]."""
    rng = np.random.default_rng(seed)
    cols = rng.integers(0, K, size=(M, per_row), dtype=np.int64)
    cols.sort(axis=1)
    bad = np.nonzero((np.diff(cols, axis=1) == 0).any(axis=1))[0]
    while bad.size:
        redo = rng.integers(0, K, size=(bad.size, per_row), dtype=np.int64)
        redo.sort(axis=1)
        cols[bad] = redo
        bad = bad[(np.diff(redo, axis=1) == 0).any(axis=1)]
    rowptr = (np.arange(M + 1, dtype=np.int64) * per_row).astype(np.int32)
    values = rng.uniform(-1.0, 1.0, size=M * per_row).astype(np.float32)
    return CSRMatrix(name, rowptr, cols.reshape(-1).astype(np.int32), values, M, K, N, "uniform", seed,
                     dict(per_row=per_row))


def banded_blocks(block_rows: int = 32768, block_cols: int = 65536, offsets=range(-4, 5), keep: float = 0.7,
                  N: int = 512, seed: int = CONFIG_SEEDS["banded-524288"], name: str = "banded-524288",
                  bh: int = 16, bw: int = 8) -> CSRMatrix:
    """Dense bh x bw blocks at block (i, 2i + d), d in offsets, kept w.p. `keep`,
    every entry N(0, 1) and stored explicitly."""
    rng = np.random.default_rng(seed)
    offs = np.asarray(list(offsets), dtype=np.int64)
    i = np.arange(block_rows, dtype=np.int64)[:, None]
    j = 2 * i + offs[None, :]
    present = (j >= 0) & (j < block_cols) & (rng.random((block_rows, offs.size)) < keep)
    bi, bd = np.nonzero(present)                     # block order: i, then d ascending
    bj = 2 * bi + offs[bd]
    nb = bi.size
    vals = rng.standard_normal(size=(nb, bh, bw), dtype=np.float32)
    # entry (b, r, c) -> row bh*i_b + r, col bw*j_b + c; a stable sort by row
    # keeps block (hence column) order inside each row
    r = np.arange(bh, dtype=np.int64)
    c = np.arange(bw, dtype=np.int64)
    rows = (bh * bi[:, None, None] + r[None, :, None] + 0 * c[None, None, :]).reshape(-1)
    cols = (bw * bj[:, None, None] + 0 * r[None, :, None] + c[None, None, :]).reshape(-1)
    order = np.argsort(rows, kind="stable")
    M = block_rows * bh
    rowptr = np.zeros(M + 1, dtype=np.int64)
    rowptr[1:] = np.cumsum(np.bincount(rows, minlength=M))
    return CSRMatrix(name, rowptr.astype(np.int32), cols[order].astype(np.int32), vals.reshape(-1)[order], M,
                     block_cols * bw, N, "normal", seed,
                     dict(blocks=int(nb), block_rule="j = 2*i + d", offsets=[int(o) for o in offs], keep=keep))


def rmat_edges(scale: int, n_edges: int, probs, rng: np.random.Generator, n_nodes: Optional[int] = None):
    """R-MAT edge list: per level pick a quadrant with probabilities (a,b,c,d)
    (normalised to sum 1); ids >= n_nodes are redrawn."""
    p = np.asarray(probs, dtype=np.float64)
    p = p / p.sum()
    ca, cab, cabc = p[0], p[0] + p[1], p[0] + p[1] + p[2]
    n_nodes = n_nodes or (1 << scale)
    src_all, dst_all = [], []
    need = n_edges
    while need > 0:
        m = need
        src = np.zeros(m, dtype=np.int64)
        dst = np.zeros(m, dtype=np.int64)
        for lvl in range(scale):
            u = rng.random(m)
            sbit = (u >= cab).astype(np.int64)                       # c or d
            dbit = (((u >= ca) & (u < cab)) | (u >= cabc)).astype(np.int64)  # b or d
            src |= sbit << lvl
            dst |= dbit << lvl
        ok = (src < n_nodes) & (dst < n_nodes)
        src_all.append(src[ok])
        dst_all.append(dst[ok])
        need -= int(ok.sum())
    return np.concatenate(src_all), np.concatenate(dst_all)


def normalized_graph(src: np.ndarray, dst: np.ndarray, n: int):
    """Symmetrise, dedupe, add self loops, values D^-1/2 (A+I) D^-1/2."""
    s = np.concatenate([src, dst, np.arange(n, dtype=np.int64)])
    d = np.concatenate([dst, src, np.arange(n, dtype=np.int64)])
    key = np.unique(s * n + d)
    rows = key // n
    cols = key % n
    deg = np.bincount(rows, minlength=n).astype(np.float64)
    inv = 1.0 / np.sqrt(deg)
    vals = (inv[rows] * inv[cols]).astype(np.float32)
    rowptr = np.zeros(n + 1, dtype=np.int64)
    rowptr[1:] = np.cumsum(np.bincount(rows, minlength=n))
    return rowptr.astype(np.int32), cols.astype(np.int32), vals


RMAT_LISTED = (0.57, 0.19, 0.19, 0.19)


def rmat_graph(scale: int = 20, n_edges: int = 16 * (1 << 20), N: int = 512,
               seed: int = CONFIG_SEEDS["rmat-2^20"], name: str = "rmat-2^20",
               n_nodes: Optional[int] = None, dense_dist: str = "uniform") -> CSRMatrix:
    rng = np.random.default_rng(seed)
    n = n_nodes or (1 << scale)
    src, dst = rmat_edges(scale, n_edges, RMAT_LISTED, rng, n)
    rowptr, colind, values = normalized_graph(src, dst, n)
    p = np.asarray(RMAT_LISTED) / sum(RMAT_LISTED)
    return CSRMatrix(name, rowptr, colind, values, n, n, N, dense_dist, seed,
                     dict(listed=list(RMAT_LISTED), normalised=[float(x) for x in p], generated_edges=n_edges))


def gcn_graph(n: int = 232965, avg_degree: int = 50, N: int = 256, seed: int = CONFIG_SEEDS["gcn-232965"],
              name: str = "gcn-232965") -> CSRMatrix:
    """R-MAT graph on n nodes (scale ceil(log2 n), ids >= n redrawn) with about
    n*avg_degree/2 generated edges before symmetrisation."""
    scale = max(1, int(np.ceil(np.log2(n))))
    return rmat_graph(scale=scale, n_edges=n * avg_degree // 2, N=N, seed=seed, name=name, n_nodes=n,
                      dense_dist="normal")


def from_mtx(path, N: int = 512, seed: int = 7) -> CSRMatrix:
    """A MatrixMarket file as a workload (the reference's dataset path,
    examples/src/mmio_highlevel.cu:255-402); dense operand U[-1, 1]."""
    from .mtx import read_mtx
    m, n, rowptr, colind, values, sym = read_mtx(path)
    return CSRMatrix(str(path), rowptr, colind, values, m, n, N, "uniform", seed, dict(symmetric=sym))


def make_config(name: str, scale_down: int = 1) -> CSRMatrix:
    """The named workload.  scale_down > 1 shrinks M/K (and edge counts) by
    that factor for quick tests while keeping the structure."""
    f = max(1, int(scale_down))
    if name == "uniform-4096":
        return uniform_bernoulli(M=4096 // f, K=4096 // f)
    if name == "uniform-65536":
        return uniform_fixed_row(M=65536 // f, K=65536 // f)
    if name == "banded-524288":
        return banded_blocks(block_rows=32768 // f, block_cols=65536 // f)
    if name == "rmat-2^20":
        s = 20 - int(np.log2(f))
        return rmat_graph(scale=s, n_edges=16 * (1 << s))
    if name == "gcn-232965":
        return gcn_graph(n=232965 // f)
    raise KeyError(name)
