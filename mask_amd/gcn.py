"""A small GCN whose neighbourhood aggregation is a pluggable CSR SpMM.

This is the caller the SR-BCRS path is measured under: the reference's GCN
script (end2end/gcn/eva_gcn_sparsene.py) trains a graph convolution network
whose aggregation ``A @ H`` goes through an external SpMM function with the
signature ``fn(rowptr, colind, values, dense, num_rows, feat_dim,
num_nodes_ori)``, e.g. ``mask_amd.external_backend_spmm.srbcrs_spmm``.

Design here:
- ``Graph`` holds A and its transpose as device CSR plus node features; the
  graphs come from the seeded synthetic matrices of ``mask_amd.datasets``.
- ``aggregate(graph, h, fn)`` is an autograd op: forward ``A @ h`` and, since
  d(A h)/dh applied to g is ``A^T g``, backward runs the same SpMM on the
  transposed CSR.
- ``GCN`` is a stack of layers ``h <- aggregate(h @ W_i)`` with ReLU and
  dropout between layers and log-softmax at the end.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Optional, Sequence, Tuple

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

Tensor = torch.Tensor
SpMMFn = Callable[..., Tensor]
CSR = Tuple[Tensor, Tensor, Tensor]


def csr_transpose(rowptr: np.ndarray, colind: np.ndarray, values: np.ndarray, n_cols: int):
    """CSR of A^T (rows sorted by column, stable in the original row order)."""
    n_rows = rowptr.shape[0] - 1
    rows = np.repeat(np.arange(n_rows, dtype=np.int64), np.diff(rowptr))
    order = np.lexsort((rows, colind))
    t_rowptr = np.zeros(n_cols + 1, np.int64)
    t_rowptr[1:] = np.cumsum(np.bincount(colind, minlength=n_cols))
    return t_rowptr.astype(np.int32), rows[order].astype(np.int32), values[order]


@dataclass
class Graph:
    name: str
    num_nodes: int
    num_edges: int
    a: CSR          # (rowptr, colind, values) of A on the device
    at: CSR         # the same for A^T
    x: Tensor       # node features, num_nodes x F


def graph_from_csr(m, feature_dim: int, device: torch.device, seed: int = 0) -> Graph:
    """A ``Graph`` for a ``datasets.CSRMatrix`` with N(0,1) features."""
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    x = torch.randn((m.M, feature_dim), generator=gen, dtype=torch.float32)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    a = (dev(m.rowptr), dev(m.colind), dev(m.values))
    at = tuple(dev(v) for v in csr_transpose(m.rowptr, m.colind, m.values, m.K))
    return Graph(m.name, m.M, m.nnz, a, at, x.to(device))


def torch_spmm(rowptr: Tensor, colind: Tensor, values: Tensor, dense: Tensor, num_rows: int, feat_dim: int,
               num_nodes_ori: int) -> Tensor:
    """The torch aggregation (torch.sparse.mm on a CSR tensor), same signature
    as the external SpMM functions, for comparison runs."""
    a = torch.sparse_csr_tensor(rowptr, colind, values, size=(num_rows, int(dense.shape[0])), device=dense.device)
    return torch.sparse.mm(a, dense)


def _spmm(fn: SpMMFn, csr: CSR, dense: Tensor) -> Tensor:
    rows = int(csr[0].numel()) - 1
    out = fn(csr[0], csr[1], csr[2], dense.contiguous(), rows, int(dense.shape[1]), rows)
    out = out[0] if isinstance(out, (list, tuple)) else out
    if not isinstance(out, Tensor):
        raise TypeError("an SpMM function must return a torch.Tensor")
    return out


class _Aggregate(torch.autograd.Function):
    """y = A h; dL/dh = A^T dL/dy (both through the same SpMM function)."""

    @staticmethod
    def forward(ctx, h: Tensor, graph: Graph, fn: SpMMFn) -> Tensor:
        ctx.graph, ctx.fn = graph, fn
        return _spmm(fn, graph.a, h)

    @staticmethod
    def backward(ctx, grad: Tensor):
        return _spmm(ctx.fn, ctx.graph.at, grad), None, None


def aggregate(graph: Graph, h: Tensor, fn: SpMMFn) -> Tensor:
    """A @ h with gradients, through ``fn``."""
    return _Aggregate.apply(h, graph, fn)


def glorot_weights(dims: Sequence[int], seed: int = 0, device: Optional[torch.device] = None):
    """Glorot-uniform weights W_i of shape dims[i] x dims[i+1]: U(-r, r) with
    r = sqrt(6 / (fan_in + fan_out))."""
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    out = []
    for fan_in, fan_out in zip(dims[:-1], dims[1:]):
        r = float(np.sqrt(6.0 / (fan_in + fan_out)))
        out.append(((torch.rand((fan_in, fan_out), generator=gen) * 2 - 1) * r).to(device))
    return out


class GCN(nn.Module):
    """Layers dims[0] -> dims[1] -> ... -> dims[-1]; each is
    ``aggregate(h @ W)``, ReLU + dropout between layers, log-softmax last."""

    def __init__(self, dims: Sequence[int], dropout: float = 0.0, spmm: Optional[SpMMFn] = None,
                 seed: Optional[int] = None) -> None:
        super().__init__()
        if len(dims) < 3:
            raise ValueError("a GCN needs at least two layers (three dims)")
        if spmm is None:
            from .external_backend_spmm import srbcrs_spmm
            spmm = srbcrs_spmm
        if seed is None:
            seed = int(torch.randint(0, 2 ** 31 - 1, (1,)).item())
        self.weights = nn.ParameterList(nn.Parameter(w) for w in glorot_weights(dims, seed))
        self.dropout = float(dropout)
        self.spmm = spmm

    def forward(self, graph: Graph, features: Optional[Tensor] = None) -> Tensor:
        h = graph.x if features is None else features
        last = len(self.weights) - 1
        for i, w in enumerate(self.weights):
            h = aggregate(graph, h @ w, self.spmm)
            if i < last:
                h = F.dropout(torch.relu(h), self.dropout, self.training)
        return torch.log_softmax(h, dim=1)


def gcn2_forward(graph: Graph, w1: Tensor, w2: Tensor, spmm: SpMMFn) -> Tensor:
    """relu(A (X W1)) then A (H W2): the GCN workload's two SpMMs at
    N = w1.shape[1] and w2.shape[1] plus the dense GEMMs (no autograd)."""
    h = torch.relu(_spmm(spmm, graph.a, graph.x @ w1))
    return _spmm(spmm, graph.a, h @ w2)
