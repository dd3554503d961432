"""GCN with a replaceable SpMM, the caller of the SR-BCRS path.

Mirrors end2end/gcn/eva_gcn_sparsene.py: ``SpMMBackend`` (:189-265),
``ReplaceableSpMMFunction`` (:267-289: forward A @ X, backward A^T @ dY
through the same SpMM), ``ReplaceableGCNConv`` (:292-314: X @ W then the
SpMM) and ``ReplaceableGCN`` (:317-343).  ``GraphData`` here is built from
the seeded synthetic graphs of ``mask_amd.datasets`` (no dataset files), and
``gcn2_forward`` is the two-layer forward relu(A (X W1)) -> A (H W2).
"""
from __future__ import annotations

import importlib
import weakref
from dataclasses import dataclass
from typing import Callable, Dict, Optional, Tuple, cast

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

Tensor = torch.Tensor


@dataclass
class GraphData:
    name: str
    num_nodes: int
    num_edges: int
    rowptr: Tensor
    colind: Tensor
    values: Tensor
    rowptr_t: Tensor
    colind_t: Tensor
    values_t: Tensor
    x: Tensor


def csr_transpose(rowptr: np.ndarray, colind: np.ndarray, values: np.ndarray, n_cols: int):
    """CSR of A^T (rows sorted by column, stable in the original row order)."""
    n_rows = rowptr.shape[0] - 1
    rows = np.repeat(np.arange(n_rows, dtype=np.int64), np.diff(rowptr))
    order = np.lexsort((rows, colind))
    t_rowptr = np.zeros(n_cols + 1, np.int64)
    t_rowptr[1:] = np.cumsum(np.bincount(colind, minlength=n_cols))
    return t_rowptr.astype(np.int32), rows[order].astype(np.int32), values[order]


def graph_from_csr(m, feature_dim: int, device: torch.device, seed: int = 0) -> GraphData:
    """GraphData for a ``datasets.CSRMatrix`` with N(0,1) features."""
    rp_t, ci_t, v_t = csr_transpose(m.rowptr, m.colind, m.values, m.K)
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    x = torch.randn((m.M, feature_dim), generator=gen, dtype=torch.float32)
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    return GraphData(m.name, m.M, m.nnz, to(m.rowptr), to(m.colind), to(m.values), to(rp_t), to(ci_t), to(v_t),
                     x.to(device))


class SpMMBackend:
    """Replaceable SpMM: ``torch`` (torch.sparse.mm) or an external function
    with the signature fn(rowptr, colind, values, dense, num_rows, feat_dim,
    num_nodes_ori), e.g. ``mask_amd.external_backend_spmm.srbcrs_spmm``."""

    def __init__(self, name: str, external_fn: Optional[Callable[..., Tensor]] = None) -> None:
        self.name = name
        self.external_fn = external_fn
        self._i32_cache: Dict[int, Tuple[weakref.ReferenceType, Tensor]] = {}

    def _to_i32_cached(self, t: Tensor) -> Tensor:
        if t.dtype == torch.int32 and t.is_contiguous():
            return t
        ent = self._i32_cache.get(id(t))
        if ent is not None and ent[0]() is t:
            return ent[1]
        c = t.to(torch.int32).contiguous()
        self._i32_cache[id(t)] = (weakref.ref(t), c)
        return c

    @staticmethod
    def build(backend: str, module_name: str = "", function_name: str = "") -> "SpMMBackend":
        if backend == "torch":
            return SpMMBackend("torch")
        if backend != "external":
            raise ValueError(f"Unsupported backend: {backend}")
        if not module_name or not function_name:
            raise ValueError("External backend requires --external-module and --external-function")
        fn = getattr(importlib.import_module(module_name), function_name)
        return SpMMBackend(f"external:{module_name}.{function_name}", fn)

    def spmm(self, rowptr: Tensor, colind: Tensor, values: Tensor, dense: Tensor) -> Tensor:
        n_rows = int(rowptr.numel() - 1)
        if self.external_fn is None:
            csr = torch.sparse_csr_tensor(rowptr, colind, values, size=(n_rows, int(dense.shape[0])),
                                          device=dense.device)
            return torch.sparse.mm(csr, dense)
        out = self.external_fn(self._to_i32_cached(rowptr), self._to_i32_cached(colind), values, dense, n_rows,
                               int(dense.shape[1]), n_rows)
        if isinstance(out, (tuple, list)):
            out = out[0]
        if not isinstance(out, torch.Tensor):
            raise TypeError("External SpMM backend must return a torch.Tensor")
        return out


class ReplaceableSpMMFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, rowptr, colind, values, rowptr_t, colind_t, values_t, dense, backend: SpMMBackend):
        ctx.backend = backend
        ctx.save_for_backward(rowptr_t, colind_t, values_t)
        return backend.spmm(rowptr, colind, values, dense.contiguous())

    @staticmethod
    def backward(ctx, *grad_outputs):
        rowptr_t, colind_t, values_t = ctx.saved_tensors
        grad_dense = ctx.backend.spmm(rowptr_t, colind_t, values_t, grad_outputs[0].contiguous())
        return None, None, None, None, None, None, grad_dense, None


class ReplaceableGCNConv(nn.Module):
    def __init__(self, in_dim: int, out_dim: int) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.empty((in_dim, out_dim), dtype=torch.float32))
        self.reset_parameters()

    def reset_parameters(self) -> None:
        nn.init.xavier_uniform_(self.weight)

    def forward(self, x: Tensor, data: GraphData, backend: SpMMBackend) -> Tensor:
        x = x @ self.weight
        out = ReplaceableSpMMFunction.apply(data.rowptr, data.colind, data.values, data.rowptr_t, data.colind_t,
                                            data.values_t, x, backend)
        return cast(Tensor, out)


class ReplaceableGCN(nn.Module):
    def __init__(self, in_dim: int, hidden_dim: int, out_dim: int, num_layers: int, dropout: float) -> None:
        super().__init__()
        if num_layers < 2:
            raise ValueError("num_layers must be >= 2")
        self.conv_in = ReplaceableGCNConv(in_dim, hidden_dim)
        self.hidden = nn.ModuleList([ReplaceableGCNConv(hidden_dim, hidden_dim) for _ in range(num_layers - 2)])
        self.conv_out = ReplaceableGCNConv(hidden_dim, out_dim)
        self.dropout = float(dropout)

    def forward(self, data: GraphData, backend: SpMMBackend) -> Tensor:
        x = F.relu(self.conv_in(data.x, data, backend))
        x = F.dropout(x, p=self.dropout, training=self.training)
        for conv in self.hidden:
            x = F.relu(conv(x, data, backend))
            x = F.dropout(x, p=self.dropout, training=self.training)
        x = self.conv_out(x, data, backend)
        return F.log_softmax(x, dim=1)


def glorot_weights(dims, seed: int = 0, device: Optional[torch.device] = None):
    """Glorot-uniform weights W_i of shape dims[i] x dims[i+1]."""
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    ws = []
    for a, b in zip(dims[:-1], dims[1:]):
        bound = float(np.sqrt(6.0 / (a + b)))
        ws.append(((torch.rand((a, b), generator=gen) * 2 - 1) * bound).to(device))
    return ws


def gcn2_forward(data: GraphData, w1: Tensor, w2: Tensor, backend: SpMMBackend) -> Tensor:
    """relu(A (X W1)) then A (H W2): the two SpMMs at N = w1.shape[1] and
    w2.shape[1] plus the dense GEMMs."""
    h = F.relu(backend.spmm(data.rowptr, data.colind, data.values, (data.x @ w1).contiguous()))
    return backend.spmm(data.rowptr, data.colind, data.values, (h @ w2).contiguous())
