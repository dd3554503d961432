"""Row sharding of the SR-BCRS SpMM, the layout a multi-GPU run would use.

The row windows are independent, so cutting them into contiguous ranges of
near-equal cost (``srbcrs_shard_windows``) gives each shard its own C rows
and no reduction.  This build has one GPU: ``RowShardedSpMM`` creates one
plan per shard on that GPU and runs them in turn, which is exactly one
shard's work at its real shape (the same rows, the whole B).  On G GPUs each
shard's plan would live on its own device, with B replicated (or
all-gathered) there.  No reference counterpart (the reference is
single-GPU).
"""
from __future__ import annotations

from typing import List, Tuple

import numpy as np
import torch
from torch import Tensor

from . import _capi
from .SRBCRSSpMM import Plan


def plan_soff(plan: Plan) -> np.ndarray:
    """row_window_offset of a plan, on the host."""
    n = plan.row_windows + 1
    t = torch.empty(n, dtype=torch.int32, device=plan.device)
    with torch.cuda.device(plan.device):
        _capi.check(_capi.lib().srbcrs_plan_export_index(plan.handle, t.data_ptr(), n, None, 0,
                                                         torch.cuda.current_stream(plan.device).cuda_stream))
    return t.cpu().numpy()


def row_shards(soff: np.ndarray, num_nodes: int, n_shards: int, blk_h: int = 16) -> List[Tuple[int, int]]:
    """[(r0, r1)] row ranges of the shards (window ranges scaled by blk_h,
    the last clipped to num_nodes); empty shards give r0 == r1."""
    b = _capi.shard_windows(soff, n_shards)
    return [(min(int(b[i]) * blk_h, num_nodes), min(int(b[i + 1]) * blk_h, num_nodes)) for i in range(n_shards)]


def slice_csr(rowptr: Tensor, colind: Tensor, values: Tensor, r0: int, r1: int) -> Tuple[Tensor, Tensor, Tensor]:
    """CSR of rows [r0, r1) (device tensors; rowptr rebased to 0)."""
    e0, e1 = int(rowptr[r0]), int(rowptr[r1])
    return (rowptr[r0:r1 + 1] - e0).contiguous(), colind[e0:e1].contiguous(), values[e0:e1].contiguous()


class RowShardedSpMM:
    """One plan per row shard; ``run`` writes every shard's rows of C."""

    def __init__(self, rowptr: Tensor, colind: Tensor, values: Tensor, num_nodes: int, n_shards: int,
                 blk_h: int = 16, blk_w: int = 8) -> None:
        full = Plan(rowptr, colind, values, num_nodes, blk_h, blk_w)
        self.ranges = row_shards(plan_soff(full), num_nodes, n_shards, blk_h)
        full.close()
        self.num_nodes = num_nodes
        self.plans: List[Plan] = []
        for r0, r1 in self.ranges:
            if r1 > r0:
                self.plans.append(Plan(*slice_csr(rowptr, colind, values, r0, r1), r1 - r0, blk_h, blk_w))
            else:
                self.plans.append(None)

    def set_schedule(self, policy: str = "row", param: int = 0) -> None:
        for p in self.plans:
            if p is not None:
                p.set_schedule(policy, param)

    def run_shard(self, i: int, dense: Tensor, out: Tensor) -> None:
        """Shard i's rows: out[r0:r1] = A[r0:r1] @ dense."""
        r0, r1 = self.ranges[i]
        if self.plans[i] is not None:
            self.plans[i].run(dense, out[r0:r1])

    def run(self, dense: Tensor, out: Tensor = None) -> Tensor:
        if out is None:
            out = torch.empty((self.num_nodes, dense.shape[1]), dtype=torch.float32, device=dense.device)
        for i in range(len(self.plans)):
            self.run_shard(i, dense, out)
        return out
