"""The MatrixMarket input path on the GPU: a committed symmetric, unsorted
.mtx file with a duplicate entry through datasets.from_mtx -> device
conversion -> SpMM, checked against the oracle (the reference's real-matrix
entry is mmio_allinone, examples/src/mmio_highlevel.cu:255-402)."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import oracle
from tests.helpers import assert_gate, dedupe_last, gate

pytestmark = pytest.mark.gpu

FIXTURE = Path(__file__).resolve().parent / "golden" / "sym_unsorted_dup.mtx"


@pytest.mark.parametrize("blk", [(16, 8), (32, 32)])
@pytest.mark.parametrize("N", [64, 512])
def test_mtx_file_through_the_kernel(gpu, blk, N):
    import torch
    from mask_amd import datasets
    from mask_amd.SRBCRSSpMM import Plan
    from tests.test_gpu_convert import _arrays, _same
    m = datasets.from_mtx(FIXTURE, N=N)
    print("[case] mtx", blk, N, m.M, m.nnz, flush=True)
    assert m.meta["symmetric"] and m.M == m.K == 90
    # the loader keeps file order inside rows: some row is unsorted, and the duplicate survives
    rows = [m.colind[m.rowptr[r]:m.rowptr[r + 1]] for r in range(m.M)]
    assert any((np.diff(c) < 0).any() for c in rows)
    assert any(len(set(c.tolist())) < len(c) for c in rows)
    assert m.rowptr[42] == m.rowptr[41]           # row 41 is empty
    t = lambda a: torch.from_numpy(a).cuda()
    plan = Plan(t(m.rowptr), t(m.colind), t(m.values), m.M, *blk)
    _same(_arrays(plan), oracle.convert(m.rowptr, m.colind, m.values, m.M, *blk))
    B = m.dense(N)
    C = plan.run(t(B)).cpu().numpy()
    # preprocess keeps the last of duplicate (row, col) entries
    rp, ci, vv = dedupe_last(m.rowptr, m.colind, m.values)
    assert_gate(gate(C, rp, ci, vv, B, m.M))
