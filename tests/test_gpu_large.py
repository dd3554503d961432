"""Maximum sizes: B and C with more than 2^31 elements each (2.2M x 1024
fp32, 9 GB apiece), nonzeros that reference the last rows of B, and output
rows at the end of C.  Any 32-bit offset arithmetic in the kernels, the
zero-row stores or the conversion would fault or land in the wrong place."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle
from tests.helpers import TOL_ELEM

pytestmark = pytest.mark.gpu


def test_int64_offsets(gpu):
    import torch
    from mask_amd.SRBCRSSpMM import Plan
    M = K = 2_200_000
    N = 1024
    assert M * N > 2**31 and K * N > 2**31
    rng = np.random.default_rng(77)
    rows = np.concatenate([np.arange(20), np.arange(M - 40, M), rng.integers(20, M - 40, 30)])
    rows = np.unique(rows)
    counts = np.zeros(M, np.int64)
    counts[rows] = 6
    rowptr = np.zeros(M + 1, np.int64)
    rowptr[1:] = np.cumsum(counts)
    colind = np.concatenate([np.sort(np.concatenate([rng.choice(np.arange(K - 5000, K), 4, replace=False),
                                                     rng.choice(np.arange(0, 10), 2, replace=False)]))
                             for _ in rows]).astype(np.int32)
    values = rng.uniform(-1, 1, colind.size).astype(np.float32)
    used = np.unique(colind)
    Bsub = rng.uniform(-1, 1, (used.size, N)).astype(np.float32)
    print("[case] int64 offsets", M, K, N, int(rowptr[-1]), flush=True)
    dev = torch.device("cuda", 0)
    B = torch.empty((K, N), dtype=torch.float32, device=dev)
    B[torch.from_numpy(used.astype(np.int64)).to(dev)] = torch.from_numpy(Bsub).to(dev)
    plan = Plan(torch.from_numpy(rowptr.astype(np.int32)).to(dev), torch.from_numpy(colind).to(dev),
                torch.from_numpy(values).to(dev), M)
    # the oracle on the rows that hold entries, with B reduced to the columns they use
    remap = np.searchsorted(used, colind).astype(np.int32)
    sub_rp = np.concatenate([[0], np.cumsum(counts[rows])]).astype(np.int32)
    C64, absAB = oracle.csr_spmm_f64(sub_rp, remap, values, Bsub, rows.size, with_abs=True)
    zero_rows = torch.from_numpy(np.setdiff1d(np.concatenate([rng.integers(0, M, 64), [M - 41, 20]]), rows)).to(dev)
    for a_op in ("compact", "dense"):
        C = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
        plan.run(B, C, a_operand=a_op)
        torch.cuda.synchronize()
        got = C[torch.from_numpy(rows).to(dev)].cpu().numpy().astype(np.float64)
        assert np.isfinite(got).all()
        assert (np.abs(got - C64) <= TOL_ELEM * absAB + 1e-30).all(), a_op
        assert (C[zero_rows] == 0).all().item(), a_op
        del C
        torch.cuda.empty_cache()
    # the CSR fallback kernel on the same operands
    from mask_amd.SRBCRSSpMM import csr_spmm
    C = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    csr_spmm(torch.from_numpy(rowptr.astype(np.int32)).to(dev), torch.from_numpy(colind).to(dev),
             torch.from_numpy(values).to(dev), B, M, max_col=int(colind.max()), out=C)
    torch.cuda.synchronize()
    got = C[torch.from_numpy(rows).to(dev)].cpu().numpy().astype(np.float64)
    assert (np.abs(got - C64) <= TOL_ELEM * absAB + 1e-30).all(), "csr"
    assert (C[zero_rows] == 0).all().item(), "csr"
