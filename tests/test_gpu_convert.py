"""Device-side conversion (is_device = 1) against the oracle, bit for bit,
and against the host conversion of the same device CSR (is_device = 2)."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle
from tests.helpers import random_csr

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[case]", *a, flush=True)


def _arrays(plan):
    import torch
    from mask_amd import _capi
    n = plan.row_windows + 1
    soff = torch.empty(n, dtype=torch.int32, device="cuda")
    sidx = torch.empty(max(plan.total_blocks * plan.blk_w, 1), dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    _capi.check(_capi.lib().srbcrs_plan_export_index(plan.handle, soff.data_ptr(), n, sidx.data_ptr(),
                                                     sidx.numel(), st))
    bp = torch.zeros(max(plan.row_windows, 1), dtype=torch.int32, device="cuda")
    e2c = torch.zeros(max(plan.nnz, 1), dtype=torch.int32, device="cuda")
    e2r = torch.zeros(max(plan.nnz, 1), dtype=torch.int32, device="cuda")
    _capi.check(_capi.lib().srbcrs_plan_write_edges(plan.handle, bp.data_ptr(), plan.row_windows, e2c.data_ptr(),
                                                    plan.nnz, e2r.data_ptr(), plan.nnz, st))
    val = plan.block_values()
    torch.cuda.synchronize()
    return dict(soff=soff.cpu().numpy(), sidx=sidx.cpu().numpy()[: plan.total_blocks * plan.blk_w],
                val=val.cpu().numpy(), block_partition=bp.cpu().numpy()[: plan.row_windows],
                edge_to_col=e2c.cpu().numpy()[: plan.nnz], edge_to_row=e2r.cpu().numpy()[: plan.nnz],
                total=plan.total_blocks, max_col=plan.max_col)


def _same(a, b):
    assert a["total"] == b["total"]
    for k in ("soff", "sidx", "block_partition", "edge_to_row", "edge_to_col"):
        assert np.array_equal(a[k], b[k]), k
    assert a["val"].tobytes() == b["val"].tobytes()


def _cases():
    yield "tiny", random_csr(1, 1, 1.0, 0)
    yield "m17", random_csr(17, 40, 0.2, 1)
    yield "unsorted-dup", random_csr(203, 700, 0.03, 2, unsorted=True, duplicates=True, empty_rows=0.2)
    yield "skewed", random_csr(500, 3000, 0.01, 3, heavy_rows=5, heavy_len=2500, empty_rows=0.3)
    yield "empty", (np.zeros(33, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32))


@pytest.mark.parametrize("blk", [(16, 8), (32, 32)])
def test_device_conversion_matches_oracle(gpu, blk):
    import torch
    from mask_amd.SRBCRSSpMM import Plan
    for name, (rp, ci, vv) in _cases():
        M = rp.shape[0] - 1
        _say("convert", name, blk, M, ci.size)
        t = lambda a: torch.from_numpy(a).cuda()
        dev = _arrays(Plan(t(rp), t(ci), t(vv), M, blk[0], blk[1], convert_on="device"))
        host = _arrays(Plan(t(rp), t(ci), t(vv), M, blk[0], blk[1], convert_on="host"))
        o = oracle.convert(rp, ci, vv, M, blk[0], blk[1])
        _same(dev, o)
        _same(host, o)
        assert dev["max_col"] == (int(ci.max()) if ci.size else -1)


@pytest.mark.parametrize("name", ["uniform-65536", "banded-524288", "rmat-2^20", "gcn-232965"])
def test_device_conversion_workloads(gpu, name):
    import torch
    from mask_amd import datasets
    from mask_amd.SRBCRSSpMM import Plan
    m = datasets.make_config(name, scale_down=8)
    _say("convert workload", name, m.M, m.nnz)
    t = lambda a: torch.from_numpy(a).cuda()
    _same(_arrays(Plan(t(m.rowptr), t(m.colind), t(m.values), m.M)), oracle.convert(m.rowptr, m.colind, m.values, m.M))


def test_device_conversion_rejects_malformed(gpu):
    import torch
    from mask_amd._capi import SrbcrsError
    from mask_amd.SRBCRSSpMM import Plan
    t = lambda a: torch.from_numpy(np.asarray(a)).cuda()
    with pytest.raises(SrbcrsError, match="non-decreasing"):
        Plan(t(np.array([0, 3, 1], np.int32)), t(np.array([0, 1, 2], np.int32)), t(np.ones(3, np.float32)), 2)
    with pytest.raises(SrbcrsError, match="non-decreasing"):
        Plan(t(np.array([0, 9], np.int32)), t(np.array([0, 1], np.int32)), t(np.ones(2, np.float32)), 1)
    with pytest.raises(SrbcrsError, match="negative"):
        Plan(t(np.array([0, 2], np.int32)), t(np.array([1, -4], np.int32)), t(np.ones(2, np.float32)), 1)


@pytest.mark.parametrize("name", ["convert_16x8_hand.json", "convert_32x32_hand.json"])
def test_device_conversion_matches_golden(gpu, name):
    """The device converter against the hand-derived fixtures."""
    import torch
    from mask_amd.SRBCRSSpMM import Plan
    from tests.test_golden import arrays, load
    g = load(name)
    rp, ci, vv = arrays(g)
    t = lambda a: torch.from_numpy(a).cuda()
    _say("golden", name)
    got = _arrays(Plan(t(rp), t(ci), t(vv), g["num_nodes"], *g["blk"]))
    assert got["total"] == g["total"]
    for k in ("soff", "sidx", "block_partition", "edge_to_row", "edge_to_col"):
        assert got[k].tolist() == g[k], k
    assert got["val"].tobytes() == np.asarray(g["val"], np.float32).tobytes()


@pytest.mark.parametrize("a_operand", ["compact", "dense"])
@pytest.mark.parametrize("blk", [(16, 8), (32, 32)])
def test_spmm_exact_golden(gpu, blk, a_operand):
    """Power-of-two A times small-integer B: every sum is exact in fp32, so
    C must equal the fixture bit for bit."""
    import torch
    from mask_amd.SRBCRSSpMM import Plan
    from tests.test_golden import arrays, load
    g = load("spmm_exact.json")
    rp, ci, vv = arrays(g)
    t = lambda a: torch.from_numpy(a).cuda()
    _say("exact spmm", blk, a_operand)
    plan = Plan(t(rp), t(ci), t(vv), g["num_nodes"], *blk)
    C = plan.run(t(np.asarray(g["B"], np.float32)), a_operand=a_operand).cpu().numpy()
    assert np.array_equal(C, np.asarray(g["C"], np.float32))
