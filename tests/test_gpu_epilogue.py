"""GPU parity of the relu epilogue (srbcrs_run_opts.epilogue): a run with
relu=True equals relu applied to the same launch's plain output, bit for bit,
on every grid order and schedule (split schedules apply it in the segment
reduction, after the partial tiles are summed), with both block shapes, the
LDS B stage, packed plans with omitted and reordered rows, a tuned setting,
srbcrs_run_noalloc, and NaN passing through; an unknown epilogue is refused
before any launch.  The reference's SpMM has no epilogue: relu(A @ B) is the
GCN layer's torch.relu of the SpMM output (torch.relu keeps NaN), which is
what the plain output is compared through."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from tests.helpers import random_csr

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[case]", *a, flush=True)


def _plan(rowptr, colind, values, M, *blk, **kw):
    import torch
    from mask_amd.SRBCRSSpMM import Plan
    t = lambda a: torch.from_numpy(a).cuda()
    return Plan(t(rowptr), t(colind), t(values), M, *blk, **kw)


def _pair(plan, dB, M, **knobs):
    """(plain output, relu output) of one launch setting, each written over NaN."""
    import torch
    N = dB.shape[1]
    plain = torch.full((M, N), float("nan"), device="cuda")
    fused = torch.full((M, N), float("nan"), device="cuda")
    plan.run(dB, plain, **knobs)
    plan.run(dB, fused, relu=True, **knobs)
    torch.cuda.synchronize()
    return plain, fused


def _check(plain, fused, what):
    import torch
    want = torch.relu(plain)
    assert torch.equal(fused, want), what
    assert not bool(torch.isnan(fused).any()), what
    assert bool((fused >= 0).all()), what


@pytest.mark.parametrize("blk", [(16, 8), (32, 32)])
def test_relu_every_schedule_and_grid_order(gpu, blk):
    import torch
    M, K, N = 16 * 41 + 7, 2200, 256
    rowptr, colind, values = random_csr(M, K, 0.01, seed=3, empty_rows=0.1, heavy_rows=3, heavy_len=K // 2)
    dB = torch.from_numpy(np.random.default_rng(3).uniform(-1, 1, (K, N)).astype(np.float32)).cuda()
    plan = _plan(rowptr, colind, values, M, *blk)
    for pol, param in (("row", 0), ("split", 4), ("strict_lb", 16), ("multi_bind", 0)):
        plan.set_schedule(pol, param)
        orders = (0, 1, 2, 3) if pol != "row" or blk != (16, 8) else (0, 1, 2, 3, 4, 5)
        for go in orders:
            for stage in (("default", "lds") if go in (0, 1, 2, 3) and blk == (16, 8) else ("default",)):
                knobs = dict(grid_order=go, b_stage=stage)
                if go == 4:
                    knobs.update(wg_cols=64, windows_per_wave=8)
                _say("relu", blk, pol, param, knobs)
                _check(*_pair(plan, dB, M, **knobs), (blk, pol, knobs))


def test_relu_packed_plans(gpu):
    """Omitted rows (sparse-row packing) stay 0; reordered rows land at their
    output rows with the epilogue applied, on the row and split schedules."""
    import torch
    M, K, N = 700, 700, 128   # square: row_rcm orders a square matrix
    rowptr, colind, values = random_csr(M, K, 0.02, seed=9, empty_rows=0.3, heavy_rows=2, heavy_len=K // 2)
    dB = torch.from_numpy(np.random.default_rng(9).uniform(-1, 1, (K, N)).astype(np.float32)).cuda()
    for order in ("sparse_rows", "row_rcm"):
        plan = _plan(rowptr, colind, values, M, row_order=order, K=K)
        for pol, param in (("row", 0), ("split", 4)):
            plan.set_schedule(pol, param)
            _say("relu packed", order, pol)
            plain, fused = _pair(plan, dB, M)
            _check(plain, fused, (order, pol))
            empty = np.flatnonzero(np.diff(rowptr) == 0)
            assert bool((fused[torch.from_numpy(empty).cuda()] == 0).all())


def test_relu_with_tuned_setting_and_nan(gpu):
    """A tuned plan run with default knobs keeps the tuned setting and applies
    the epilogue; NaN in B reaches C as NaN through relu, as torch.relu
    keeps it."""
    import torch
    M, K, N = 1000, 1500, 192
    rowptr, colind, values = random_csr(M, K, 0.01, seed=12)
    B = np.random.default_rng(12).uniform(-1, 1, (K, N)).astype(np.float32)
    dB = torch.from_numpy(B).cuda()
    plan = _plan(rowptr, colind, values, M)
    plan.tune(dB, nonzero_sweep=True)
    _say("relu tuned")
    _check(*_pair(plan, dB, M), "tuned")
    B[int(colind[0])] = np.nan
    dB = torch.from_numpy(B).cuda()
    plain, fused = _pair(plan, dB, M)
    nan = torch.isnan(plain)
    assert bool(nan.any())
    assert torch.equal(torch.isnan(fused), nan)
    assert torch.equal(fused[~nan], torch.relu(plain)[~nan])


def test_relu_noalloc_and_refusal(gpu):
    import torch
    from mask_amd import _capi
    from mask_amd._capi import SrbcrsError
    L = _capi.lib()
    M, K, N = 600, 800, 128
    rowptr, colind, values = random_csr(M, K, 0.02, seed=21, heavy_rows=3, heavy_len=K // 2)
    dB = torch.from_numpy(np.random.default_rng(21).uniform(-1, 1, (K, N)).astype(np.float32)).cuda()
    plan = _plan(rowptr, colind, values, M)
    plan.set_schedule("split", 4)
    st = torch.cuda.current_stream().cuda_stream
    ref = plan.run(dB, relu=True)
    got = torch.full((M, N), float("nan"), device="cuda")
    opts = _capi.RunOpts(epilogue=_capi.EPILOGUE_RELU)
    _say("relu noalloc")
    _capi.check(L.srbcrs_run_noalloc(plan.handle, dB.data_ptr(), K, N, dB.stride(0), got.data_ptr(), got.stride(0),
                                     M, ctypes.byref(opts), st))
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    out = torch.full((M, N), 7.0, device="cuda")
    bad = _capi.RunOpts(epilogue=2)
    with pytest.raises(SrbcrsError, match="epilogue"):
        _capi.check(L.srbcrs_run_ex(plan.handle, dB.data_ptr(), K, N, dB.stride(0), out.data_ptr(), out.stride(0),
                                    M, ctypes.byref(bad), st))
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
