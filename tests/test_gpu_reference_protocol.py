"""The reference harness's own correctness protocol on the GPU.

custom_format_e2e.cu:1336-1342 replaces a matrix's values by p % 5 + 1 (p =
the entry's position in the CSR) and fills B with ((i % 29) - 14) / 14 (i =
the row-major element index), then checks every element with
|got - ref| <= 1e-3 + 1e-3 |ref| (verify, :1200-1240).  Those inputs run here
through the library on the reference's shapes, checked with that gate and the
north-star gate against the fp64 oracle.

The same protocol with B scaled by 14 (integers -14..14) makes every product
and every partial sum an integer below 2^24, so fp32 arithmetic is exact in
any summation order: the result must equal the integer product bit for bit
for every schedule (split segments included), launch knob, A source and block
shape.  A dropped, repeated or misplaced term changes an integer, so this
pins the indexing without a tolerance.
"""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import assert_gate, dedupe_last, exact_product, gate, protocol_dense, protocol_values

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[case]", *a, flush=True)


def _matrix(name):
    from mask_amd import datasets
    if name == "mtx":
        from pathlib import Path
        return datasets.from_mtx(Path(__file__).resolve().parent / "golden" / "sym_unsorted_dup.mtx", N=64)
    base, scale = {"uniform-4096": ("uniform-4096", 1), "uniform-65536/8": ("uniform-65536", 8),
                   "banded/64": ("banded-524288", 64), "rmat/64": ("rmat-2^20", 64),
                   "gcn/32": ("gcn-232965", 32)}[name]
    return datasets.make_config(base, scale_down=scale)


def _plan(m, blk=(16, 8)):
    import torch
    from mask_amd.SRBCRSSpMM import Plan
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    vals = protocol_values(m.nnz)
    return Plan(t(m.rowptr), t(m.colind), t(vals), m.M, *blk), vals


@pytest.mark.parametrize("name,N", [("mtx", 64), ("uniform-4096", 64), ("uniform-4096", 512),
                                    ("uniform-65536/8", 512), ("rmat/64", 512)])
def test_reference_protocol_gate(gpu, name, N):
    """The reference's inputs and its verify gate (plus the north-star gate)."""
    import torch
    m = _matrix(name)
    _say("protocol", name, m.M, m.nnz, N)
    plan, vals = _plan(m)
    B = protocol_dense(m.K, N)
    C = plan.run(torch.from_numpy(B).cuda()).cpu().numpy()
    rp, ci, vv = dedupe_last(m.rowptr, m.colind, vals)
    assert_gate(gate(C, rp, ci, vv, B, m.M))


SCHEDULES = [("row", 0), ("split", 0), ("split", 8), ("strict_lb", 0), ("multi_bind", 0), ("auto", 0)]


@pytest.mark.parametrize("name", ["mtx", "uniform-4096", "banded/64", "rmat/64", "gcn/32"])
@pytest.mark.parametrize("blk", [(16, 8), (32, 32)])
def test_integer_protocol_is_exact(gpu, name, blk):
    """14 x the protocol's B: every schedule gives the exact integer product."""
    import torch
    m = _matrix(name)
    N = 64
    plan, vals = _plan(m, blk)
    B_int = (14 * protocol_dense(m.K, N)).round().astype(np.float32)
    assert np.abs(B_int).max() == 14
    want = exact_product(m.rowptr, m.colind, vals, B_int, m.M)
    assert np.abs(want).max() < 2 ** 24
    dB = torch.from_numpy(B_int).cuda()
    for sched in SCHEDULES:
        _say("integer", name, blk, sched, m.M, m.nnz)
        plan.set_schedule(*sched)
        C = plan.run(dB).cpu().numpy()
        assert np.array_equal(C[: m.M], want.astype(np.float32)), (name, blk, sched)


@pytest.mark.parametrize("knobs", [dict(depth=4, wg_cols=64, grid_order=3, b_stage="lds"),
                                   dict(depth=2, wg_cols=256, grid_order=1, windows_per_wave=8),
                                   dict(depth=8, wg_cols=128, grid_order=2, a_operand="dense"),
                                   dict(depth=2, wg_cols=128, grid_order=3, a_operand="compact")])
def test_integer_protocol_knobs_exact(gpu, knobs):
    """Launch knobs at N = 512 on a skewed graph, split schedule: exact."""
    import torch
    m = _matrix("rmat/64")
    N = 512
    plan, vals = _plan(m)
    plan.set_schedule("split", 0)
    B_int = (14 * protocol_dense(m.K, N)).round().astype(np.float32)
    want = exact_product(m.rowptr, m.colind, vals, B_int, m.M).astype(np.float32)
    _say("integer knobs", knobs, m.M, m.nnz)
    C = plan.run(torch.from_numpy(B_int).cuda(), **knobs).cpu().numpy()
    assert np.array_equal(C[: m.M], want)
