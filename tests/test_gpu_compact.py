"""The compact block-value operand (the kernel's default A source) against the
dense reference-layout operand: identical bits on every kernel variant, and
the gate against the fp64 oracle."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import assert_gate, dedupe_last, gate, random_csr

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[case]", *a, flush=True)


def _both(plan, B, **kw):
    import torch
    outs = []
    for a in ("compact", "dense"):
        C = torch.full((plan.num_nodes, B.shape[1]), float("nan"), device=B.device)
        plan.run(B, C, a_operand=a, **kw)
        outs.append(C)
    torch.cuda.synchronize()
    return outs[0].cpu().numpy(), outs[1].cpu().numpy()


@pytest.mark.parametrize("blk", [(16, 8), (32, 32)])
def test_compact_equals_dense_all_variants(gpu, blk):
    import torch
    from mask_amd.SRBCRSSpMM import Plan
    rp, ci, vv = random_csr(517, 900, 0.02, 11, unsorted=True, duplicates=True, empty_rows=0.1, heavy_rows=3,
                            heavy_len=800)
    M = rp.shape[0] - 1
    t = lambda a: torch.from_numpy(a).cuda()
    plan = Plan(t(rp), t(ci), t(vv), M, blk[0], blk[1])
    rng = np.random.default_rng(3)
    for N in (16, 64, 128, 256):
        Bh = rng.uniform(-1, 1, (900, N)).astype(np.float32)
        B = t(Bh)
        for pol in (("row", 0), ("split", 0), ("strict_lb", 0), ("multi_bind", 4)):
            plan.set_schedule(*pol)
            for depth in (2, 4, 8):
                _say("compact-vs-dense", blk, N, pol, depth)
                c, d = _both(plan, B, depth=depth)
                assert c.tobytes() == d.tobytes()
            assert_gate(gate(c, *dedupe_last(rp, ci, vv), Bh, M))


def test_compact_signed_and_explicit_zeros(gpu):
    """Stored -0.0 keeps its sign bit, stored +0.0 is rebuilt as +0.0, and
    both operands give the same bits (including -0.0 results)."""
    import torch
    from mask_amd.SRBCRSSpMM import Plan
    M, K, N = 64, 64, 64
    rng = np.random.default_rng(9)
    rows, cols, vals = [], [], []
    for r in range(M):
        cs = np.sort(rng.choice(K, size=5, replace=False))
        for j, c in enumerate(cs):
            rows.append(r)
            cols.append(c)
            vals.append([-0.0, 0.0, 1.5, -2.0, 0.25][j])
    rp = np.zeros(M + 1, np.int32)
    np.add.at(rp, np.asarray(rows) + 1, 1)
    rp = np.cumsum(rp).astype(np.int32)
    ci = np.asarray(cols, np.int32)
    vv = np.asarray(vals, np.float32)
    t = lambda a: torch.from_numpy(a).cuda()
    plan = Plan(t(rp), t(ci), t(vv), M)
    Bh = -np.abs(rng.uniform(0.5, 1, (K, N))).astype(np.float32)
    Bh[:, ::3] = 0.0   # products -0.0 * 0.0 and 0.0 * 0.0 in the same sums
    _say("signed zeros")
    c, d = _both(plan, t(Bh))
    assert c.tobytes() == d.tobytes()
    assert_gate(gate(c, rp, ci, vv, Bh, M))


@pytest.mark.parametrize("packing,row_order", [("active_fixed_blocks_dense", "identity"),
                                               ("column_condensed_dense", "row_rcm"),
                                               ("column_condensed_dense", "jaccard_greedy"),
                                               ("column_condensed_dense", "sparse_rows")])
def test_compact_equals_dense_packings(gpu, packing, row_order):
    import torch
    from mask_amd.SRBCRSSpMM import Plan
    rp, ci, vv = random_csr(400, 400, 0.03, 21, duplicates=True, empty_rows=0.2)   # square: row_rcm needs it
    M = rp.shape[0] - 1
    t = lambda a: torch.from_numpy(a).cuda()
    plan = Plan(t(rp), t(ci), t(vv), M, packing=packing, dup="sum", row_order=row_order, K=400)
    Bh = np.random.default_rng(2).uniform(-1, 1, (400, 128)).astype(np.float32)
    _say("packing", packing, row_order)
    c, d = _both(plan, t(Bh))
    assert c.tobytes() == d.tobytes()


def test_compact_empty_matrix(gpu):
    """An empty matrix has no blocks: both operands run and give zeros."""
    import torch
    from mask_amd.SRBCRSSpMM import Plan
    t = lambda a: torch.from_numpy(a).cuda()
    plan = Plan(t(np.zeros(17, np.int32)), t(np.zeros(0, np.int32)), t(np.zeros(0, np.float32)), 16)
    _say("empty compact")
    c, d = _both(plan, t(np.ones((4, 32), np.float32)))
    assert not c.any() and not d.any()


def test_tune_keeps_bits_and_sticks(gpu):
    """srbcrs_plan_tune picks a setting; default-knob runs use it and give
    the same bits as the untuned default; a schedule change drops it."""
    import torch
    from mask_amd.SRBCRSSpMM import Plan
    rp, ci, vv = random_csr(700, 700, 0.01, 31, heavy_rows=2, heavy_len=600)
    t = lambda a: torch.from_numpy(a).cuda()
    plan = Plan(t(rp), t(ci), t(vv), 700)
    for pol in (("row", 0), ("split", 0)):
        plan.set_schedule(*pol)
        for N in (64, 128):
            B = t(np.random.default_rng(N).uniform(-1, 1, (700, N)).astype(np.float32))
            _say("tune", pol, N)
            ref = plan.run(B).clone()
            C = torch.full_like(ref, float("nan"))
            choice = plan.tune(B, C, reps=1)
            assert choice["depth"] in (2, 4, 8) and choice["wg_cols"] in (64, 128, 256)
            assert choice["a_operand"] in ("compact", "dense")
            assert torch.equal(C, ref)          # tune leaves the product in C
            again = plan.run(B)
            assert torch.equal(again, ref)
            assert N in plan.tuned_widths
    plan.set_schedule("row", 0)
    assert not plan.tuned_widths


def test_tune_rejects_bad_reps(gpu):
    import torch
    from mask_amd._capi import SrbcrsError
    from mask_amd.SRBCRSSpMM import Plan
    rp, ci, vv = random_csr(64, 64, 0.05, 1)
    t = lambda a: torch.from_numpy(a).cuda()
    plan = Plan(t(rp), t(ci), t(vv), 64)
    B = t(np.ones((64, 32), np.float32))
    with pytest.raises(SrbcrsError, match="reps"):
        plan.tune(B, reps=0)
