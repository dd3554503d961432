"""GPU tests of the drop-in module surface (mask_amd.SRBCRSSpMM mirrors the
reference's SRBCRSSpMM extension) and of the 32x32 base variant."""
from __future__ import annotations

import itertools

import numpy as np
import pytest

from oracle import oracle
from tests.helpers import assert_gate, gate, random_csr

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[case]", *a, flush=True)


def _dev_csr(rowptr, colind, values):
    import torch
    return (torch.from_numpy(colind).cuda(), torch.from_numpy(rowptr).cuda(), torch.from_numpy(values).cuda())


@pytest.mark.parametrize("blk", [(16, 8), (32, 32)])
def test_preprocess_tuple_matches_oracle(gpu, blk):
    import torch
    from mask_amd import SRBCRSSpMM as S
    bh, bw = blk
    M, K = 203, 700
    rowptr, colind, values = random_csr(M, K, 0.03, seed=5, unsorted=True, empty_rows=0.2)
    _say("preprocess", blk, M, K)
    ci, rp, vv = _dev_csr(rowptr, colind, values)
    mo = (M + bh - 1) // bh
    bp = torch.zeros(mo, dtype=torch.int32, device="cuda")
    e2c = torch.zeros(colind.size, dtype=torch.int32, device="cuda")
    e2r = torch.zeros(colind.size, dtype=torch.int32, device="cuda")
    fn = S.preprocess_gpu_16x8 if blk == (16, 8) else S.preprocess_gpu
    rwo, rowid, tile_id, toff, a2x, total = fn(ci, rp, vv, M, bh, bw, bp, e2c, e2r)
    torch.cuda.synchronize()
    o = oracle.convert(rowptr, colind, values, M, bh, bw)
    assert total == o["total"]
    assert np.array_equal(rwo.cpu().numpy(), o["soff"])
    assert np.array_equal(tile_id.cpu().numpy(), o["sidx"])
    assert np.array_equal(bp.cpu().numpy(), o["block_partition"])
    assert np.array_equal(e2c.cpu().numpy(), o["edge_to_col"])
    assert np.array_equal(e2r.cpu().numpy(), o["edge_to_row"])
    assert rowid.numel() == total and int(rowid.abs().sum()) == 0
    assert toff.numel() == 1 and a2x.numel() == 1
    # the plan's device values are the oracle's swizzled blocks, bit for bit
    val = S.plan_for(rwo).block_values()
    assert val.cpu().numpy().tobytes() == o["val"].tobytes()


@pytest.mark.parametrize("blk", [(16, 8), (32, 32)])
@pytest.mark.parametrize("N", [16, 64, 96, 512])
def test_run_matches_oracle(gpu, blk, N):
    import torch
    from mask_amd import SRBCRSSpMM as S
    bh, bw = blk
    M, K = 150, 400
    rowptr, colind, values = random_csr(M, K, 0.05, seed=N, empty_rows=0.1)
    B = np.random.default_rng(N).uniform(-1, 1, (K, N)).astype(np.float32)
    _say("run", blk, M, K, N)
    ci, rp, vv = _dev_csr(rowptr, colind, values)
    z = torch.zeros(1, dtype=torch.int32, device="cuda")
    pre = S.preprocess_gpu_16x8 if blk == (16, 8) else S.preprocess_gpu
    run = S.run_SRBCRS_16x8 if blk == (16, 8) else S.run_SRBCRS
    runb = S.run_SRBCRS_16x8_balance if blk == (16, 8) else S.run_SRBCRS_balance
    rwo, _, tid, toff, a2x, _ = pre(ci, rp, vv, M, bh, bw, z, z, z)
    dB = torch.from_numpy(B).cuda()
    (out,) = run(dB, rwo, tid, toff, a2x, M, colind.size, "")
    torch.cuda.synchronize()
    assert out.shape == (M, N)
    assert_gate(gate(out.cpu().numpy(), rowptr, colind, values, B, M))
    (outb,) = runb(dB, rwo, tid, toff, a2x, M, "")
    assert torch.equal(out, outb)
    for plan_str in ("split:2", "strict_lb:3", "multi_bind"):
        (o2,) = run(dB, rwo, tid, toff, a2x, M, colind.size, plan_str)
        assert_gate(gate(o2.cpu().numpy(), rowptr, colind, values, B, M))


def test_run_errors(gpu, monkeypatch):
    import torch
    from mask_amd import SRBCRSSpMM as S
    M, K = 40, 50
    rowptr, colind, values = random_csr(M, K, 0.1, seed=1)
    ci, rp, vv = _dev_csr(rowptr, colind, values)
    z = torch.zeros(1, dtype=torch.int32, device="cuda")
    rwo, _, tid, toff, a2x, _ = S.preprocess_gpu_16x8(ci, rp, vv, M, 16, 8, z, z, z)
    dB = torch.ones((K, 64), device="cuda")
    with pytest.raises(RuntimeError, match="cache miss"):
        S.run_SRBCRS_16x8(dB, rwo.clone(), tid, toff, a2x, M, 0, "")
    with pytest.raises(RuntimeError, match="num_nodes mismatch"):
        S.run_SRBCRS_16x8(dB, rwo, tid, toff, a2x, M + 1, 0, "")
    with pytest.raises(RuntimeError, match="variant mismatch"):
        S.run_SRBCRS(dB, rwo, tid, toff, a2x, M, 0, "")
    with pytest.raises(RuntimeError, match="divisible by 16/32/64"):
        S.run_SRBCRS_16x8(torch.ones((K, 40), device="cuda"), rwo, tid, toff, a2x, M, 0, "")
    with pytest.raises(RuntimeError, match="blk_h mismatch"):
        S.preprocess_gpu_16x8(ci, rp, vv, M, 32, 8, z, z, z)
    with pytest.raises(RuntimeError, match="must be float32"):
        S.run_SRBCRS_16x8(dB.double(), rwo, tid, toff, a2x, M, 0, "")
    monkeypatch.setenv("SRBCRS_TILE_B", "7")
    with pytest.raises(RuntimeError, match="Invalid SRBCRS_TILE_B"):
        S.run_SRBCRS_16x8(dB, rwo, tid, toff, a2x, M, 0, "")
    monkeypatch.delenv("SRBCRS_TILE_B")
    (out,) = S.run_SRBCRS_16x8(torch.ones((K, 0), device="cuda"), rwo, tid, toff, a2x, M, 0, "")
    assert out.shape == (M, 0)
    # a matrix without blocks is refused like the reference (CSR fallback disabled)
    e_rp = torch.zeros(M + 1, dtype=torch.int32, device="cuda")
    e_ci = torch.zeros(0, dtype=torch.int32, device="cuda")
    e_v = torch.zeros(0, dtype=torch.float32, device="cuda")
    r2, _, t2, o2, x2, total = S.preprocess_gpu_16x8(e_ci, e_rp, e_v, M, 16, 8, z, z, z)
    assert total == 0
    with pytest.raises(RuntimeError, match="empty preprocessed blocks"):
        S.run_SRBCRS_16x8(dB, r2, t2, o2, x2, M, 0, "")
    # B with too few rows for the matrix's columns is refused before launch
    from mask_amd._capi import SrbcrsError
    with pytest.raises(SrbcrsError, match="references column"):
        S.plan_for(rwo).run(torch.ones((int(colind.max()), 64), device="cuda"))


@pytest.mark.parametrize("packing", ["column_condensed_dense", "active_fixed_blocks_dense"])
@pytest.mark.parametrize("order", ["row_rcm", "first_col_sort", "jaccard_greedy", "sparse_rows"])
@pytest.mark.parametrize("blk", [(16, 8), (32, 32)])
def test_packed_plans_match_oracle(gpu, packing, order, blk):
    """Reordered / sparse-row / fixed-block plans with summed duplicates:
    the inverse row map is applied in the store, omitted rows are zero."""
    import torch
    from mask_amd.SRBCRSSpMM import Plan
    M = K = 300
    N = 128
    rowptr, colind, values = random_csr(M, K, 0.03, seed=len(order) + blk[0], duplicates=True, empty_rows=0.3,
                                        heavy_rows=2, heavy_len=250)
    B = np.random.default_rng(3).uniform(-1, 1, (K, N)).astype(np.float32)
    _say("packed", packing, order, blk)
    plan = Plan(*(torch.from_numpy(a).cuda() for a in (rowptr, colind, values)), M, blk[0], blk[1],
                packing=packing, dup="sum", row_order=order, K=K)
    dB = torch.from_numpy(B).cuda()
    for pol in (("row", 0), ("split", 2), ("strict_lb", 7)):
        plan.set_schedule(*pol)
        out = torch.full((M, N), float("nan"), device="cuda")
        plan.run(dB, out)
        torch.cuda.synchronize()
        assert_gate(gate(out.cpu().numpy(), rowptr, colind, values, B, M))   # duplicates summed
    # the row map applied at task boundaries inside a wave's stream (several
    # windows per wave), on both B rings: the same bits as one window per wave
    plan.set_schedule("row", 0)
    ref = plan.run(dB).cpu().numpy()
    for wpw, stage, depth in ((3, "registers", 4), (3, "lds", 4), (16, "lds", 2), (16, "registers", 8)):
        got = plan.run(dB, windows_per_wave=wpw, b_stage=stage, depth=depth).cpu().numpy()
        assert np.array_equal(got, ref), (wpw, stage, depth)


def test_generated_operator_on_packed_plan(gpu):
    import torch
    from mask_amd.build import GENERATED
    from mask_amd.emitter import GeneratedOperator
    from mask_amd.SRBCRSSpMM import Plan
    M = K = 400
    rowptr, colind, values = random_csr(M, K, 0.02, seed=17, empty_rows=0.4)
    B = np.random.default_rng(17).uniform(-1, 1, (K, 256)).astype(np.float32)
    _say("generated packed", M)
    plan = Plan(*(torch.from_numpy(a).cuda() for a in (rowptr, colind, values)), M, packing="column_condensed_dense",
                dup="sum", row_order="sparse_rows", K=K)
    op = GeneratedOperator(GENERATED / "sr_bcrs_16x8.so")
    dB = torch.from_numpy(B).cuda()
    for pol, param in (("row", 0), ("split", 2)):
        plan.set_schedule(pol, param)
        ref = plan.run(dB)
        out = op.run(plan, dB, schedule=pol, schedule_param=param)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), pol


def test_32x32_knobs_and_schedules(gpu):
    import torch
    from mask_amd.SRBCRSSpMM import Plan
    M, K, N = 300, 2000, 128
    rowptr, colind, values = random_csr(M, K, 0.02, seed=8, empty_rows=0.3, heavy_rows=4, heavy_len=900)
    B = np.random.default_rng(8).uniform(-1, 1, (K, N)).astype(np.float32)
    _say("32x32 knobs", M, K, N)
    plan = Plan(*(torch.from_numpy(a).cuda() for a in (rowptr, colind, values)), M, 32, 32)
    dB = torch.from_numpy(B).cuda()
    ref = plan.run(dB).cpu().numpy()
    assert_gate(gate(ref, rowptr, colind, values, B, M))
    for depth, tile_b, wgc, go in itertools.product([2, 4, 8], [0, 16, 32], [0, 64], [1, 2]):
        out = plan.run(dB, depth=depth, tile_b=tile_b, wg_cols=wgc, grid_order=go)
        assert np.array_equal(out.cpu().numpy(), ref), (depth, tile_b, wgc, go)
    for pol in (("split", 0), ("split", 2), ("strict_lb", 5), ("multi_bind", 0)):
        plan.set_schedule(*pol)
        assert_gate(gate(plan.run(dB).cpu().numpy(), rowptr, colind, values, B, M))


def test_base_variant_runs_on_a_16x8_plan(gpu, monkeypatch):
    """run_SRBCRS (32x32 preprocess) executes on a 16x8 plan of the same CSR
    by default -- within the gate, and bit-equal to the 16x8 plan's own run --
    and on the 32x32 blocks themselves with SPARSENE_SRBCRS_BASE_NATIVE=1
    (bit-equal to the 32x32 plan's run).  The preprocess outputs stay the
    32x32 arrays either way."""
    import torch
    from mask_amd import SRBCRSSpMM as S
    M, K, N = 300, 500, 128
    rowptr, colind, values = random_csr(M, K, 0.03, seed=77, heavy_rows=2, heavy_len=400)
    B = np.random.default_rng(77).uniform(-1, 1, (K, N)).astype(np.float32)
    ci, rp, vv = _dev_csr(rowptr, colind, values)
    z = torch.zeros(1, dtype=torch.int32, device="cuda")
    rwo, _, tid, toff, a2x, total = S.preprocess_gpu(ci, rp, vv, M, 32, 32, z, z, z)
    assert total == oracle.convert(rowptr, colind, values, M, 32, 32)["total"]
    dB = torch.from_numpy(B).cuda()
    _say("base variant execution", M, N)
    monkeypatch.delenv("SPARSENE_SRBCRS_BASE_NATIVE", raising=False)
    (fast,) = S.run_SRBCRS(dB, rwo, tid, toff, a2x, M, colind.size, "row")
    entry = S._cache[int(rwo.data_ptr())]
    assert entry.exec_plan is not None and (entry.exec_plan.blk_h, entry.exec_plan.blk_w) == (16, 8)
    p16 = S.Plan(rp, ci, vv, M, 16, 8)
    assert torch.equal(fast, p16.run(dB))
    assert_gate(gate(fast.cpu().numpy(), rowptr, colind, values, B, M))
    monkeypatch.setenv("SPARSENE_SRBCRS_BASE_NATIVE", "1")
    (native,) = S.run_SRBCRS(dB, rwo, tid, toff, a2x, M, colind.size, "row")
    p32 = S.Plan(rp, ci, vv, M, 32, 32)
    assert torch.equal(native, p32.run(dB))
    assert_gate(gate(native.cpu().numpy(), rowptr, colind, values, B, M))
