"""GPU parity of the gfx950 SR-BCRS SpMM against the CPU oracle.

Every case prints its name/shape before touching the GPU so that a failing
run names its case.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle
from tests.helpers import assert_gate, dedupe_last, gate, random_csr

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def _run_plan(rowptr, colind, values, M, B, policy=("row", 0), device=None, blk=(16, 8)):
    torch = _torch()
    from mask_amd.SRBCRSSpMM import Plan
    dev = device or torch.device("cuda", 0)
    plan = Plan(torch.from_numpy(rowptr).to(dev), torch.from_numpy(colind).to(dev), torch.from_numpy(values).to(dev),
                M, blk[0], blk[1])
    plan.set_schedule(*policy)
    dB = torch.from_numpy(B).to(dev)
    out = plan.run(dB)
    torch.cuda.synchronize()
    return out.cpu().numpy(), plan


def _say(*a):
    print("[case]", *a, flush=True)


def test_identity_is_exact(gpu):
    """A = I: every MFMA lane mapping error shows up as a wrong element."""
    for M, N in ((64, 64), (100, 128), (48, 16), (40, 32)):
        _say("identity", M, N)
        rowptr = np.arange(M + 1, dtype=np.int32)
        colind = np.arange(M, dtype=np.int32)
        values = np.ones(M, np.float32)
        B = np.random.default_rng(M).uniform(-1, 1, (M, N)).astype(np.float32)
        C, _ = _run_plan(rowptr, colind, values, M, B)
        assert np.array_equal(C, B)


def test_permutation_scaled_exact(gpu):
    """One nonzero per row at a permuted column with a power-of-two value:
    C is an exactly scaled row gather of B."""
    M, N = 300, 96
    rng = np.random.default_rng(5)
    perm = rng.permutation(M).astype(np.int32)
    scale = (2.0 ** rng.integers(-3, 4, size=M)).astype(np.float32)
    rowptr = np.arange(M + 1, dtype=np.int32)
    B = rng.uniform(-1, 1, (M, N)).astype(np.float32)
    _say("permutation", M, N)
    C, _ = _run_plan(rowptr, perm, scale, M, B)
    assert np.array_equal(C, scale[:, None] * B[perm])


def test_dense_block_matches_matmul(gpu):
    """A fully dense 16 x 8k matrix: every block full, C = A @ B."""
    M, K, N = 16, 64, 64
    rng = np.random.default_rng(9)
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    rowptr = (np.arange(M + 1) * K).astype(np.int32)
    colind = np.tile(np.arange(K, dtype=np.int32), M)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    _say("dense", M, K, N)
    C, _ = _run_plan(rowptr, colind, A.reshape(-1), M, B)
    assert_gate(gate(C, rowptr, colind, A.reshape(-1), B, M))
    np.testing.assert_allclose(C, A.astype(np.float64) @ B.astype(np.float64), rtol=0, atol=1e-5)


@pytest.mark.parametrize("N", [16, 32, 48, 64, 96, 128, 192, 256, 512])
@pytest.mark.parametrize("M", [1, 17, 250])
def test_random_shapes(gpu, M, N):
    K = 333
    rowptr, colind, values = random_csr(M, K, 0.05, seed=M * 1000 + N, empty_rows=0.1)
    B = np.random.default_rng(N).uniform(-1, 1, (K, N)).astype(np.float32)
    _say("random", M, K, N)
    C, _ = _run_plan(rowptr, colind, values, M, B)
    assert_gate(gate(C, rowptr, colind, values, B, M))


def test_unsorted_and_duplicates(gpu):
    M, K, N = 200, 500, 64
    rowptr, colind, values = random_csr(M, K, 0.04, seed=3, unsorted=True, duplicates=True)
    B = np.random.default_rng(1).uniform(-1, 1, (K, N)).astype(np.float32)
    _say("unsorted+dup", M, K, N)
    C, _ = _run_plan(rowptr, colind, values, M, B)
    rp, ci, vv = dedupe_last(rowptr, colind, values)   # last write wins
    assert_gate(gate(C, rp, ci, vv, B, M))


def test_empty_matrix_writes_zeros(gpu):
    torch = _torch()
    M, K, N = 37, 10, 32
    rowptr = np.zeros(M + 1, np.int32)
    colind = np.zeros(0, np.int32)
    values = np.zeros(0, np.float32)
    B = np.ones((K, N), np.float32)
    from mask_amd.SRBCRSSpMM import Plan
    _say("empty", M, N)
    plan = Plan(torch.from_numpy(rowptr).cuda(), torch.from_numpy(colind).cuda(), torch.from_numpy(values).cuda(), M)
    out = torch.full((M, N), 7.0, device="cuda")
    plan.run(torch.from_numpy(B).cuda(), out)
    torch.cuda.synchronize()
    assert plan.total_blocks == 0
    assert torch.count_nonzero(out).item() == 0


@pytest.mark.parametrize("policy", [("row", 0), ("split", 0), ("split", 3), ("strict_lb", 0), ("strict_lb", 5),
                                    ("multi_bind", 0)])
def test_schedules_skewed(gpu, policy):
    """Skewed rows (a few very long rows): every schedule within the gate,
    and each is deterministic run to run."""
    torch = _torch()
    M, K, N = 400, 3000, 128
    rowptr, colind, values = random_csr(M, K, 0.01, seed=11, heavy_rows=20, heavy_len=1500, empty_rows=0.2)
    B = np.random.default_rng(2).uniform(-1, 1, (K, N)).astype(np.float32)
    _say("schedule", policy, M, K, N)
    C, plan = _run_plan(rowptr, colind, values, M, B, policy)
    assert_gate(gate(C, rowptr, colind, values, B, M))
    C2 = plan.run(torch.from_numpy(B).cuda()).cpu().numpy()
    assert np.array_equal(C, C2)


def test_split_without_cuts_is_bitwise_row(gpu):
    """A split schedule whose cap exceeds every window runs the task kernel
    on exactly the row kernel's work: identical bits."""
    M, K, N = 300, 800, 64
    rowptr, colind, values = random_csr(M, K, 0.03, seed=21, empty_rows=0.1)
    B = np.random.default_rng(3).uniform(-1, 1, (K, N)).astype(np.float32)
    _say("split-vs-row", M, K, N)
    C_row, _ = _run_plan(rowptr, colind, values, M, B, ("row", 0))
    C_split, _ = _run_plan(rowptr, colind, values, M, B, ("split", 100000))
    assert np.array_equal(C_row, C_split)


@pytest.mark.parametrize("name,scale_down,N", [("uniform-4096", 1, 64), ("uniform-65536", 8, 512),
                                               ("banded-524288", 64, 512), ("rmat-2^20", 64, 512),
                                               ("gcn-232965", 32, 256), ("gcn-232965", 32, 64)])
def test_workloads_scaled(gpu, name, scale_down, N):
    from mask_amd import datasets
    m = datasets.make_config(name, scale_down=scale_down)
    B = m.dense(N)
    _say("workload", name, m.M, m.nnz, N)
    policy = ("split", 0) if name.startswith(("rmat", "gcn")) else ("row", 0)
    C, _ = _run_plan(m.rowptr, m.colind, m.values, m.M, B, policy)
    assert_gate(gate(C, m.rowptr, m.colind, m.values, B, m.M))


def test_csr_fallback(gpu):
    torch = _torch()
    from mask_amd.SRBCRSSpMM import csr_spmm
    for M, K, N in ((300, 500, 64), (129, 77, 512), (50, 40, 48)):
        _say("csr", M, K, N)
        rowptr, colind, values = random_csr(M, K, 0.05, seed=M + N, empty_rows=0.1)
        B = np.random.default_rng(N).uniform(-1, 1, (K, N)).astype(np.float32)
        out = csr_spmm(torch.from_numpy(rowptr).cuda(), torch.from_numpy(colind).cuda(),
                       torch.from_numpy(values).cuda(), torch.from_numpy(B).cuda(), M)
        torch.cuda.synchronize()
        assert_gate(gate(out.cpu().numpy(), rowptr, colind, values, B, M))


@pytest.mark.parametrize("blk", [(16, 8), (32, 32)])
def test_knobs_are_bitwise_invariant(gpu, blk):
    """Depth, tile_b, workgroup width, grid order and windows-per-wave change
    only the mapping, never the per-element accumulation order: every
    combination reproduces the default result bit for bit (for 32x32
    blocks, wg_cols 256 and 512 select the 128-column waves)."""
    torch = _torch()
    import itertools
    M, K, N = 333, 900, 256
    rowptr, colind, values = random_csr(M, K, 0.02, seed=31, empty_rows=0.3, heavy_rows=3, heavy_len=400)
    B = np.random.default_rng(4).uniform(-1, 1, (K, N)).astype(np.float32)
    _say("knobs", blk, M, K, N)
    ref, plan = _run_plan(rowptr, colind, values, M, B, blk=blk)
    dB = torch.from_numpy(B).cuda()
    for depth, tile_b, wgc, go, wpw in itertools.product([2, 4, 8], [0, 16, 32], [0, 64, 256], [1, 2, 3], [1, 3, 16]):
        out = plan.run(dB, depth=depth, tile_b=tile_b, wg_cols=wgc, grid_order=go, windows_per_wave=wpw)
        assert np.array_equal(out.cpu().numpy(), ref), (depth, tile_b, wgc, go, wpw)
    # B staged through LDS by direct-to-LDS loads: same MFMA inputs, same bits
    for depth, wgc, go, wpw, a_op in itertools.product([2, 4, 8], [0, 64, 128, 256], [1, 3], [1, 3],
                                                       ["compact", "dense"]):
        out = plan.run(dB, depth=depth, wg_cols=wgc, grid_order=go, windows_per_wave=wpw, a_operand=a_op,
                       b_stage="lds")
        assert np.array_equal(out.cpu().numpy(), ref), ("lds", depth, wgc, go, wpw, a_op)
    for pol in (("split", 0), ("strict_lb", 7), ("multi_bind", 0)):
        plan.set_schedule(*pol)
        base = plan.run(dB).cpu().numpy()
        for depth, wgc, go, bst in itertools.product([4, 8], [0, 64, 512], [1, 2, 3], ["registers", "lds"]):
            out = plan.run(dB, depth=depth, wg_cols=wgc, grid_order=go, b_stage=bst)
            assert np.array_equal(out.cpu().numpy(), base), (pol, depth, wgc, go, bst)


@pytest.mark.parametrize("blk", [(16, 8), (32, 32)])
def test_lds_stage_largest_lds_footprint(gpu, blk):
    """LDS-staged B at its largest per-workgroup footprint (4 waves x depth 8
    x 8 rows x 128 columns = 128 KB of the 160 KB LDS): launches and gives
    the register ring's bits."""
    torch = _torch()
    M, K, N = 200, 300, 512
    rowptr, colind, values = random_csr(M, K, 0.05, seed=77, heavy_rows=2, heavy_len=250)
    B = np.random.default_rng(5).uniform(-1, 1, (K, N)).astype(np.float32)
    _say("lds footprint", blk)
    ref, plan = _run_plan(rowptr, colind, values, M, B, blk=blk)
    dB = torch.from_numpy(B).cuda()
    for depth in (2, 4, 8):
        out = plan.run(dB, depth=depth, wg_cols=512, b_stage="lds")
        assert np.array_equal(out.cpu().numpy(), ref), depth
