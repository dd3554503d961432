"""GPU parity of the merged-window grid (grid_order 4, spmm_merged): every
legal setting reproduces the default row kernel bit for bit (each window
receives its blocks' MFMAs in its own order), passes the fp64 oracle gate,
handles ragged groups (windows with different block counts, empty windows,
a last group with fewer than W windows, M % 16 != 0), row maps and omitted
rows of packed plans, and refuses what it cannot run before launching
anything."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import assert_gate, gate, random_csr

pytestmark = pytest.mark.gpu

MERGED = 4
SETTINGS = [(64, 8, 2), (64, 4, 2), (64, 4, 4), (128, 4, 2), (128, 4, 4)]   # (wg_cols, windows per group, depth)


def _say(*a):
    print("[case]", *a, flush=True)


def _plan(rowptr, colind, values, M, **kw):
    import torch
    from mask_amd.SRBCRSSpMM import Plan
    t = lambda a: torch.from_numpy(a).cuda()
    return Plan(t(rowptr), t(colind), t(values), M, **kw)


@pytest.mark.parametrize("M,K,N,density,seed", [
    (16 * 37 + 5, 3000, 512, 0.005, 1),     # ragged last window, last group short of W windows
    (640, 700, 128, 0.03, 2),
    (257, 257, 1024, 0.02, 3),              # 16 chunks of 64 columns: two per XCD
    (900, 2500, 64, 0.01, 4),               # one chunk: every XCD on its own groups
])
def test_merged_bitwise_equals_row_kernel(gpu, M, K, N, density, seed):
    import torch
    rowptr, colind, values = random_csr(M, K, density, seed=seed, empty_rows=0.15, heavy_rows=2,
                                        heavy_len=K // 3)
    B = np.random.default_rng(seed).uniform(-1, 1, (K, N)).astype(np.float32)
    plan = _plan(rowptr, colind, values, M)
    dB = torch.from_numpy(B).cuda()
    _say("merged", M, K, N)
    ref = plan.run(dB).cpu().numpy()
    assert_gate(gate(ref, rowptr, colind, values, B, M))
    for wg, W, depth in SETTINGS:
        ch = N // wg
        if N % wg or ch == 0 or (ch > 8 and ch % 8) or (ch < 8 and 8 % ch):
            continue
        out = torch.full((M, N), float("nan"), device="cuda")
        plan.run(dB, out, depth=depth, wg_cols=wg, grid_order=MERGED, windows_per_wave=W)
        assert np.array_equal(out.cpu().numpy(), ref), (wg, W, depth)


def test_merged_uniform_pattern_full_rows(gpu):
    """The uniform workload's shape at 1/16 scale (16 nonzeros per row at
    distinct random columns): every row checked against the oracle and
    against the default kernel's bits, twice (the interleaved copy is built
    on the first run and reused)."""
    import torch
    from mask_amd import datasets
    m = datasets.make_config("uniform-4096")
    rng = np.random.default_rng(11)
    M = K = 4096
    cols = np.stack([rng.choice(K, 16, replace=False) for _ in range(M)])
    cols.sort(axis=1)
    rowptr = np.arange(0, 16 * M + 1, 16, dtype=np.int32)
    colind = cols.ravel().astype(np.int32)
    values = rng.uniform(-1, 1, colind.size).astype(np.float32)
    B = rng.uniform(-1, 1, (K, 512)).astype(np.float32)
    plan = _plan(rowptr, colind, values, M)
    dB = torch.from_numpy(B).cuda()
    _say("merged uniform-like", M, m.name)
    ref = plan.run(dB).cpu().numpy()
    for _ in range(2):
        out = plan.run(dB, wg_cols=64, grid_order=MERGED, windows_per_wave=8)
        got = out.cpu().numpy()
        assert np.array_equal(got, ref)
    assert_gate(gate(got, rowptr, colind, values, B, M))


def test_merged_packed_plans(gpu):
    """Row maps (reordered packings) are applied in the store and omitted
    rows are zeroed, as on the default grid."""
    import torch
    M = K = 600
    N = 128
    rowptr, colind, values = random_csr(M, K, 0.02, seed=21, empty_rows=0.3)
    B = np.random.default_rng(21).uniform(-1, 1, (K, N)).astype(np.float32)
    dB = torch.from_numpy(B).cuda()
    for order in ("row_rcm", "jaccard_greedy", "sparse_rows"):
        _say("merged packed", order)
        plan = _plan(rowptr, colind, values, M, row_order=order, K=K)
        ref = plan.run(dB).cpu().numpy()
        out = torch.full((M, N), float("nan"), device="cuda")
        plan.run(dB, out, wg_cols=64, grid_order=MERGED, windows_per_wave=8)
        assert np.array_equal(out.cpu().numpy(), ref), order
        assert_gate(gate(ref, rowptr, colind, values, B, M))


def test_merged_default_knobs(gpu):
    """grid_order 4 with every other knob 0 runs the documented defaults
    (64-column waves, 8 windows, depth 2) and gives the row kernel's bits."""
    import torch
    M, K, N = 500, 900, 256
    rowptr, colind, values = random_csr(M, K, 0.02, seed=12)
    plan = _plan(rowptr, colind, values, M)
    dB = torch.from_numpy(np.random.default_rng(12).uniform(-1, 1, (K, N)).astype(np.float32)).cuda()
    _say("merged defaults", M, N)
    ref = plan.run(dB).cpu().numpy()
    assert np.array_equal(plan.run(dB, grid_order=MERGED).cpu().numpy(), ref)
    assert np.array_equal(plan.run(dB, grid_order=MERGED, wg_cols=128).cpu().numpy(), ref)   # 128 x 4 windows
    assert np.array_equal(plan.run(dB, grid_order=MERGED, wg_cols=128, windows_per_wave=4).cpu().numpy(), ref)


def test_merged_refusals_leave_c_untouched(gpu):
    import torch
    from mask_amd._capi import SrbcrsError
    M, K = 300, 400
    rowptr, colind, values = random_csr(M, K, 0.03, seed=5)
    plan = _plan(rowptr, colind, values, M)
    cases = [
        (192, dict(wg_cols=64, windows_per_wave=8), "divide 8"),          # 3 chunks
        (128, dict(wg_cols=128, windows_per_wave=2), "windows_per_wave"),
        (128, dict(wg_cols=256, windows_per_wave=4), "wg_cols"),
        (128, dict(wg_cols=64, windows_per_wave=8, depth=8), "depth"),
        (128, dict(wg_cols=64, windows_per_wave=8, depth=4), "8 windows"),
        (128, dict(wg_cols=128, windows_per_wave=8), "8 windows"),
        (128, dict(wg_cols=64, windows_per_wave=8, a_operand="dense"), "compact"),
        (96, dict(wg_cols=64, windows_per_wave=4), "multiples of 64"),
    ]
    for N, kw, msg in cases:
        _say("merged refusal", N, kw)
        dB = torch.ones((K, N), device="cuda")
        out = torch.full((M, N), 7.0, device="cuda")
        with pytest.raises(SrbcrsError, match=msg):
            plan.run(dB, out, grid_order=MERGED, **kw)
        torch.cuda.synchronize()
        assert bool((out == 7.0).all())
    plan.set_schedule("split", 0)
    out = torch.full((M, 64), 7.0, device="cuda")
    with pytest.raises(SrbcrsError, match="row"):
        plan.run(torch.ones((K, 64), device="cuda"), out, grid_order=MERGED, wg_cols=64, windows_per_wave=8)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())


def test_merged_many_generations(gpu):
    """A grid of several generations of resident waves with runs of empty
    groups and groups of very different block counts (many null units):
    bits equal the row kernel's on every row, and a row sample passes the
    oracle gate."""
    import torch
    rng = np.random.default_rng(3)
    M = K = 72000
    counts = rng.integers(0, 9, size=M)
    counts[16 * 100:16 * 140] = 0           # 40 empty windows: whole empty groups
    rowptr = np.zeros(M + 1, np.int64)
    rowptr[1:] = np.cumsum(counts)
    colind = np.concatenate([np.sort(rng.choice(K, c, replace=False)) for c in counts]).astype(np.int32)
    values = rng.uniform(-1, 1, colind.size).astype(np.float32)
    rowptr = rowptr.astype(np.int32)
    N = 512
    dB = torch.from_numpy(rng.uniform(-1, 1, (K, N)).astype(np.float32)).cuda()
    plan = _plan(rowptr, colind, values, M)
    _say("merged persistent", M, N)
    ref = plan.run(dB).cpu().numpy()
    for wg, W, depth in SETTINGS:
        out = torch.full((M, N), float("nan"), device="cuda")
        plan.run(dB, out, depth=depth, wg_cols=wg, grid_order=MERGED, windows_per_wave=W)
        assert np.array_equal(out.cpu().numpy(), ref), (wg, W, depth)
    rows = np.sort(rng.choice(M, 2048, replace=False))
    sub = ref[rows]
    rp = np.concatenate([[0], np.cumsum(counts[rows])]).astype(np.int32)
    idx = np.concatenate([np.arange(rowptr[r], rowptr[r + 1]) for r in rows])
    assert_gate(gate(sub, rp, colind[idx], values[idx], dB.cpu().numpy(), rows.size))
