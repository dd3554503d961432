"""GPU parity of the nonzero sweep (grid_order 5, spmm_nzsweep): every legal
setting equals the CPU oracle's fp32 CSR product (oracle_csr_spmm_f32: each
product rounded, then added in ascending column order) bit for bit, passes
the fp64 oracle gate, handles ragged groups (empty windows and rows, a last
group short of W windows, M % 16 != 0, long rows), row maps and omitted
rows of packed plans and last-wins duplicates, is deterministic, and refuses
what it cannot run before launching anything."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle
from tests.helpers import assert_gate, dedupe_last, gate, random_csr

pytestmark = pytest.mark.gpu

NZ = 5
SETTINGS = [(W, U, D) for W in (4, 8) for (U, D) in ((16, 2), (16, 4), (32, 2), (32, 4), (64, 2))]


def _say(*a):
    print("[case]", *a, flush=True)


def _plan(rowptr, colind, values, M, **kw):
    import torch
    from mask_amd.SRBCRSSpMM import Plan
    t = lambda a: torch.from_numpy(a).cuda()
    return Plan(t(rowptr), t(colind), t(values), M, **kw)


def _run(plan, dB, M, N, W, U, D):
    import torch
    out = torch.full((M, N), float("nan"), device="cuda")
    plan.run(dB, out, grid_order=NZ, windows_per_wave=W, tile_b=U, depth=D)
    return out.cpu().numpy()


@pytest.mark.parametrize("M,K,N,density,seed", [
    (16 * 37 + 5, 3000, 512, 0.005, 1),     # ragged last window, last group short of W windows
    (640, 700, 128, 0.03, 2),
    (257, 257, 1024, 0.02, 3),              # 16 chunks of 64 columns: two per XCD
    (900, 2500, 64, 0.01, 4),               # one chunk
    (500, 900, 192, 0.02, 6),               # 3 chunks: not XCD-pinned
    (333, 600, 640, 0.02, 7),               # 10 chunks: not XCD-pinned
])
def test_nzsweep_equals_fp32_csr_oracle(gpu, M, K, N, density, seed):
    import torch
    rowptr, colind, values = random_csr(M, K, density, seed=seed, empty_rows=0.15, heavy_rows=2,
                                        heavy_len=K // 3)
    B = np.random.default_rng(seed).uniform(-1, 1, (K, N)).astype(np.float32)
    plan = _plan(rowptr, colind, values, M)
    dB = torch.from_numpy(B).cuda()
    want = oracle.csr_spmm_f32(rowptr, colind, values, B, M)
    _say("nzsweep", M, K, N)
    for W, U, D in SETTINGS:
        got = _run(plan, dB, M, N, W, U, D)
        assert np.array_equal(got, want), (W, U, D, float(np.nanmax(np.abs(got - want))))
    assert_gate(gate(got, rowptr, colind, values, B, M))
    # within fp32 rounding of the MFMA kernels' product
    ref = plan.run(dB).cpu().numpy()
    assert_gate(gate(ref, rowptr, colind, values, B, M))


def test_nzsweep_uniform_pattern_deterministic(gpu):
    """The uniform workload's shape at 1/16 scale (16 values per row at
    distinct random columns), run twice per setting (the stream is built on
    the first run and reused): equal to the oracle bit for bit both times."""
    import torch
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
    want = oracle.csr_spmm_f32(rowptr, colind, values, B, M)
    _say("nzsweep uniform-like", M)
    for W, U, D in ((8, 32, 2), (4, 16, 2), (8, 64, 2)):
        for _ in range(2):
            assert np.array_equal(_run(plan, dB, M, 512, W, U, D), want), (W, U, D)


def test_nzsweep_packed_plans_and_duplicates(gpu):
    """Row maps (reordered packings) are applied in the store, omitted rows
    are zeroed, and duplicated (row, col) entries follow the plan's
    last-wins policy (the oracle runs on the deduplicated CSR)."""
    import torch
    M = K = 600
    N = 128
    rowptr, colind, values = random_csr(M, K, 0.02, seed=21, empty_rows=0.3)
    B = np.random.default_rng(21).uniform(-1, 1, (K, N)).astype(np.float32)
    dB = torch.from_numpy(B).cuda()
    want = oracle.csr_spmm_f32(rowptr, colind, values, B, M)
    for order in ("row_rcm", "jaccard_greedy", "sparse_rows"):
        _say("nzsweep packed", order)
        plan = _plan(rowptr, colind, values, M, row_order=order, K=K)
        assert np.array_equal(_run(plan, dB, M, N, 8, 32, 2), want), order
    rowptr, colind, values = random_csr(M, K, 0.02, seed=22, duplicates=True, unsorted=True)
    drp, dci, dvv = dedupe_last(rowptr, colind, values)
    plan = _plan(rowptr, colind, values, M)
    _say("nzsweep duplicates")
    assert np.array_equal(_run(plan, dB, M, N, 8, 32, 2), oracle.csr_spmm_f32(drp, dci, dvv, B, M))


def test_nzsweep_default_knobs(gpu):
    """grid_order 5 with every other knob 0 runs the documented defaults
    (8 windows, sub-batches of 32, depth 2)."""
    import torch
    M, K, N = 500, 900, 256
    rowptr, colind, values = random_csr(M, K, 0.02, seed=12)
    B = np.random.default_rng(12).uniform(-1, 1, (K, N)).astype(np.float32)
    plan = _plan(rowptr, colind, values, M)
    dB = torch.from_numpy(B).cuda()
    _say("nzsweep defaults", M, N)
    want = oracle.csr_spmm_f32(rowptr, colind, values, B, M)
    assert np.array_equal(plan.run(dB, grid_order=NZ).cpu().numpy(), want)
    assert np.array_equal(plan.run(dB, grid_order=NZ, wg_cols=64).cpu().numpy(), want)


def test_nzsweep_refusals_leave_c_untouched(gpu):
    import torch
    from mask_amd._capi import SrbcrsError
    M, K = 300, 400
    rowptr, colind, values = random_csr(M, K, 0.03, seed=5)
    plan = _plan(rowptr, colind, values, M)
    cases = [
        (96, dict(), "multiple of 64"),
        (128, dict(windows_per_wave=2), "windows_per_wave"),
        (128, dict(windows_per_wave=16), "windows_per_wave"),
        (128, dict(wg_cols=128), "64 columns"),
        (128, dict(tile_b=64, depth=4), "tile_b"),
        (128, dict(depth=8), "tile_b, depth"),
        (128, dict(a_operand="dense"), "compact"),
        (128, dict(b_stage="lds"), "registers"),
    ]
    for N, kw, msg in cases:
        _say("nzsweep refusal", N, kw)
        dB = torch.ones((K, N), device="cuda")
        out = torch.full((M, N), 7.0, device="cuda")
        with pytest.raises(SrbcrsError, match=msg):
            plan.run(dB, out, grid_order=NZ, **kw)
        torch.cuda.synchronize()
        assert bool((out == 7.0).all())
    # misaligned B (16-byte loads)
    big = torch.ones((K * 128 + 1,), device="cuda")
    dB = big[1:].view(K, 128)
    out = torch.full((M, 128), 7.0, device="cuda")
    with pytest.raises(SrbcrsError, match="aligned"):
        plan.run(dB, out, grid_order=NZ)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
    plan.set_schedule("split", 0)
    out = torch.full((M, 64), 7.0, device="cuda")
    with pytest.raises(SrbcrsError, match="row"):
        plan.run(torch.ones((K, 64), device="cuda"), out, grid_order=NZ)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
    # 32x32 blocks have no compact copy for this kernel
    p32 = _plan(rowptr, colind, values, M, blk_h=32, blk_w=32)
    out = torch.full((M, 64), 7.0, device="cuda")
    with pytest.raises(SrbcrsError, match="16x8"):
        p32.run(torch.ones((K, 64), device="cuda"), out, grid_order=NZ)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())


def test_nzsweep_many_generations(gpu):
    """Several generations of resident waves, runs of empty groups and groups
    of very different sizes: every row equals the oracle's fp32 product."""
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
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    dB = torch.from_numpy(B).cuda()
    plan = _plan(rowptr, colind, values, M)
    want = oracle.csr_spmm_f32(rowptr, colind, values, B, M)
    _say("nzsweep generations", M, N)
    for W, U, D in ((8, 32, 2), (4, 16, 4), (8, 32, 4)):
        assert np.array_equal(_run(plan, dB, M, N, W, U, D), want), (W, U, D)


def test_nzsweep_noalloc_needs_built_stream(gpu):
    """srbcrs_run_noalloc refuses a nonzero-sweep setting whose stream is not
    built (C untouched) and, once srbcrs_run_ex has built it, gives the same
    bits."""
    import ctypes
    import torch
    from mask_amd import _capi
    L = _capi.lib()
    M, K, N = 700, 900, 128
    rowptr, colind, values = random_csr(M, K, 0.02, seed=31)
    plan = _plan(rowptr, colind, values, M)
    B = torch.from_numpy(np.random.default_rng(31).uniform(-1, 1, (K, N)).astype(np.float32)).cuda()
    opts = _capi.RunOpts(2, 32, 0, NZ, 8, 0, 0)
    st = torch.cuda.current_stream().cuda_stream

    def call(fn, C):
        return fn(plan.handle, B.data_ptr(), K, N, B.stride(0), C.data_ptr(), C.stride(0), M,
                  ctypes.byref(opts), st)

    _say("nzsweep noalloc")
    got = torch.full((M, N), 7.0, device="cuda")
    assert call(L.srbcrs_run_noalloc, got) == _capi.SRBCRS_EINVAL
    assert "not built" in L.srbcrs_last_error().decode()
    torch.cuda.synchronize()
    assert bool((got == 7.0).all())
    ref = torch.full((M, N), float("nan"), device="cuda")
    _capi.check(call(L.srbcrs_run_ex, ref))
    _capi.check(call(L.srbcrs_run_noalloc, got))
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


def test_tune_ex_admits_the_sweep(gpu):
    """srbcrs_plan_tune_ex with SRBCRS_TUNE_NONZERO_SWEEP keeps a setting
    whose later default-knob runs give its own bits (the fp32 CSR product's
    when it picked the sweep, the MFMA kernels' otherwise); unknown flag
    bits are refused."""
    import ctypes
    import torch
    from mask_amd import _capi
    rng = np.random.default_rng(41)
    M = K = 8192
    cols = np.stack([np.sort(rng.choice(K, 16, replace=False)) for _ in range(M)])
    rowptr = np.arange(0, 16 * M + 1, 16, dtype=np.int32)
    colind = cols.ravel().astype(np.int32)
    values = rng.uniform(-1, 1, colind.size).astype(np.float32)
    B = rng.uniform(-1, 1, (K, 512)).astype(np.float32)
    plan = _plan(rowptr, colind, values, M)
    dB = torch.from_numpy(B).cuda()
    mfma = plan.run(dB).cpu().numpy()
    csr = oracle.csr_spmm_f32(rowptr, colind, values, B, M)
    _say("tune_ex")
    choice = plan.tune(dB, reps=2, nonzero_sweep=True)
    got = plan.run(dB).cpu().numpy()
    assert np.array_equal(got, csr if choice["grid_order"] == NZ else mfma), choice
    out = torch.empty((M, 512), device="cuda")
    rc = _capi.lib().srbcrs_plan_tune_ex(plan.handle, dB.data_ptr(), K, 512, 512, out.data_ptr(), 512, M, 1, 2,
                                         None, torch.cuda.current_stream().cuda_stream)
    assert rc == _capi.SRBCRS_EINVAL and "flags" in _capi.lib().srbcrs_last_error().decode()


def test_dropin_dispatch_under_csr_fallback(gpu, monkeypatch):
    """run_SRBCRS_16x8 with SPARSENE_ALLOW_CSR_FALLBACK=1 runs the nonzero
    sweep on low-block-fill plans (bits = the fp32 CSR oracle's) and the MFMA
    kernels on dense-block plans, on widths the sweep refuses and without the
    opt-in (bits = the default run's)."""
    import torch
    from mask_amd import SRBCRSSpMM as S

    def run(rowptr, colind, values, M, K, N, seed):
        B = np.random.default_rng(seed).uniform(-1, 1, (K, N)).astype(np.float32)
        ci, rp, vv = (torch.from_numpy(a).cuda() for a in (colind, rowptr, values))
        z = torch.zeros(1, dtype=torch.int32, device="cuda")
        rwo, _, tid, toff, a2x, _ = S.preprocess_gpu_16x8(ci, rp, vv, M, 16, 8, z, z, z)
        dB = torch.from_numpy(B).cuda()
        (out,) = S.run_SRBCRS_16x8(dB, rwo, tid, toff, a2x, M, int(colind.size), "")
        plan = S.plan_for(rwo)
        return out.cpu().numpy(), plan.run(dB).cpu().numpy(), oracle.csr_spmm_f32(rowptr, colind, values, B, M)

    # the GCN bridge leaves SRBCRS_TILE_B set for the module, as the reference's does
    monkeypatch.delenv("SRBCRS_TILE_B", raising=False)
    M = K = 2048
    sparse = random_csr(M, K, 0.004, seed=51)             # ~1 value per block column: fill ~0.06
    rng = np.random.default_rng(52)                       # dense 16x8 blocks on the diagonal: fill 1
    rows = np.repeat(np.arange(M), 8)
    cols = (rows // 8) * 8 + np.tile(np.arange(8), M)
    rp = np.zeros(M + 1, np.int32)
    rp[1:] = np.cumsum(np.bincount(rows, minlength=M))
    dense_blocks = (rp, cols.astype(np.int32), rng.uniform(-1, 1, cols.size).astype(np.float32))
    _say("dispatch")
    monkeypatch.setenv("SPARSENE_ALLOW_CSR_FALLBACK", "1")
    got, mfma, csr = run(*sparse, M, K, 128, 1)
    assert np.array_equal(got, csr) and not np.array_equal(got, mfma)
    got, mfma, csr = run(*sparse, M, K, 96, 2)            # N % 64 != 0: refused, MFMA default
    assert np.array_equal(got, mfma)
    got, mfma, csr = run(*dense_blocks, M, K, 128, 3)
    assert np.array_equal(got, mfma)
    monkeypatch.delenv("SPARSENE_ALLOW_CSR_FALLBACK")
    got, mfma, csr = run(*sparse, M, K, 128, 4)
    assert np.array_equal(got, mfma)


def test_nzsweep_b_beyond_2gib(gpu):
    """B rows whose byte offsets pass 2^31 (K * ldb * 4 between 2 and 4 GiB,
    which the 32-bit buffer offsets allow): B is a 64-column view of a
    600000 x 1024 buffer (2.46 GB), and rows reference columns above 524288
    (offsets above 2^31).  Equal to the oracle's fp32 product bit for bit."""
    import torch
    rng = np.random.default_rng(61)
    M, K, N, LD = 4096, 600000, 64, 1024
    rows = []
    for c in rng.integers(0, 12, size=M):
        # about half of each row's columns in the top eighth of B
        cand = np.concatenate([rng.choice(K, c // 2 + 1, replace=False), rng.integers(K - K // 8, K, c // 2 + 1)])
        rows.append(np.sort(np.unique(cand))[:c])
    rowptr = np.zeros(M + 1, np.int64)
    rowptr[1:] = np.cumsum([r.size for r in rows])
    rowptr = rowptr.astype(np.int32)
    colind = np.concatenate(rows).astype(np.int32)
    values = rng.uniform(-1, 1, colind.size).astype(np.float32)
    assert int(colind.max()) * LD * 4 >= 2 ** 31
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    big = torch.zeros((K, LD), device="cuda")
    big[:, :N] = torch.from_numpy(B).cuda()
    dB = big[:, :N]
    plan = _plan(rowptr, colind, values, M)
    _say("nzsweep beyond 2 GiB", K, LD)
    out = torch.full((M, N), float("nan"), device="cuda")
    plan.run(dB, out, grid_order=NZ)
    want = oracle.csr_spmm_f32(rowptr, colind, values, B, M)
    assert np.array_equal(out.cpu().numpy(), want)
    del big, dB
    torch.cuda.empty_cache()


def test_nzsweep_empty_matrix_and_wide_c(gpu):
    """A matrix without stored values writes zeros to every row; C with a
    leading dimension above N (a view of a wider buffer) keeps the columns
    outside the view untouched."""
    import torch
    M, K, N = 300, 400, 128
    rowptr = np.zeros(M + 1, np.int32)
    plan = _plan(rowptr, np.zeros(0, np.int32), np.zeros(0, np.float32), M)
    dB = torch.ones((K, N), device="cuda")
    out = torch.full((M, N), 7.0, device="cuda")
    _say("nzsweep empty")
    plan.run(dB, out, grid_order=NZ)
    assert bool((out == 0).all())
    rowptr, colind, values = random_csr(M, K, 0.03, seed=71)
    B = np.random.default_rng(71).uniform(-1, 1, (K, N)).astype(np.float32)
    plan = _plan(rowptr, colind, values, M)
    wide = torch.full((M, 3 * N), 7.0, device="cuda")
    plan.run(torch.from_numpy(B).cuda(), wide[:, N:2 * N], grid_order=NZ)
    got = wide.cpu().numpy()
    assert np.array_equal(got[:, N:2 * N], oracle.csr_spmm_f32(rowptr, colind, values, B, M))
    assert (got[:, :N] == 7.0).all() and (got[:, 2 * N:] == 7.0).all()


def test_nzsweep_refuses_a_stream_of_padding(gpu):
    """One row far longer than its group's others would put one of its values
    per sub-batch and pad the rest (200000 values, 6.4 M entries): the sweep
    refuses before any launch (C untouched), and the drop-in's dispatch falls
    back to the MFMA kernels."""
    import torch
    from mask_amd._capi import SrbcrsError
    rng = np.random.default_rng(81)
    M, K, N = 64, 300000, 64
    rows = [np.sort(rng.choice(K, 200000, replace=False))] + [np.sort(rng.choice(K, 2, replace=False))
                                                              for _ in range(M - 1)]
    rowptr = np.zeros(M + 1, np.int32)
    rowptr[1:] = np.cumsum([r.size for r in rows])
    colind = np.concatenate(rows).astype(np.int32)
    values = rng.uniform(-1, 1, colind.size).astype(np.float32)
    plan = _plan(rowptr, colind, values, M)
    dB = torch.ones((K, N), device="cuda")
    out = torch.full((M, N), 7.0, device="cuda")
    _say("nzsweep padding refusal")
    with pytest.raises(SrbcrsError, match="pad"):
        plan.run(dB, out, grid_order=NZ)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
    assert not plan.run_sweep_if_sparse(dB, out)
    assert bool((out == 7.0).all())
