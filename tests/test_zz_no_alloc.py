"""srbcrs_run_noalloc through the C ABI: the allocation-free entry point
gives the bits of srbcrs_run_ex on the same plan and operands, on two calls
in a row (the second smaller), for split schedules (partial tiles in the
library's fixed scratch array) and the row schedule; it rejects a schedule
whose partial tiles exceed the scratch, before any launch (C untouched,
packed plans' omitted rows included); it allocates nothing, also under HIP
graph capture on a fresh plan."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from tests.helpers import assert_gate, gate, random_csr

pytestmark = pytest.mark.gpu


def _run(fn, plan, B, C, opts=None):
    import torch
    from mask_amd import _capi
    st = torch.cuda.current_stream().cuda_stream
    return fn(plan.handle, B.data_ptr(), B.shape[0], B.shape[1], B.stride(0), C.data_ptr(), C.stride(0),
              C.shape[0], ctypes.byref(opts) if opts is not None else None, st)


@pytest.mark.parametrize("blk", [(16, 8), (32, 32)])
def test_noalloc_matches_run_ex_twice(gpu, blk):
    import torch
    from mask_amd import _capi
    from mask_amd.SRBCRSSpMM import Plan
    L = _capi.lib()
    assert L.srbcrs_noalloc_scratch_floats() == 16 << 20
    cases = [(900, 2500, 256, 31), (300, 700, 64, 32)]     # the second call is smaller
    for pol, param in (("split", 4), ("strict_lb", 16), ("row", 0)):
        for M, K, N, seed in cases:
            print("[case] noalloc", blk, pol, M, K, N, flush=True)
            rowptr, colind, values = random_csr(M, K, 0.02, seed=seed, heavy_rows=4, heavy_len=K // 2,
                                                empty_rows=0.1)
            B = torch.from_numpy(np.random.default_rng(seed).uniform(-1, 1, (K, N)).astype(np.float32)).cuda()
            plan = Plan(*(torch.from_numpy(a).cuda() for a in (rowptr, colind, values)), M, *blk)
            plan.set_schedule(pol, param)
            ref = torch.full((M, N), float("nan"), device="cuda")
            got = torch.full((M, N), float("nan"), device="cuda")
            _capi.check(_run(L.srbcrs_run_ex, plan, B, ref))
            _capi.check(_run(L.srbcrs_run_noalloc, plan, B, got))
            torch.cuda.synchronize()
            assert torch.equal(got, ref), (pol, M, N)
            assert_gate(gate(got.cpu().numpy(), rowptr, colind, values, B.cpu().numpy(), M))


def test_noalloc_rejects_oversized_partials(gpu):
    """A split whose partial tiles (slots x 16 rows x ldc floats) exceed the
    64 MiB scratch is refused with a clear error and launches nothing."""
    import torch
    from mask_amd import _capi
    from mask_amd.SRBCRSSpMM import Plan
    L = _capi.lib()
    M, K = 4096, 64
    # every row holds all 64 columns: each 16-row window has 8 blocks; cap 1 -> 8 slots per window
    rowptr = np.arange(0, (M + 1) * K, K, dtype=np.int32)
    colind = np.tile(np.arange(K, dtype=np.int32), M)
    values = np.ones(M * K, np.float32)
    plan = Plan(*(torch.from_numpy(a).cuda() for a in (rowptr, colind, values)), M)
    plan.set_schedule("split", 1)
    N = 576    # 256 windows x 8 slots x 16 rows x 576 = 18.9 M floats > 16 M (16,777,216)
    B = torch.ones((K, N), device="cuda")
    C = torch.zeros((M, N), device="cuda")
    rc = _run(L.srbcrs_run_noalloc, plan, B, C)
    assert rc == _capi.SRBCRS_EINVAL
    assert "scratch" in L.srbcrs_last_error().decode()
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(C)) == 0
    # a packing that leaves rows out (their zeroing is a launch of its own):
    # the refused call must not have zeroed them either
    colind2 = np.concatenate([colind[rowptr[r]:rowptr[r + 1]] for r in range(1, M, 2)])
    rowptr2 = np.concatenate([[0], np.cumsum([K if r % 2 else 0 for r in range(M)])]).astype(np.int32)  # even rows empty
    values2 = np.ones(colind2.size, np.float32)
    sparse = Plan(*(torch.from_numpy(a).cuda() for a in (rowptr2, colind2, values2)), M, row_order="sparse_rows", K=K)
    sparse.set_schedule("split", 1)
    N2 = 1152   # 128 windows x 8 slots x 16 rows x 1152 = 18.9 M floats > 16 M
    B2 = torch.ones((K, N2), device="cuda")
    C2 = torch.full((M, N2), 7.0, device="cuda")
    rc = _run(L.srbcrs_run_noalloc, sparse, B2, C2)
    assert rc == _capi.SRBCRS_EINVAL and "scratch" in L.srbcrs_last_error().decode()
    torch.cuda.synchronize()
    assert bool((C2 == 7.0).all())
    # the allocating entry point runs the same schedule
    _capi.check(_run(L.srbcrs_run_ex, plan, B, C))
    torch.cuda.synchronize()
    assert float(C[0, 0]) == 64.0


def test_noalloc_allocates_nothing_and_captures(gpu):
    """On fresh plans (no srbcrs_run_ex before), srbcrs_run_noalloc leaves the
    device's free memory unchanged, and it can be captured into a HIP graph
    (allocation is forbidden under capture); every replay, with eager work
    between replays, equals srbcrs_run_ex bit for bit."""
    import torch
    from mask_amd import _capi
    from mask_amd.SRBCRSSpMM import Plan
    L = _capi.lib()
    M, K, N = 900, 2500, 256
    rowptr, colind, values = random_csr(M, K, 0.02, seed=41, heavy_rows=4, heavy_len=K // 2, empty_rows=0.1)
    B = torch.from_numpy(np.random.default_rng(41).uniform(-1, 1, (K, N)).astype(np.float32)).cuda()
    mk = lambda: Plan(*(torch.from_numpy(a).cuda() for a in (rowptr, colind, values)), M)
    print("[case] noalloc free memory", flush=True)
    plan = mk()
    plan.set_schedule("split", 4)
    out = torch.full((M, N), float("nan"), device="cuda")
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    _capi.check(_run(L.srbcrs_run_noalloc, plan, B, out))
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    print("[case] noalloc graph capture", flush=True)
    plan2 = mk()
    plan2.set_schedule("split", 4)
    got = torch.full((M, N), float("nan"), device="cuda")
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        _capi.check(_run(L.srbcrs_run_noalloc, plan2, B, got))
    ref = torch.full((M, N), float("nan"), device="cuda")
    plan3 = mk()
    plan3.set_schedule("split", 4)
    _capi.check(_run(L.srbcrs_run_ex, plan3, B, ref))
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    for i in range(3):
        got.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, ref), i
        _capi.check(_run(L.srbcrs_run_ex, plan3, B, out))   # eager work between replays
        torch.cuda.synchronize()
    assert_gate(gate(got.cpu().numpy(), rowptr, colind, values, B.cpu().numpy(), M))
