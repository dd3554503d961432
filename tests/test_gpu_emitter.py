"""The HIP emitter's generated operators on the GPU: they instantiate the
same kernel templates with the strategy's parameters, so their output must
equal the library's bit for bit, for every schedule."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import assert_gate, gate, random_csr

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[case]", *a, flush=True)


@pytest.mark.parametrize("blk,lds", [((16, 8), False), ((32, 32), False), ((16, 8), True)])
def test_generated_operator_matches_library(gpu, blk, lds):
    """lds: the operator of a strategy that materializes B in shared memory
    (B staged through LDS by direct-to-LDS loads)."""
    import torch
    from mask_amd.build import GENERATED
    from mask_amd.emitter import GeneratedOperator
    from mask_amd.SRBCRSSpMM import Plan
    bh, bw = blk
    op = GeneratedOperator(GENERATED / f"sr_bcrs_{bh}x{bw}{'_lds' if lds else ''}.so")
    assert op.params.b_lds == lds
    M, K, N = 500, 3000, 256
    rowptr, colind, values = random_csr(M, K, 0.01, seed=13, heavy_rows=4, heavy_len=1200, empty_rows=0.2)
    B = np.random.default_rng(13).uniform(-1, 1, (K, N)).astype(np.float32)
    _say("generated", blk, lds, M, K, N)
    plan = Plan(*(torch.from_numpy(a).cuda() for a in (rowptr, colind, values)), M, bh, bw)
    dB = torch.from_numpy(B).cuda()
    for pol, param in (("row", 0), ("split", 3), ("strict_lb", 16), ("multi_bind", 0)):
        plan.set_schedule(pol, param)
        ref = plan.run(dB)
        out = op.run(plan, dB, schedule=pol, schedule_param=param)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), pol
        assert_gate(gate(out.cpu().numpy(), rowptr, colind, values, B, M))
    # "auto" means the same schedule on both paths (the library's rule), so the same bits
    plan.set_schedule("auto", 0)
    ref = plan.run(dB)
    auto = op.run(plan, dB)
    torch.cuda.synchronize()
    assert torch.equal(auto, ref)
    assert_gate(gate(auto.cpu().numpy(), rowptr, colind, values, B, M))
    # both A sources of the operator give the library's bits
    for a_op in ("compact", "dense"):
        for pol, param in (("row", 0), ("split", 3)):
            plan.set_schedule(pol, param)
            ref = plan.run(dB, a_operand=a_op)
            got = op.run(plan, dB, schedule=pol, schedule_param=param, a_operand=a_op)
            torch.cuda.synchronize()
            assert torch.equal(got, ref), (a_op, pol)


def test_generated_operator_rejects_bad_operands(gpu):
    import torch
    from mask_amd.build import GENERATED
    from mask_amd.emitter import GeneratedOperator
    from mask_amd.SRBCRSSpMM import Plan
    op = GeneratedOperator(GENERATED / "sr_bcrs_16x8.so")
    M, K = 40, 60
    rowptr, colind, values = random_csr(M, K, 0.1, seed=2)
    plan = Plan(*(torch.from_numpy(a).cuda() for a in (rowptr, colind, values)), M)
    with pytest.raises(RuntimeError, match="rejected"):
        op.run(plan, torch.ones((K, 64), device="cuda"), schedule="row")   # 64 % 128 != 0
    with pytest.raises(RuntimeError, match="fewer rows"):
        op.run(plan, torch.ones((int(colind.max()), 128), device="cuda"), schedule="row")
    dB = torch.ones((K, 128), device="cuda")
    with pytest.raises(RuntimeError, match="rows, the plan writes"):
        op.run(plan, dB, out=torch.empty((M - 1, 128), device="cuda"), schedule="row")
    with pytest.raises(RuntimeError, match="float32"):
        op.run(plan, dB.double(), schedule="row")
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        op.run(plan, dB.cpu(), schedule="row")
    with pytest.raises(RuntimeError, match="row-major"):
        op.run(plan, torch.ones((128, K), device="cuda").t(), schedule="row")


def test_generated_c_abi_checks_operands(gpu):
    """The generated C entry itself refuses inconsistent operands (status -1,
    nothing launched): a C with fewer rows than M, a wrong offsets length
    (Mo), a half-given compact copy."""
    import torch
    from mask_amd.build import GENERATED
    from mask_amd.emitter import GeneratedOperator
    from mask_amd.SRBCRSSpMM import Plan
    op = GeneratedOperator(GENERATED / "sr_bcrs_16x8.so")
    M, K, N = 40, 60, 128
    rowptr, colind, values = random_csr(M, K, 0.1, seed=2)
    plan = Plan(*(torch.from_numpy(a).cuda() for a in (rowptr, colind, values)), M)
    d = plan.desc
    B = torch.ones((K, N), device="cuda")
    C = torch.empty((M, N), device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    run = op._lib.sparsene_generated_run
    Mo = plan.row_windows + 1
    ok = run(B.data_ptr(), C.data_ptr(), d.d_soff, d.d_val, d.d_sidx, K, M, Mo, N, plan.total_blocks, N, N, M,
             None, None, None, st)
    assert ok == 0
    assert run(B.data_ptr(), C.data_ptr(), d.d_soff, d.d_val, d.d_sidx, K, M, Mo, N, plan.total_blocks, N, N,
               M - 1, None, None, None, st) == -1
    assert run(B.data_ptr(), C.data_ptr(), d.d_soff, d.d_val, d.d_sidx, K, M, Mo + 1, N, plan.total_blocks, N, N,
               M, None, None, None, st) == -1
    assert run(B.data_ptr(), C.data_ptr(), d.d_soff, d.d_val, d.d_sidx, K, M, Mo, N, plan.total_blocks, N, N, M,
               None, d.d_val, None, st) == -1
    torch.cuda.synchronize()
