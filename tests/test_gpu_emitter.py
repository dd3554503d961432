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
    # the operator's own default ("auto") schedule
    auto = op.run(plan, dB)
    assert_gate(gate(auto.cpu().numpy(), rowptr, colind, values, B, M))


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
