"""Plan-owned device memory: the split schedules' partial buffer grows
geometrically as N rises, replaced buffers and task tables are retired (not
freed) so earlier captured launches keep valid addresses, and
srbcrs_plan_trim frees them; results stay bit-identical throughout."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import assert_gate, gate, random_csr

pytestmark = pytest.mark.gpu


def test_growth_and_trim(gpu):
    import torch
    from mask_amd.SRBCRSSpMM import Plan
    M, K = 20000, 1500   # split partial tiles of a few hundred MB at N = 512
    rowptr, colind, values = random_csr(M, K, 0.03, seed=9, heavy_rows=3, heavy_len=900)
    plan = Plan(*(torch.from_numpy(a).cuda() for a in (rowptr, colind, values)), M)
    rng = np.random.default_rng(9)
    refs = {}
    print("[case] plan growth", flush=True)
    for pol in (("split", 8), ("strict_lb", 16), ("split", 6)):
        plan.set_schedule(*pol)
        for N in (32, 64, 128, 256, 512):
            B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
            out = plan.run(torch.from_numpy(B).cuda())
            torch.cuda.synchronize()
            refs[(pol, N)] = (B, out.cpu().numpy())
            if N in (32, 512):
                assert_gate(gate(refs[(pol, N)][1], rowptr, colind, values, B, M))
    torch.cuda.synchronize()
    free_before = torch.cuda.mem_get_info()[0]
    plan.trim()
    torch.cuda.synchronize()
    # the retired partial buffers (hundreds of MB) came back to the device
    assert torch.cuda.mem_get_info()[0] > free_before + (64 << 20)
    # the plan still runs every width with the same bits after the trim
    for N in (512, 32, 256):
        B, ref = refs[(("split", 6), N)]
        assert np.array_equal(plan.run(torch.from_numpy(B).cuda()).cpu().numpy(), ref), N
    plan.trim()   # nothing retired: a no-op
