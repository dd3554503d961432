"""Seeded random sweep over shapes, strides, schedules, block shapes, A
sources and launch knobs: every case passes the fp64 gate, the compact and
dense A sources agree bit for bit, and nothing outside C[:M, :N] is written
(B and C are strided views into wider buffers)."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import assert_gate, dedupe_last, gate, random_csr

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", range(40))
def test_random_case(gpu, seed):
    import torch
    from mask_amd.SRBCRSSpMM import Plan
    rng = np.random.default_rng(1000 + seed)
    M = int(rng.integers(1, 1500))
    K = int(rng.integers(1, 1500))
    N = 16 * int(rng.integers(1, 33))                     # 16 .. 512
    pad_b, pad_c = int(rng.choice([0, 1, 4, 16])), int(rng.choice([0, 2, 4, 32]))
    blk = [(16, 8), (32, 32)][int(rng.integers(0, 2))]
    policy = [("row", 0), ("split", 0), ("split", 3), ("strict_lb", 0), ("multi_bind", 0), ("auto", 0)][
        int(rng.integers(0, 6))]
    depth = int(rng.choice([0, 2, 4, 8]))
    wg = int(rng.choice([0, 64, 128, 256]))
    order = int(rng.integers(0, 4))
    b_stage = ["registers", "lds"][seed % 2]
    dens = float(rng.choice([0.001, 0.01, 0.05, 0.2]))
    rp, ci, vv = random_csr(M, K, dens, seed=seed, unsorted=bool(seed % 3 == 0), duplicates=bool(seed % 4 == 0),
                            empty_rows=float(rng.choice([0.0, 0.3])), heavy_rows=int(rng.integers(0, 3)),
                            heavy_len=min(K, int(rng.integers(1, 1200))))
    print("[case] sweep", seed, dict(M=M, K=K, N=N, pad_b=pad_b, pad_c=pad_c, blk=blk, policy=policy, depth=depth,
                                     wg=wg, order=order, b_stage=b_stage, dens=dens, nnz=int(rp[-1])), flush=True)
    t = lambda a: torch.from_numpy(a).cuda()
    plan = Plan(t(rp), t(ci), t(vv), M, blk[0], blk[1])
    plan.set_schedule(*policy)
    Bh = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    Bbig = torch.full((K, N + pad_b), 7.0, device="cuda")
    Bbig[:, :N] = t(Bh)
    outs = []
    for a_op in ("compact", "dense"):
        Cbig = torch.full((M + 3, N + pad_c), -3.0, device="cuda")
        C = Cbig[:, :N]
        plan.run(Bbig[:, :N], C, depth=depth, wg_cols=wg, grid_order=order, a_operand=a_op, b_stage=b_stage)
        torch.cuda.synchronize()
        cb = Cbig.cpu().numpy()
        assert (cb[:, N:] == -3.0).all() and (cb[M:, :] == -3.0).all(), "write outside C[:M, :N]"
        outs.append(cb[:M, :N].copy())
    assert outs[0].tobytes() == outs[1].tobytes()
    assert_gate(gate(outs[0], *dedupe_last(rp, ci, vv), Bh, M))
