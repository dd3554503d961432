"""Row sharding on one GPU: per-shard plans over row-sliced CSRs reproduce
the full plan's C bit for bit (row schedule and a fixed split cap, which
cut every window the same way in both), for 16x8 and 32x32 blocks."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import random_csr

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("blk", [(16, 8), (32, 32)])
@pytest.mark.parametrize("n_shards", [2, 3, 8])
def test_row_shards_bitwise_equal_full(gpu, blk, n_shards):
    import torch
    from mask_amd.SRBCRSSpMM import Plan
    from mask_amd.sharding import RowShardedSpMM
    M, K, N = 1237, 900, 128
    rp, ci, vv = random_csr(M, K, 0.02, seed=n_shards, heavy_rows=4, heavy_len=800, empty_rows=0.2)
    t = lambda a: torch.from_numpy(a).cuda()
    B = t(np.random.default_rng(5).uniform(-1, 1, (K, N)).astype(np.float32))
    full = Plan(t(rp), t(ci), t(vv), M, *blk)
    sh = RowShardedSpMM(t(rp), t(ci), t(vv), M, n_shards, *blk)
    assert sh.ranges[0][0] == 0 and sh.ranges[-1][1] == M
    assert all(a[1] == b[0] for a, b in zip(sh.ranges, sh.ranges[1:]))
    for pol in (("row", 0), ("split", 8)):
        print("[case] shards", blk, n_shards, pol, sh.ranges, flush=True)
        full.set_schedule(*pol)
        sh.set_schedule(*pol)
        ref = full.run(B)
        got = sh.run(B, torch.full_like(ref, float("nan")))
        torch.cuda.synchronize()
        assert torch.equal(got, ref), pol
