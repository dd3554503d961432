"""The SpMM run path under HIP graph capture (torch.cuda.CUDAGraph): after
one eager run has sized the plan's buffers, a captured run replays correctly
many times, with eager work and new B values between the replays."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import random_csr

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[case]", *a, flush=True)


@pytest.mark.parametrize("policy", [("row", 0), ("split", 0), ("strict_lb", 5)])
def test_graph_replay_matches_eager(gpu, policy):
    import torch
    from mask_amd.SRBCRSSpMM import Plan
    M, K, N = 613, 700, 128
    rp, ci, vv = random_csr(M, K, 0.02, 41, heavy_rows=3, heavy_len=650, empty_rows=0.1)
    t = lambda a: torch.from_numpy(a).cuda()
    plan = Plan(t(rp), t(ci), t(vv), M)
    plan.set_schedule(*policy)
    rng = np.random.default_rng(7)
    B = t(rng.uniform(-1, 1, (K, N)).astype(np.float32))
    C = torch.empty((M, N), device="cuda")
    _say("graph", policy)
    plan.run(B, C)                      # eager: sizes the partial buffer of split schedules
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            plan.run(B, C)
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(4):
        B.copy_(t(rng.uniform(-1, 1, (K, N)).astype(np.float32)))
        C.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        got = C.clone()
        ref = plan.run(B)               # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (policy, rep)


def test_graph_survives_partial_buffer_growth(gpu):
    """A run that needs a larger partial buffer (wider N, split schedule)
    after a graph was captured grows the buffer without freeing the old one,
    so replays of the earlier graph still write valid memory and stay
    correct; a schedule change keeps the captured task tables alive too."""
    import torch
    from mask_amd.SRBCRSSpMM import Plan
    M, K = 613, 700
    rp, ci, vv = random_csr(M, K, 0.02, 43, heavy_rows=3, heavy_len=650)
    t = lambda a: torch.from_numpy(a).cuda()
    plan = Plan(t(rp), t(ci), t(vv), M)
    plan.set_schedule("split", 3)
    rng = np.random.default_rng(9)
    B = t(rng.uniform(-1, 1, (K, 64)).astype(np.float32))
    C = torch.empty((M, 64), device="cuda")
    _say("graph growth")
    plan.run(B, C)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            plan.run(B, C)
    torch.cuda.current_stream().wait_stream(s)
    ref = plan.run(B).clone()
    wide = plan.run(t(rng.uniform(-1, 1, (K, 512)).astype(np.float32)))   # grows the partial buffer
    plan.set_schedule("strict_lb", 4)                                      # replaces the task tables
    plan.run(t(rng.uniform(-1, 1, (K, 512)).astype(np.float32)))
    torch.cuda.synchronize()
    for _ in range(3):
        C.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(C, ref)
    assert wide.shape == (M, 512)
