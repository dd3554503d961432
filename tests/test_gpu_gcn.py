"""GCN drop-in on the GPU: srbcrs_spmm variants, autograd forward/backward
through the replaceable SpMM, and the two-layer forward of the GCN workload."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle
from tests.helpers import assert_gate, gate, random_csr

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[case]", *a, flush=True)


@pytest.mark.parametrize("variant", ["base", "16x8", "strict_lb", "multi_binding", "16x8_strict_lb",
                                     "16x8_multi_binding"])
@pytest.mark.parametrize("N", [40, 64, 256])
def test_srbcrs_spmm_variants(gpu, monkeypatch, variant, N):
    import torch
    from mask_amd import external_backend_spmm as E
    monkeypatch.setenv("SPARSENE_SRBCRS_VARIANT", variant)
    monkeypatch.delenv("SPARSENE_ALLOW_CSR_FALLBACK", raising=False)
    E.reset_backend_state()
    M = 230
    rowptr, colind, values = random_csr(M, M, 0.03, seed=N, heavy_rows=3, heavy_len=200, empty_rows=0.1)
    B = np.random.default_rng(N).uniform(-1, 1, (M, N)).astype(np.float32)
    _say("srbcrs_spmm", variant, M, N)
    t = lambda a: torch.from_numpy(a).cuda()
    out = E.srbcrs_spmm(t(rowptr).long(), t(colind).long(), t(values), t(B), M, N, M)
    torch.cuda.synchronize()
    assert out.shape == (M, N)            # N = 40 is padded to 48 and unpadded
    assert_gate(gate(out.cpu().numpy(), rowptr, colind, values, B, M))


def _dense_graph(m):
    A = np.zeros((m.M, m.K), np.float64)
    for r in range(m.M):
        for e in range(m.rowptr[r], m.rowptr[r + 1]):
            A[r, m.colind[e]] += m.values[e]
    return A


def test_gcn_forward_backward_matches_fp64(gpu, monkeypatch):
    """A three-layer GCN with the SR-BCRS SpMM: loss and weight gradients match
    a dense fp64 autograd reference (backward runs A^T through the SpMM)."""
    import torch
    from mask_amd import datasets, external_backend_spmm as E
    from mask_amd.gcn import GCN, graph_from_csr
    monkeypatch.setenv("SPARSENE_SRBCRS_VARIANT", "16x8")
    E.reset_backend_state()
    m = datasets.gcn_graph(n=3000, avg_degree=12, N=64)
    _say("gcn autograd", m.M, m.nnz)
    dev = torch.device("cuda", 0)
    data = graph_from_csr(m, 48, dev, seed=3)
    model = GCN((48, 64, 64, 16), dropout=0.0, spmm=E.srbcrs_spmm, seed=0).to(dev)
    y = torch.randint(0, 16, (m.M,), device=dev)
    loss = F_nll(model(data), y)
    loss.backward()
    grads = [p.grad.double().cpu() for p in model.parameters()]

    # fp64 dense reference with the same weights
    A = torch.from_numpy(_dense_graph(m))
    ws = [p.detach().double().cpu().clone().requires_grad_(True) for p in model.parameters()]
    x = data.x.double().cpu()
    h = x
    for i, w in enumerate(ws):
        h = A @ (h @ w)
        if i < len(ws) - 1:
            h = torch.relu(h)
    ref_loss = torch.nn.functional.nll_loss(torch.log_softmax(h, 1), y.cpu())
    ref_loss.backward()
    assert abs(float(loss) - float(ref_loss)) <= 1e-5 * max(1.0, abs(float(ref_loss)))
    for g, w in zip(grads, ws):
        err = (g - w.grad).abs().max().item()
        scale = w.grad.abs().max().item()
        assert err <= 1e-4 * scale + 1e-7, (err, scale)


def F_nll(logp, y):
    import torch
    return torch.nn.functional.nll_loss(logp, y)


def test_gcn2_forward_workload(gpu, monkeypatch):
    """The GCN workload's two-layer forward (SpMM at N=256 and N=64) on a
    scaled graph: each SpMM within the gate against the fp64 oracle."""
    import torch
    from mask_amd import datasets, external_backend_spmm as E
    from mask_amd.gcn import gcn2_forward, glorot_weights, graph_from_csr
    monkeypatch.setenv("SPARSENE_SRBCRS_VARIANT", "16x8")
    E.reset_backend_state()
    m = datasets.make_config("gcn-232965", scale_down=16)
    _say("gcn2", m.M, m.nnz)
    dev = torch.device("cuda", 0)
    data = graph_from_csr(m, 512, dev, seed=1)
    w1, w2 = glorot_weights([512, 256, 64], seed=2, device=dev)
    spmm = lambda d: E.srbcrs_spmm(*data.a, d.contiguous(), m.M, d.shape[1], m.M)
    out = gcn2_forward(data, w1, w2, E.srbcrs_spmm)
    torch.cuda.synchronize()
    # layer by layer against the oracle on the same fp32 dense inputs
    xw = (data.x @ w1).cpu().numpy()
    h_ref, habs = oracle.csr_spmm_f64(m.rowptr, m.colind, m.values, xw, m.M, with_abs=True)
    h = torch.relu(spmm(data.x @ w1))
    met = oracle.error_metrics(h.cpu().numpy(), np.maximum(h_ref, 0), habs)
    assert met["max_ratio"] <= 1e-4 and met["ref_gate"], met
    hw = (h @ w2).cpu().numpy()
    o_ref, oabs = oracle.csr_spmm_f64(m.rowptr, m.colind, m.values, hw, m.M, with_abs=True)
    met2 = oracle.error_metrics(out.cpu().numpy(), o_ref, oabs)
    assert met2["max_ratio"] <= 1e-4 and met2["ref_gate"], met2


def test_fallback_env_uses_native_csr_kernel(gpu, monkeypatch):
    """SPARSENE_ALLOW_CSR_FALLBACK=1 + a run failure (no blocks) lands on the
    native CSR HIP kernel, never on a CPU path; without the flag it raises."""
    import torch
    from mask_amd import external_backend_spmm as E
    M = 40
    rowptr = np.zeros(M + 1, np.int32)
    colind = np.zeros(0, np.int32)
    values = np.zeros(0, np.float32)
    B = np.ones((M, 64), np.float32)
    t = lambda a: torch.from_numpy(a).cuda()
    monkeypatch.setenv("SPARSENE_SRBCRS_VARIANT", "16x8")
    monkeypatch.delenv("SPARSENE_ALLOW_CSR_FALLBACK", raising=False)
    E.reset_backend_state()
    with pytest.raises(RuntimeError, match="CSR fallback is disabled"):
        E.srbcrs_spmm(t(rowptr), t(colind), t(values), t(B), M, 64, M)
    monkeypatch.setenv("SPARSENE_ALLOW_CSR_FALLBACK", "1")
    E.reset_backend_state()
    out = E.srbcrs_spmm(t(rowptr), t(colind), t(values), t(B), M, 64, M)
    assert out.is_cuda and torch.count_nonzero(out).item() == 0
