"""Property-based parity of the host converter and the schedules against the
oracle restatement (hypothesis drives the shapes; no GPU)."""
from __future__ import annotations

import numpy as np
import pytest

hypothesis = pytest.importorskip("hypothesis")
from hypothesis import HealthCheck, given, settings, strategies as st  # noqa: E402

from mask_amd import _capi  # noqa: E402
from oracle import oracle  # noqa: E402


@st.composite
def csr(draw):
    M = draw(st.integers(1, 70))
    K = draw(st.integers(1, 90))
    nnz = draw(st.integers(0, min(400, 4 * M * K)))
    rows = np.sort(np.asarray(draw(st.lists(st.integers(0, M - 1), min_size=nnz, max_size=nnz)), np.int64))
    cols = np.asarray(draw(st.lists(st.integers(0, K - 1), min_size=nnz, max_size=nnz)), np.int32)
    vals = np.asarray(draw(st.lists(st.floats(-4, 4, width=32, allow_subnormal=False), min_size=nnz,
                                    max_size=nnz)), np.float32)
    rowptr = np.zeros(M + 1, np.int32)
    np.add.at(rowptr, rows + 1, 1)
    return np.cumsum(rowptr).astype(np.int32), cols, vals, M   # rows keep the drawn (unsorted) column order


@settings(max_examples=120, deadline=None, suppress_health_check=[HealthCheck.too_slow])
@given(csr(), st.sampled_from([(16, 8), (32, 32)]))
def test_host_converter_equals_oracle(a, blk):
    rowptr, colind, values, M = a
    h = _capi.convert_host(rowptr, colind, values, M, *blk)
    o = oracle.convert(rowptr, colind, values, M, *blk)
    assert h["total"] == o["total"]
    for k in ("soff", "sidx", "block_partition", "edge_to_row", "edge_to_col"):
        assert np.array_equal(h[k], o[k]), k
    assert h["val"].tobytes() == o["val"].tobytes()


@st.composite
def soffs(draw):
    lens = draw(st.lists(st.integers(0, 300), min_size=1, max_size=60))
    return np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)


def _cover(s, soff):
    """Every block of every window is covered exactly once, in window order."""
    seen = np.zeros(int(soff[-1]), np.int32)
    for b, e, w in zip(s["task_begin"], s["task_end"], s["task_window"]):
        assert soff[w] <= b <= e <= soff[w + 1]
        seen[b:e] += 1
    assert (seen == 1).all()


@settings(max_examples=150, deadline=None)
@given(soffs(), st.sampled_from(["row", "split", "strict_lb", "multi_bind", "auto"]), st.integers(0, 40))
def test_schedules_cover_every_block_once(soff, policy, param):
    s = _capi.build_schedule(soff, policy, param)
    _cover(s, soff)
    # a window with several tasks reduces through slots; a single-task window stores directly
    per_win = np.bincount(s["task_window"], minlength=soff.size - 1) if s["task_window"].size else np.zeros(0)
    multi = set(np.nonzero(per_win > 1)[0].tolist())
    assert set(s["red_window"].tolist()) >= multi
