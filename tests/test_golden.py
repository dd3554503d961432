"""The oracle and the host converter against the hand-derived fixtures of
tests/golden/ (written by tests/golden/make_golden.py, no converter
involved)."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from mask_amd import _capi
from oracle import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    return json.loads((GOLDEN / name).read_text())


def arrays(g):
    return (np.asarray(g["rowptr"], np.int32), np.asarray(g["colind"], np.int32),
            np.asarray(g["values"], np.float32))


def assert_matches(out, g):
    assert int(out["total"]) == g["total"]
    for k in ("soff", "sidx", "block_partition", "edge_to_row", "edge_to_col"):
        assert np.asarray(out[k]).tolist() == g[k], k
    assert np.asarray(out["val"], np.float32).tobytes() == np.asarray(g["val"], np.float32).tobytes()


@pytest.mark.parametrize("name", ["convert_16x8_hand.json", "convert_32x32_hand.json"])
def test_oracle_and_host_converter_match_golden(name):
    g = load(name)
    rp, ci, vv = arrays(g)
    bh, bw = g["blk"]
    assert_matches(oracle.convert(rp, ci, vv, g["num_nodes"], bh, bw), g)
    assert_matches(_capi.convert_host(rp, ci, vv, g["num_nodes"], bh, bw), g)


def test_oracle_spmm_matches_exact_golden():
    g = load("spmm_exact.json")
    rp, ci, vv = arrays(g)
    B = np.asarray(g["B"], np.float32)
    C64 = oracle.csr_spmm_f64(rp, ci, vv, B, g["num_nodes"])
    assert np.array_equal(C64, np.asarray(g["C"], np.float64))
    C32 = oracle.csr_spmm_f32(rp, ci, vv, B, g["num_nodes"])
    assert np.array_equal(C32, np.asarray(g["C"], np.float32))
