"""MatrixMarket input path (no GPU): the loader against a hand-computed case
and the loop restatement of the reference's mmio_allinone."""
from __future__ import annotations

import gzip

import numpy as np
import pytest

from mask_amd import _capi
from mask_amd.mtx import read_mtx, write_mtx
from oracle import oracle


def _write(tmp_path, text, name="a.mtx"):
    p = tmp_path / name
    p.write_text(text)
    return p


def test_symmetric_hand_case(tmp_path):
    # lower triangle of a 3x3 symmetric matrix, diagonal (2,2) once
    p = _write(tmp_path, "%%MatrixMarket matrix coordinate real symmetric\n% c\n3 3 4\n"
                         "2 1 5.0\n3 1 6.0\n2 2 7.0\n3 2 8.0\n")
    m, n, rp, ci, vv, sym = read_mtx(p)
    assert (m, n, sym) == (3, 3, True)
    # rows filled in file order, mirror right after its source
    assert rp.tolist() == [0, 2, 5, 7]
    assert ci.tolist() == [1, 2, 0, 1, 2, 0, 1]
    assert vv.tolist() == [5.0, 6.0, 5.0, 7.0, 8.0, 6.0, 8.0]


def test_pattern_integer_general(tmp_path):
    p = _write(tmp_path, "%%MatrixMarket matrix coordinate pattern general\n2 4 3\n2 4\n1 3\n2 1\n")
    m, n, rp, ci, vv, sym = read_mtx(p)
    assert (m, n, sym) == (2, 4, False)
    assert rp.tolist() == [0, 1, 3] and ci.tolist() == [2, 3, 0] and vv.tolist() == [1.0, 1.0, 1.0]
    p = _write(tmp_path, "%%MatrixMarket matrix coordinate integer general\n2 2 2\n1 1 3\n2 2 -4\n", "i.mtx")
    assert read_mtx(p)[4].tolist() == [3.0, -4.0]
    with pytest.raises(ValueError, match="banner"):
        read_mtx(_write(tmp_path, "garbage\n1 1 1\n", "g.mtx"))
    with pytest.raises(ValueError, match="out of range"):
        read_mtx(_write(tmp_path, "%%MatrixMarket matrix coordinate real general\n2 2 1\n3 1 1.0\n", "o.mtx"))


@pytest.mark.parametrize("symmetric", [False, True])
def test_loader_matches_loop_restatement(tmp_path, symmetric):
    rng = np.random.default_rng(int(symmetric))
    m = n = 120
    nnz = 600
    r = rng.integers(0, m, nnz)
    c = rng.integers(0, n, nnz)
    if symmetric:
        r, c = np.maximum(r, c), np.minimum(r, c)
    v = rng.standard_normal(nnz)
    p = tmp_path / "r.mtx"
    write_mtx(p, m, n, r, c, v, symmetric=symmetric)
    got = read_mtx(p)
    exp = oracle.read_mtx_loop(p)
    assert got[:2] == exp[:2] and got[5] == exp[5]
    for a, b in zip(got[2:5], exp[2:5]):
        assert a.tobytes() == b.tobytes()
    gz = tmp_path / "r.mtx.gz"
    gz.write_bytes(gzip.compress(p.read_bytes()))
    assert read_mtx(gz)[3].tobytes() == got[3].tobytes()
    # and the loaded CSR converts bit-exactly (unsorted rows, duplicates)
    a = _capi.convert_host(got[2], got[3], got[4], m)
    b = oracle.convert(got[2], got[3], got[4], m)
    assert a["val"].tobytes() == b["val"].tobytes() and np.array_equal(a["sidx"], b["sidx"])
