"""Pins for the CPU oracle (oracle/srbcrs_oracle.c).

Each check is independent of the oracle's own formulas: hand-computed known
answers, the generic CuTe Swizzle<B,M,S> definition, brute-force dense
re-assembly, numpy dense matmul, and hand-worked partitions.  The reference
ships no golden vectors for this path, so these are the pins.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle
from tests.helpers import dedupe_last, random_csr


# ---- swizzle ----------------------------------------------------------------

def cute_swizzle(offset: int, B: int, M: int, S: int) -> int:
    """CuTe Swizzle<BBits, MBase, SShift> from its documented definition:
    the B bits starting at bit M+max(0,S) (YYY) are XORed into the B bits
    starting at bit M-min(0,S) (ZZZ)."""
    bit_msk = (1 << B) - 1
    yyy = bit_msk << (M + max(0, S))
    return offset ^ ((offset & yyy) >> S if S >= 0 else (offset & yyy) << -S)


def test_swizzle_matches_generic_definition():
    for o in range(2048):
        assert oracle.swizzle(o) == cute_swizzle(o, 2, 2, 3)


def test_swizzle_hand_values_and_bijection():
    # 0b0100000 (row 4 of 16x8) -> bit 5 copied onto bit 2
    assert oracle.swizzle(32) == 36
    assert oracle.swizzle(64) == 72
    assert oracle.swizzle(96) == 108
    assert oracle.swizzle(43) == 47      # row 5, col 3
    assert oracle.swizzle(7) == 7        # rows 0..3 untouched
    for n in (128, 1024):
        img = sorted(oracle.swizzle(o) for o in range(n))
        assert img == list(range(n))
    # only bits 2..3 can change, and (c, c^1) stay adjacent
    for o in range(1024):
        assert (oracle.swizzle(o) ^ o) & ~0b1100 == 0
        if o % 2 == 0:
            assert oracle.swizzle(o + 1) == oracle.swizzle(o) + 1


# ---- conversion: hand-computed known answer ---------------------------------

def _hand_case():
    # 18 rows -> two windows (the second holds rows 16, 17 only)
    rows = {0: [(3, 1.0), (10, 2.0)],
            1: [(10, 3.0), (1, 4.0)],                 # unsorted
            3: [(30 + i, 10.0 + i) for i in range(8)],
            5: [(20, 5.0), (3, 6.0)],
            12: [(1, 7.0)],
            16: [(7, 8.0)],
            17: [(7, 9.0), (7, 11.0)]}               # duplicate: last write wins
    rowptr = [0]
    colind, values = [], []
    for r in range(18):
        for c, v in rows.get(r, []):
            colind.append(c)
            values.append(v)
        rowptr.append(len(colind))
    return np.array(rowptr, np.int32), np.array(colind, np.int32), np.array(values, np.float32)


def test_convert_hand_case():
    rowptr, colind, values = _hand_case()
    out = oracle.convert(rowptr, colind, values, 18)
    # window 0 unique columns: 1 3 10 20 30..37 (12) -> 2 blocks, padded with 37
    assert out["total"] == 3
    assert out["soff"].tolist() == [0, 2, 3]
    assert out["block_partition"].tolist() == [2, 1]
    assert out["sidx"].tolist() == [1, 3, 10, 20, 30, 31, 32, 33,
                                    34, 35, 36, 37, 37, 37, 37, 37,
                                    7, 7, 7, 7, 7, 7, 7, 7]
    val = np.zeros(3 * 128, np.float32)
    # block 0 (offset = 8 r + c, swizzled when r has bit 2 or 3 set)
    val[0 * 128 + 1] = 1.0       # r0 col 3  -> c1
    val[0 * 128 + 2] = 2.0       # r0 col 10 -> c2
    val[0 * 128 + 10] = 3.0      # r1 col 10 -> o 10
    val[0 * 128 + 8] = 4.0       # r1 col 1  -> o 8
    for i in range(4):           # r3 cols 30..33 -> c 4..7, o 28..31
        val[0 * 128 + 28 + i] = 10.0 + i
    val[0 * 128 + 47] = 5.0      # r5 col 20 -> o 43 -> 47
    val[0 * 128 + 45] = 6.0      # r5 col 3  -> o 41 -> 45
    val[0 * 128 + 108] = 7.0     # r12 col 1 -> o 96 -> 108
    for i in range(4):           # block 1: r3 cols 34..37 -> c 0..3, o 24..27
        val[1 * 128 + 24 + i] = 14.0 + i
    val[2 * 128 + 0] = 8.0       # window 1, r0 col 7
    val[2 * 128 + 8] = 11.0      # r1 col 7, last of the two writes
    assert out["val"].tobytes() == val.tobytes()
    assert out["edge_to_row"].tolist() == [0, 0, 1, 1] + [3] * 8 + [5, 5, 12, 16, 17, 17]
    assert out["edge_to_col"].tolist() == [1, 2, 2, 0] + list(range(4, 12)) + [3, 1, 0, 0, 0, 0]


def test_convert_32x32_hand_case():
    # one 32-row window, 33 unique columns -> 2 blocks of 32
    rowptr = np.array([0, 33] + [33] * 30 + [34], np.int32)
    colind = np.array(list(range(100, 133)) + [5], np.int32)
    values = np.arange(1, 35, dtype=np.float32)
    out = oracle.convert(rowptr, colind, values, 32, 32, 32)
    assert out["soff"].tolist() == [0, 2]
    assert out["sidx"].tolist() == [5] + list(range(100, 131)) + [131, 132] + [132] * 30
    val = np.zeros(2 * 1024, np.float32)
    for i in range(31):                  # row 0 cols 100..130 -> c 1..31
        val[1 + i] = 1.0 + i
    val[1024 + 0] = 32.0                 # col 131 -> block 1 c0
    val[1024 + 1] = 33.0                 # col 132 -> c1
    val[oracle.swizzle(31 * 32 + 0)] = 34.0   # row 31 col 5 -> o 992 -> 1004
    assert oracle.swizzle(992) == 1004
    assert out["val"].tobytes() == val.tobytes()


def test_convert_empty_and_partial_windows():
    rowptr = np.zeros(21, np.int32)      # 20 rows, no entries
    out = oracle.convert(rowptr, np.zeros(0, np.int32), np.zeros(0, np.float32), 20)
    assert out["total"] == 0 and out["soff"].tolist() == [0, 0, 0]
    assert out["sidx"].size == 0 and out["val"].size == 0


def _dense_from_csr_lastwins(rowptr, colind, values, M, K):
    A = np.zeros((M, K), np.float32)
    for r in range(M):
        for e in range(rowptr[r], rowptr[r + 1]):
            A[r, colind[e]] = values[e]
    return A


def _dense_from_srbcrs(out, M, K, bh, bw):
    inv = np.argsort([oracle.swizzle(o) for o in range(bh * bw)])   # brute-force inverse
    A = np.zeros((M, K), np.float32)
    soff, sidx, val = out["soff"], out["sidx"], out["val"]
    for w in range(soff.shape[0] - 1):
        for b in range(soff[w], soff[w + 1]):
            blk = val[b * bh * bw:(b + 1) * bh * bw][inv].reshape(bh, bw)
            for r in range(bh):
                row = w * bh + r
                if row >= M:
                    assert not blk[r].any()
                    continue
                for c in range(bw):
                    if blk[r, c] != 0:
                        A[row, sidx[b * bw + c]] = blk[r, c]
    return A


@pytest.mark.parametrize("bh,bw", [(16, 8), (32, 32)])
@pytest.mark.parametrize("seed", range(4))
def test_convert_dense_reassembly(seed, bh, bw):
    M, K = 77 + seed * 13, 150
    rowptr, colind, values = random_csr(M, K, 0.06, seed, unsorted=seed % 2 == 1, duplicates=seed >= 2,
                                        empty_rows=0.2)
    out = oracle.convert(rowptr, colind, values, M, bh, bw)
    A = _dense_from_csr_lastwins(rowptr, colind, values, M, K)
    assert np.array_equal(_dense_from_srbcrs(out, M, K, bh, bw), A)
    # structure invariants
    soff, sidx = out["soff"], out["sidx"]
    assert soff[-1] == out["total"] == sidx.size // bw
    for w in range(soff.size - 1):
        s = sidx[soff[w] * bw:soff[w + 1] * bw]
        rows = range(w * bh, min(M, (w + 1) * bh))
        uniq = sorted({int(colind[e]) for r in rows for e in range(rowptr[r], rowptr[r + 1])})
        assert s[:len(uniq)].tolist() == uniq
        assert (s[len(uniq):] == (uniq[-1] if uniq else 0)).all()
        assert soff[w + 1] - soff[w] == -(-len(uniq) // bw)
    rp, ci, vv = dedupe_last(rowptr, colind, values)
    assert np.count_nonzero(out["val"]) == np.count_nonzero(vv)


# ---- SpMM oracles ------------------------------------------------------------

def test_csr_spmm_f64_matches_dense_matmul():
    M, K, N = 60, 90, 24
    rowptr, colind, values = random_csr(M, K, 0.1, 7, unsorted=True)
    B = np.random.default_rng(1).uniform(-1, 1, (K, N)).astype(np.float32)
    A = np.zeros((M, K), np.float64)
    for r in range(M):
        for e in range(rowptr[r], rowptr[r + 1]):
            A[r, colind[e]] += values[e]
    C, absAB = oracle.csr_spmm_f64(rowptr, colind, values, B, M, with_abs=True)
    np.testing.assert_allclose(C, A @ B.astype(np.float64), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(absAB, np.abs(A) @ np.abs(B.astype(np.float64)), rtol=1e-12, atol=1e-12)


def test_csr_spmm_special_cases():
    M, N = 40, 16
    B = np.random.default_rng(2).uniform(-1, 1, (M, N)).astype(np.float32)
    eye_rp = np.arange(M + 1, dtype=np.int32)
    eye_ci = np.arange(M, dtype=np.int32)
    ones = np.ones(M, np.float32)
    assert np.array_equal(oracle.csr_spmm_f64(eye_rp, eye_ci, ones, B, M), B.astype(np.float64))
    assert np.array_equal(oracle.csr_spmm_f32(eye_rp, eye_ci, ones, B, M), B)
    # B = ones -> row sums of A
    rowptr, colind, values = random_csr(M, M, 0.2, 3)
    C = oracle.csr_spmm_f64(rowptr, colind, values, np.ones((M, 3), np.float32), M)
    sums = np.array([values[rowptr[r]:rowptr[r + 1]].astype(np.float64).sum() for r in range(M)])
    np.testing.assert_allclose(C, np.repeat(sums[:, None], 3, 1), rtol=1e-12, atol=1e-14)


def test_csr_spmm_f32_within_bound():
    M, K, N = 200, 300, 64
    rowptr, colind, values = random_csr(M, K, 0.2, 4)
    B = np.random.default_rng(4).uniform(-1, 1, (K, N)).astype(np.float32)
    C = oracle.csr_spmm_f32(rowptr, colind, values, B, M, nthreads=2)
    C64, absAB = oracle.csr_spmm_f64(rowptr, colind, values, B, M, with_abs=True)
    met = oracle.error_metrics(C, C64, absAB)
    assert met["max_ratio"] < 1e-5 and met["ref_gate"]
    # a dropped term is caught by the gate
    C_bad = C.copy()
    C_bad[5] -= values[rowptr[5]] * B[colind[rowptr[5]]]
    assert oracle.error_metrics(C_bad, C64, absAB)["max_ratio"] > 1e-4


def test_csr_spmm_f32_is_the_unfused_sequential_sum():
    """The fp32 oracle's exact arithmetic, which the nonzero sweep must match
    bit for bit: per row, acc = fl(acc + fl(v * B[c])) in stored order from
    +0, no fused multiply-add.  Restated with numpy float32 elementwise
    operations (each rounded on its own); a fused multiply-add, a different
    order or a pairwise sum would differ in some of these 64 x 48 outputs
    (checked here for the fused form)."""
    M, K, N = 64, 90, 48
    rowptr, colind, values = random_csr(M, K, 0.3, 8)
    B = np.random.default_rng(8).uniform(-1, 1, (K, N)).astype(np.float32)
    want = np.zeros((M, N), np.float32)
    fused = np.zeros((M, N), np.float32)
    for r in range(M):
        acc = np.zeros(N, np.float32)
        accf = np.zeros(N, np.float32)
        for e in range(rowptr[r], rowptr[r + 1]):
            acc = acc + values[e] * B[colind[e]]
            # v * b + acc with the product unrounded (the fused form, up to a float64 rounding)
            accf = (np.float64(values[e]) * B[colind[e]].astype(np.float64) + accf).astype(np.float32)
        want[r], fused[r] = acc, accf
    got = oracle.csr_spmm_f32(rowptr, colind, values, B, M, nthreads=3)
    assert np.array_equal(got, want)
    assert not np.array_equal(got, fused)


# ---- partitions (hand-worked) -------------------------------------------------

def test_strict_lb_hand_case():
    soff = np.cumsum([0, 3, 0, 5, 2]).astype(np.int32)      # lengths 3 0 5 2
    p = oracle.strict_lb(soff, workload=4)
    assert p["frag_begin"].tolist() == [0, 3, 4, 8, 10]
    assert p["frag_window"].tolist() == [0, 2, 2, 3]
    assert p["group_off"].tolist() == [0, 2, 3, 4]
    # exact multiple: no trailing group
    p = oracle.strict_lb(np.array([0, 4, 8], np.int32), workload=4)
    assert p["group_off"].tolist() == [0, 1, 2]
    # empty matrix still yields one (empty) group
    p = oracle.strict_lb(np.array([0, 0, 0], np.int32), workload=4)
    assert p["group_off"].tolist() == [0, 0] and p["frag_begin"].tolist() == [0]


def test_multi_bind_hand_case():
    soff = np.cumsum([0, 1, 10, 1, 0]).astype(np.int32)     # mean 3, window 1 > 6
    p = oracle.multi_bind(soff)
    assert p["part_window"].tolist() == [0, 1, 1, 1, 1, 2]
    assert p["part_off"].tolist() == [0, 1, 4, 7, 9, 11, 12]  # 10 = 3+3+2+2
    assert p["window_split"].tolist() == [0, 1, 0, 0]


def test_segment_auto_hand_cases():
    lens = [2] * 100 + [200]
    soff = np.cumsum([0] + lens).astype(np.int32)
    s = oracle.segment_auto(soff)
    assert s["heavy"] and s["cap"] == 32                    # p95 = 2 -> max(32, min(128, 4))
    assert s["win_seg_off"][-1] - s["win_seg_off"][-2] == 7  # ceil(200 / 32)
    assert s["seg_end"][-1] == 400 and s["seg_end"][-2] == 392
    s = oracle.segment_auto(np.cumsum([0, 3, 5, 0, 2]).astype(np.int32))
    assert not s["heavy"] and s["cap"] == 5
    assert s["seg_end"].tolist() == [3, 8, 8, 10]           # the empty window keeps one segment
    s = oracle.segment_auto(np.cumsum([0, 3, 5, 2]).astype(np.int32), requested=2)
    assert s["cap"] == 2 and s["seg_end"].tolist() == [2, 3, 5, 7, 8, 10]


def _csr_from_rows(rows, m):
    rp, ci, vv = [0], [], []
    for r in range(m):
        for c, v in rows.get(r, []):
            ci.append(c)
            vv.append(v)
        rp.append(len(ci))
    return np.array(rp, np.int32), np.array(ci, np.int32), np.array(vv, np.float32)


def test_first_col_order_hand_case():
    rp, ci, _ = _csr_from_rows({0: [(5, 1.0)], 1: [(7, 1.0), (2, 1.0)], 3: [(2, 1.0)], 4: [(0, 1.0)]}, 5)
    assert oracle.row_order(rp, ci, 5, 9, "first_col_sort").tolist() == [4, 1, 3, 0, 2]


def test_rcm_hand_cases():
    # path 0-1-2-3: start at the lowest-degree, lowest-id end, BFS, reverse
    rp, ci, _ = _csr_from_rows({0: [(1, 1.0)], 1: [(2, 1.0)], 2: [(3, 1.0)]}, 4)
    assert oracle.row_order(rp, ci, 4, 4, "row_rcm").tolist() == [3, 2, 1, 0]
    # star centre 0 with leaves 1..3 and an isolated 4 (degree 0 starts first)
    rp, ci, _ = _csr_from_rows({0: [(1, 1.0), (2, 1.0), (3, 1.0), (0, 1.0)]}, 5)
    assert oracle.row_order(rp, ci, 5, 5, "row_rcm").tolist() == [4, 3, 2, 0, 1]
    with pytest.raises(ValueError, match="square"):
        oracle.row_order(rp, ci, 5, 6, "row_rcm")


def test_rcm_recovers_band_structure():
    """A banded matrix under a random symmetric permutation: RCM brings the
    bandwidth back near the original (a plausible ordering bug would not)."""
    n, bw = 400, 3
    rng = np.random.default_rng(0)
    perm = rng.permutation(n)
    inv = np.argsort(perm)
    rows = {}
    for i in range(n):
        for j in range(max(0, i - bw), min(n, i + bw + 1)):
            rows.setdefault(int(inv[i]), []).append((int(inv[j]), 1.0))
    rp, ci, _ = _csr_from_rows({r: sorted(v) for r, v in rows.items()}, n)
    order = oracle.row_order(rp, ci, n, n, "row_rcm")
    assert sorted(order.tolist()) == list(range(n))
    pos = np.empty(n, np.int64)
    pos[order] = np.arange(n)
    band = max(abs(pos[r] - pos[c]) for r in range(n) for c in ci[rp[r]:rp[r + 1]])
    scrambled = max(abs(r - c) for r in range(n) for c in ci[rp[r]:rp[r + 1]])
    assert band <= 2 * bw and scrambled > 50


def _splitmix64(v):
    M = (1 << 64) - 1
    v = (v + 0x9E3779B97F4A7C15) & M
    v = ((v ^ (v >> 30)) * 0xBF58476D1CE4E5B9) & M
    v = ((v ^ (v >> 27)) * 0x94D049BB133111EB) & M
    return v ^ (v >> 31)


def _jaccard_greedy_py(rp, ci, m, k):
    """Brute-force restatement from the description (minhash buckets of 64,
    greedy nearest Jaccard on column sets, ties to the lower row id)."""
    sets = [list(ci[rp[r]:rp[r + 1]]) for r in range(m)]
    sig = [min((_splitmix64(int(c) & 0xFFFFFFFF) for c in s), default=(1 << 64) - 1) for s in sets]
    first = [min((int(c) for c in s if 0 <= c < k), default=k) for s in sets]
    ranked = sorted(range(m), key=lambda r: (sig[r], first[r], r))
    out = []
    for b in range(0, m, 64):
        bucket = ranked[b:b + 64]
        cur, rem = bucket[0], bucket[1:]
        out.append(cur)
        while rem:
            def jac(a, c):
                A, C = set(sets[a]), set(sets[c])
                return len(A & C) / len(A | C) if (A | C) else 1.0
            best = max(rem, key=lambda c: (jac(cur, c), -c))
            rem.remove(best)
            out.append(best)
            cur = best
    return out


def test_splitmix64_reference_vector():
    # first output of SplitMix64 seeded with 0 (Vigna's reference generator)
    assert _splitmix64(0) == 0xE220A8397B1DCDAF


@pytest.mark.parametrize("seed", range(3))
def test_jaccard_greedy_matches_bruteforce(seed):
    m, k = 150, 60
    rp, ci, _ = random_csr(m, k, 0.08, seed, empty_rows=0.1)     # sorted rows: the merge walk is exact
    assert oracle.row_order(rp, ci, m, k, "jaccard_greedy").tolist() == _jaccard_greedy_py(rp, ci, m, k)


def test_sparse_rows_order():
    rp, ci, _ = _csr_from_rows({1: [(0, 1.0)], 3: [(2, 1.0)]}, 5)
    assert oracle.row_order(rp, ci, 5, 3, "sparse_rows").tolist() == [1, 3]


def test_pack_hand_cases():
    # r0: col 3 twice (summed), r1: col 9; rows reordered [1, 0]
    rp, ci, vv = _csr_from_rows({0: [(3, 1.0), (3, 2.0)], 1: [(9, 4.0)]}, 2)
    p = oracle.pack(rp, ci, vv, 10, [1, 0])
    assert p["soff"].tolist() == [0, 1]
    assert p["sidx"].tolist() == [3, 9, 9, 9, 9, 9, 9, 9]
    val = np.zeros(128, np.float32)
    val[1] = 4.0          # new row 0 (old row 1), condensed col 1
    val[8] = 3.0          # new row 1 (old row 0), condensed col 0, 1 + 2 summed
    assert p["val"].tobytes() == val.tobytes()
    f = oracle.pack(rp, ci, vv, 10, [1, 0], packing=1)
    assert f["sidx"].tolist() == list(range(8)) + [8, 9, 9, 9, 9, 9, 9, 9]   # clamped to k - 1
    val = np.zeros(256, np.float32)
    val[11] = 3.0         # block 0: new row 1, col 3
    val[128 + 1] = 4.0    # block 1: new row 0, col 9 -> local 1
    assert f["val"].tobytes() == val.tobytes()
    with pytest.raises(ValueError, match="out of range"):
        oracle.pack(rp, ci, vv, 9, [0, 1])


def test_pack_identity_equals_canonical_conversion():
    m, k = 97, 300
    rp, ci, vv = random_csr(m, k, 0.05, seed=4, unsorted=True)
    a = oracle.pack(rp, ci, vv, k, np.arange(m))
    b = oracle.convert(rp, ci, vv, m)
    assert np.array_equal(a["soff"], b["soff"]) and np.array_equal(a["sidx"], b["sidx"])
    assert a["val"].tobytes() == b["val"].tobytes()


def test_segment_reduce_matches_numpy():
    rng = np.random.default_rng(0)
    wso = np.array([0, 2, 2, 5], np.int32)
    partial = rng.standard_normal((5, 16, 8)).astype(np.float32)
    out = oracle.segment_reduce(partial, wso, 16, 8)
    exp = np.concatenate([partial[0] + partial[1], np.zeros((16, 8), np.float32),
                          partial[2] + partial[3] + partial[4]])
    assert np.array_equal(out, exp)


def test_integer_protocol_product_matches_f64_oracle():
    """The exact integer product the GPU protocol test compares against equals
    the fp64 oracle's (fp64 is exact at these magnitudes), duplicates
    included, and the protocol's dense values are what the reference writes."""
    from tests.helpers import exact_product, protocol_dense, protocol_values, random_csr
    assert protocol_values(7).tolist() == [1, 2, 3, 4, 5, 1, 2]
    d = protocol_dense(2, 16)
    assert d[0, 0] == np.float32(-1.0) and d[0, 14] == 0.0 and d[1, 0] == np.float32((16 % 29 - 14) / 14.0)
    rowptr, colind, _ = random_csr(70, 90, 0.1, seed=5, unsorted=True, duplicates=True, empty_rows=0.1)
    vals = protocol_values(colind.shape[0])
    B = (14 * protocol_dense(90, 48)).round().astype(np.float32)
    want = exact_product(rowptr, colind, vals, B, 70)
    from tests.helpers import dedupe_last
    rp, ci, vv = dedupe_last(rowptr, colind, vals)
    C64 = oracle.csr_spmm_f64(rp, ci, vv, B, 70)
    assert np.array_equal(np.asarray(C64), want.astype(np.float64))
