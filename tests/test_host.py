"""Host-side parity (no GPU): the C-ABI library's converter and schedules
against the oracle, its exports against include/srbcrs.h, error paths, and
the Python drop-in module's argument checks."""
from __future__ import annotations

import ctypes
import os
import re
from pathlib import Path

import numpy as np
import pytest

from mask_amd import _capi, datasets
from oracle import oracle
from tests.helpers import random_csr

ROOT = Path(__file__).resolve().parent.parent


def _header_functions():
    text = (ROOT / "include" / "srbcrs.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(srbcrs_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    names = _header_functions()
    assert len(names) >= 15
    assert sorted(_capi.EXPORTS) == names
    L = _capi.lib()
    for n in names:
        assert hasattr(L, n), n
    assert b"gfx950" in L.srbcrs_version()


def test_loader_refuses_experiment_builds(tmp_path):
    """A decomposition build (results wrong on purpose) carries
    "+experiment:<name>" in srbcrs_version(); the product loader refuses it
    unless MASK_AMD_ALLOW_EXPERIMENT=1.  Built here as a stamped C-ABI object
    linked with the product's other objects."""
    import shutil
    import subprocess
    import sys
    from mask_amd import build as B
    objs = [B.PKG / "_build" / (s.rsplit(".", 1)[0] + ".o") for s in B.SOURCES if s != "srbcrs_capi.cpp"]
    if not all(o.exists() for o in objs) or not shutil.which(B._hipcc()):
        pytest.skip("library objects not built")
    capi = tmp_path / "capi_stamped.o"
    B._run([B._hipcc(), *B.DEVICE_FLAGS, "-DSRBCRS_EXPERIMENT_TAG=loader_check", f"-I{ROOT / 'include'}", "-x", "hip",
            "-c", str(B.CSRC / "srbcrs_capi.cpp"), "-o", str(capi)])
    lib = tmp_path / "libmask_srbcrs_loader_check.so"
    B._run([B._hipcc(), f"--offload-arch={B.ARCH}", "-shared", "-fPIC", "-o", str(lib), str(capi), *map(str, objs),
            "-lpthread"])
    code = "from mask_amd import _capi; print(_capi.lib().srbcrs_version().decode())"
    env = dict(os.environ, MASK_AMD_SRBCRS_LIB=str(lib))
    env.pop("MASK_AMD_ALLOW_EXPERIMENT", None)
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True, text=True)
    assert r.returncode != 0 and "decomposition build" in r.stderr, r.stderr[-500:]
    env["MASK_AMD_ALLOW_EXPERIMENT"] = "1"
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True, text=True)
    assert r.returncode == 0 and "+experiment:loader_check" in r.stdout, r.stderr[-500:]
    assert "+experiment:" not in _capi.lib().srbcrs_version().decode()


def test_probe_entry_points_stay_out_of_the_public_abi():
    """The measurement probes are exported by the library (bench.py binds
    them) but declared only in the internal header, not in include/srbcrs.h."""
    import bench
    public = _header_functions()
    L = _capi.lib()
    for name in bench.PROBE_SIGS:
        assert name not in public and hasattr(L, name), name
    internal = (ROOT / "mask_amd" / "csrc" / "srbcrs_probe.h").read_text()
    assert all(name in internal for name in bench.PROBE_SIGS)


def _same(a, b):
    for k in ("soff", "sidx", "block_partition", "edge_to_row", "edge_to_col"):
        assert np.array_equal(a[k], b[k]), k
    assert a["total"] == b["total"]
    assert a["val"].tobytes() == b["val"].tobytes()


@pytest.mark.parametrize("bh,bw", [(16, 8), (32, 32)])
@pytest.mark.parametrize("case", range(6))
def test_converter_matches_oracle(case, bh, bw):
    M = [1, 15, 16, 17, 250, 1000][case]
    K = [1, 40, 300, 9, 700, 5000][case]
    rowptr, colind, values = random_csr(M, K, min(0.5, 3.0 / K + 0.02), seed=case, unsorted=case % 2 == 0,
                                        duplicates=case >= 3, empty_rows=0.25, heavy_rows=2 if M > 100 else 0,
                                        heavy_len=min(K, 600))
    _same(_capi.convert_host(rowptr, colind, values, M, bh, bw), oracle.convert(rowptr, colind, values, M, bh, bw))


@pytest.mark.parametrize("name", ["uniform-4096", "uniform-65536", "banded-524288", "rmat-2^20", "gcn-232965"])
def test_converter_matches_oracle_on_workloads(name):
    m = datasets.make_config(name, scale_down=1 if name == "uniform-4096" else 32)
    _same(_capi.convert_host(m.rowptr, m.colind, m.values, m.M), oracle.convert(m.rowptr, m.colind, m.values, m.M))


def test_converter_full_size_uniform_65536():
    """The metric's workload at full size, bit-exact (1M nonzeros)."""
    m = datasets.make_config("uniform-65536")
    _same(_capi.convert_host(m.rowptr, m.colind, m.values, m.M), oracle.convert(m.rowptr, m.colind, m.values, m.M))


def test_converter_rejects_bad_input():
    rowptr = np.array([0, 2, 1], np.int32)
    with pytest.raises(_capi.SrbcrsError, match="non-decreasing") as e:
        _capi.convert_host(rowptr, np.array([0, 1], np.int32), np.ones(2, np.float32), 2)
    assert e.value.code == _capi.SRBCRS_EINVAL
    with pytest.raises(_capi.SrbcrsError, match="negative"):
        _capi.convert_host(np.array([0, 1], np.int32), np.array([-3], np.int32), np.ones(1, np.float32), 1)
    with pytest.raises(_capi.SrbcrsError, match="16x8 or 32x32"):
        _capi.convert_host(np.array([0, 1], np.int32), np.array([0], np.int32), np.ones(1, np.float32), 1, 16, 16)
    with pytest.raises(_capi.SrbcrsError, match="exceeds colind length"):
        _capi.convert_host(np.array([0, 5], np.int32), np.array([0], np.int32), np.ones(1, np.float32), 1)
    with pytest.raises(_capi.SrbcrsError, match="num_nodes"):
        _capi.convert_host(np.array([0], np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32), 0)


# ---- schedules ------------------------------------------------------------------

def _soff_cases():
    rng = np.random.default_rng(0)
    yield np.array([0], np.int32)
    yield np.cumsum([0, 3, 0, 5, 2]).astype(np.int32)
    yield np.cumsum([0, 1, 10, 1, 0]).astype(np.int32)
    yield np.cumsum([0] + [2] * 100 + [200]).astype(np.int32)
    for _ in range(4):
        lens = rng.zipf(1.6, size=rng.integers(1, 400)).clip(0, 3000)
        lens[rng.random(lens.size) < 0.2] = 0
        yield np.cumsum(np.concatenate([[0], lens])).astype(np.int32)


def _check_cover(s, soff):
    """Every block is in exactly one task of its window; every window is
    written exactly once (one direct task, or a reduce entry)."""
    Mo = soff.size - 1
    tb, te, tw, ts = s["task_begin"], s["task_end"], s["task_window"], s["task_slot"]
    covered = np.zeros(int(soff[-1]), np.int32)
    for b, e, w in zip(tb, te, tw):
        assert soff[w] <= b <= e <= soff[w + 1]
        covered[b:e] += 1
    assert (covered == 1).all()
    assert s["group_off"][0] == 0 and s["group_off"][-1] == tb.size
    assert (np.diff(s["group_off"]) >= 0).all()
    writes = np.zeros(Mo, np.int32)
    for w, sl in zip(tw, ts):
        if sl < 0:
            writes[w] += 1
    slots_seen = []
    for i, w in enumerate(s["red_window"]):
        writes[w] += 1
        lo, hi = s["red_slot_off"][i], s["red_slot_off"][i + 1]
        slots_seen += list(range(lo, hi))
        # the reduce sums this window's task slots, in task order
        assert [int(x) for x in ts[(tw == w) & (ts >= 0)]] == list(range(lo, hi))
    assert (writes == 1).all()
    assert sorted(slots_seen) == list(range(s["n_slots"]))


@pytest.mark.parametrize("workload", [0, 4, 64])
def test_strict_lb_matches_oracle(workload):
    for soff in _soff_cases():
        s = _capi.build_schedule(soff, "strict_lb", workload)
        o = oracle.strict_lb(soff, workload or 64)
        assert s["task_begin"].tolist() == o["frag_begin"][:-1].tolist()
        assert s["task_end"].tolist() == o["frag_begin"][1:].tolist()
        assert s["task_window"].tolist() == o["frag_window"].tolist()
        assert s["group_off"].tolist() == o["group_off"].tolist()
        _check_cover(s, soff)


def test_multi_bind_matches_oracle():
    for soff in _soff_cases():
        s = _capi.build_schedule(soff, "multi_bind")
        o = oracle.multi_bind(soff)
        assert s["task_window"].tolist() == o["part_window"].tolist()
        assert s["task_begin"].tolist() == o["part_off"][:-1].tolist()
        assert s["task_end"].tolist() == o["part_off"][1:].tolist()
        assert s["group_off"].tolist() == list(range(o["part_window"].size + 1))
        _check_cover(s, soff)


@pytest.mark.parametrize("cap", [0, 1, 3, 32])
def test_split_matches_oracle(cap):
    for soff in _soff_cases():
        s = _capi.build_schedule(soff, "split", cap)
        o = oracle.segment_auto(soff, cap)
        assert s["task_end"].tolist() == o["seg_end"].tolist()
        wso = o["win_seg_off"]
        assert s["task_window"].tolist() == np.repeat(np.arange(soff.size - 1), np.diff(wso)).tolist()
        _check_cover(s, soff)


def test_row_schedule_and_errors():
    soff = np.cumsum([0, 3, 0, 5]).astype(np.int32)
    s = _capi.build_schedule(soff, "row")
    assert s["task_begin"].tolist() == [0, 3, 3] and s["task_end"].tolist() == [3, 3, 8]
    assert (s["task_slot"] == -1).all() and s["n_slots"] == 0 and s["red_window"].size == 0
    with pytest.raises(_capi.SrbcrsError, match="unknown schedule policy"):
        _capi.build_schedule(soff, "bogus")
    with pytest.raises(_capi.SrbcrsError, match="non-decreasing"):
        _capi.build_schedule(np.array([0, 5, 2], np.int32), "row")


def test_auto_schedule_picks_split_on_heavy_tail_else_row():
    """"auto" = the split rule's heavy-tail test: longest window > max(64,
    4 x p95) -> the split:0 tables; otherwise the row tables."""
    flat = np.cumsum([0] + [5] * 40 + [60]).astype(np.int32)          # longest 60 <= 64
    assert _same_tables(_capi.build_schedule(flat, "auto")) == _same_tables(_capi.build_schedule(flat, "row"))
    heavy = np.cumsum([0] + [5] * 40 + [300]).astype(np.int32)        # 300 > max(64, 20)
    a, b = _capi.build_schedule(heavy, "auto"), _capi.build_schedule(heavy, "split")
    assert _same_tables(a) == _same_tables(b) and a["n_slots"] > 0
    ratio = np.cumsum([0] + [20] * 40 + [79]).astype(np.int32)         # 79 <= 4 x 20
    assert _same_tables(_capi.build_schedule(ratio, "auto")) == _same_tables(_capi.build_schedule(ratio, "row"))


def _same_tables(s):
    return {k: (v.tolist() if isinstance(v, np.ndarray) else v) for k, v in s.items()}


# ---- drop-in module argument checks (no GPU needed to reach them) ------------------

def test_dropin_rejects_host_tensors():
    torch = pytest.importorskip("torch")
    from mask_amd import SRBCRSSpMM as S
    t = torch.zeros(4, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="colind must be a CUDA tensor"):
        S.preprocess_gpu_16x8(t, t, t.float(), 3, 16, 8, t, t, t)
    with pytest.raises(RuntimeError, match="dense must be a CUDA tensor"):
        S.run_SRBCRS_16x8(t.float().reshape(2, 2), t, t, t, t, 3, 4, "")


def test_tile_b_selection(monkeypatch):
    from mask_amd import SRBCRSSpMM as S
    monkeypatch.delenv("SRBCRS_TILE_B", raising=False)
    assert S._tile_b_for(512) == 64 and S._tile_b_for(96) == 32 and S._tile_b_for(48) == 16
    assert S._tile_b_for(40) == 0
    monkeypatch.setenv("SRBCRS_TILE_B", "32")
    assert S._tile_b_for(64) == 32
    with pytest.raises(RuntimeError, match="SRBCRS_TILE_B=32 requires"):
        S._tile_b_for(48)
    monkeypatch.setenv("SRBCRS_TILE_B", "8")
    with pytest.raises(RuntimeError, match="Invalid SRBCRS_TILE_B=8"):
        S._tile_b_for(64)


def test_exeplan_schedule_parsing(monkeypatch):
    from mask_amd import SRBCRSSpMM as S
    monkeypatch.delenv("SPARSENE_SRBCRS_SCHEDULE", raising=False)
    assert S._schedule_from_exeplan("") is None
    assert S._schedule_from_exeplan("whatever") is None
    assert S._schedule_from_exeplan("strict_lb:32") == ("strict_lb", 32)
    monkeypatch.setenv("SPARSENE_SRBCRS_SCHEDULE", "split")
    assert S._schedule_from_exeplan("") == ("split", 0)


# ---- GCN bridge host logic ------------------------------------------------------------

def test_select_tile_b_and_padding(monkeypatch):
    torch = pytest.importorskip("torch")
    from mask_amd import external_backend_spmm as E
    monkeypatch.delenv("SPARSENE_SRBCRS_TILE_B", raising=False)
    # least padding, ties to the larger tile (external_backend_spmm.py:72-84)
    assert E._select_tile_b(512, "SPARSENE_SRBCRS_TILE_B") == 64
    assert E._select_tile_b(40, "SPARSENE_SRBCRS_TILE_B") == 16    # 48 vs 64
    assert E._select_tile_b(96, "SPARSENE_SRBCRS_TILE_B") == 32
    assert E._select_tile_b(100, "SPARSENE_SRBCRS_TILE_B") == 16   # 112 vs 128
    monkeypatch.setenv("SPARSENE_SRBCRS_TILE_B", "64")
    assert E._select_tile_b(40, "SPARSENE_SRBCRS_TILE_B") == 64
    monkeypatch.setenv("SPARSENE_SRBCRS_TILE_B", "junk")
    assert E._select_tile_b(40, "SPARSENE_SRBCRS_TILE_B") == 16
    d = torch.arange(12, dtype=torch.float32).reshape(3, 4)
    p, cols = E._pad_dense_to_tile(d, 16)
    assert cols == 4 and p.shape == (3, 16) and torch.equal(p[:, :4], d) and not p[:, 4:].any()


def test_variant_normalisation():
    from mask_amd import external_backend_spmm as E
    n = E.canonical_variant
    assert n("") == "base" and n("SR_BCRS") == "base" and n("default") == "base"
    assert n("sr_bcrs_16x8") == "16x8" and n("16_8") == "16x8"
    assert n("multibind_16x8") == "16x8_multi_binding" and n("16x8_multi_bind") == "16x8_multi_binding"
    assert n("srbcrs_16x8_strict_lb") == "16x8_strict_lb" and n("strictlb_16x8") == "16x8_strict_lb"
    assert n("strict-lb") == "strict_lb" and n("multi-binding") == "multi_binding"
    assert n("nonsense") == "nonsense"
    assert E.VARIANTS["16x8_strict_lb"] == ((16, 8), ("strict_lb", 0))
    assert E.SRBCRSBackend("base").spec.block == (32, 32)
    assert E.SRBCRSBackend("nonsense").spec == E.VARIANTS["base"]


def test_csr_transpose_matches_dense():
    from mask_amd.gcn import csr_transpose
    M, K = 50, 70
    rowptr, colind, values = random_csr(M, K, 0.1, seed=2)
    A = np.zeros((M, K), np.float32)
    for r in range(M):
        A[r, colind[rowptr[r]:rowptr[r + 1]]] = values[rowptr[r]:rowptr[r + 1]]
    trp, tci, tv = csr_transpose(rowptr, colind, values, K)
    At = np.zeros((K, M), np.float32)
    for r in range(K):
        assert (np.diff(tci[trp[r]:trp[r + 1]]) > 0).all()
        At[r, tci[trp[r]:trp[r + 1]]] = tv[trp[r]:trp[r + 1]]
    assert np.array_equal(At, A.T)


# ---- row orders and generated-operator packings (library vs oracle) --------------

_ORDER_CASES = [
    dict(m=300, k=300, density=0.02, seed=1),
    dict(m=257, k=257, density=0.05, seed=2, unsorted=True, duplicates=True, empty_rows=0.2),
    dict(m=1000, k=1000, density=0.004, seed=3, empty_rows=0.3, heavy_rows=3, heavy_len=300),
]


@pytest.mark.parametrize("method", ["row_rcm", "first_col_sort", "jaccard_greedy", "sparse_rows", "identity"])
@pytest.mark.parametrize("case", range(len(_ORDER_CASES)))
def test_row_orders_match_oracle(method, case):
    c = dict(_ORDER_CASES[case])
    m, k = c.pop("m"), c.pop("k")
    rp, ci, _ = random_csr(m, k, c.pop("density"), c.pop("seed"), **c)
    assert np.array_equal(_capi.row_order_host(rp, ci, m, k, method), oracle.row_order(rp, ci, m, k, method))


def test_row_orders_on_workload_graph():
    m = datasets.gcn_graph(n=4000, avg_degree=10)
    for method in ("row_rcm", "first_col_sort", "jaccard_greedy"):
        assert np.array_equal(_capi.row_order_host(m.rowptr, m.colind, m.M, m.K, method),
                              oracle.row_order(m.rowptr, m.colind, m.M, m.K, method)), method


@pytest.mark.parametrize("packing", ["column_condensed_dense", "active_fixed_blocks_dense"])
@pytest.mark.parametrize("blk", [(16, 8), (32, 32)])
@pytest.mark.parametrize("order_kind", ["identity", "row_rcm", "sparse_rows"])
def test_packing_matches_oracle(packing, blk, order_kind):
    m = k = 333
    rp, ci, vv = random_csr(m, k, 0.03, seed=7, unsorted=True, duplicates=True, empty_rows=0.25)
    order = oracle.row_order(rp, ci, m, k, order_kind)
    a = _capi.pack_host(rp, ci, vv, m, k, order=None if order_kind == "identity" else order, blk_h=blk[0],
                        blk_w=blk[1], packing=packing, dup="sum")
    b = oracle.pack(rp, ci, vv, k, order, blk[0], blk[1], packing=0 if packing.startswith("column") else 1)
    assert np.array_equal(a["soff"], b["soff"]) and np.array_equal(a["sidx"], b["sidx"])
    assert a["val"].tobytes() == b["val"].tobytes()


def test_packing_last_write_equals_canonical_conversion():
    m, k = 200, 500
    rp, ci, vv = random_csr(m, k, 0.04, seed=9, unsorted=True, duplicates=True)
    a = _capi.pack_host(rp, ci, vv, m, k, dup="last")
    b = oracle.convert(rp, ci, vv, m)
    assert np.array_equal(a["soff"], b["soff"]) and np.array_equal(a["sidx"], b["sidx"])
    assert a["val"].tobytes() == b["val"].tobytes()


def test_packing_rejects_bad_options():
    rp, ci, vv = random_csr(20, 30, 0.2, seed=1)
    with pytest.raises(_capi.SrbcrsError, match="distinct rows"):
        _capi.pack_host(rp, ci, vv, 20, 30, order=[0, 0, 1])
    with pytest.raises(_capi.SrbcrsError, match="out of range"):
        _capi.pack_host(rp, ci, vv, 20, 5)
    with pytest.raises(_capi.SrbcrsError, match="square"):
        _capi.row_order_host(rp, ci, 20, 30, "row_rcm")


def test_header_is_c99_and_c_client_builds(tmp_path):
    """include/srbcrs.h compiles as C99 (no C++ in the ABI) and a plain C
    client links against the library."""
    import subprocess
    from tests.c_client import ROOT, compile_client
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-fsyntax-only", "-x", "c",
                    str(ROOT / "include" / "srbcrs.h")], check=True)
    assert compile_client(tmp_path / "client").exists()


def test_ctypes_structs_and_constants_match_the_header(tmp_path):
    """The ctypes mirrors of the ABI's structs have the C layout (size and
    every field's offset, from a C99 program compiled against
    include/srbcrs.h) and the constants the Python side passes equal the
    header's #defines: a field added to one side only fails here."""
    import subprocess
    structs = {"srbcrs_plan_desc": _capi.PlanDesc, "srbcrs_pack_opts": _capi.PackOpts,
               "srbcrs_run_opts": _capi.RunOpts}
    lines = ['#include <stddef.h>', '#include <stdio.h>', '#include "srbcrs.h"', "int main(void) {"]
    for cname, py in structs.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _ in py._fields_:
            lines.append(f'  printf("{cname} {f} %zu\\n", offsetof({cname}, {f}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)],
                   check=True)
    got = dict(l.rsplit(" ", 1) for l in subprocess.run([str(exe)], check=True, capture_output=True,
                                                        text=True).stdout.splitlines())
    for cname, py in structs.items():
        assert int(got[f"{cname} size"]) == ctypes.sizeof(py), cname
        for f, _ in py._fields_:
            assert int(got[f"{cname} {f}"]) == getattr(py, f).offset, (cname, f)
    text = (ROOT / "include" / "srbcrs.h").read_text()
    defs = {k: int(v) for k, v in re.findall(r"#define (SRBCRS_[A-Z_0-9]+) \(?(-?\d+)\)?", text)}
    assert defs["SRBCRS_OK"] == _capi.SRBCRS_OK and defs["SRBCRS_EINVAL"] == _capi.SRBCRS_EINVAL
    assert defs["SRBCRS_ESTATE"] == _capi.SRBCRS_ESTATE and defs["SRBCRS_ENOMEM"] == _capi.SRBCRS_ENOMEM
    assert defs["SRBCRS_TUNE_NONZERO_SWEEP"] == _capi.SRBCRS_TUNE_NONZERO_SWEEP
    assert (defs["SRBCRS_EPILOGUE_NONE"], defs["SRBCRS_EPILOGUE_RELU"]) == (_capi.EPILOGUE_NONE, _capi.EPILOGUE_RELU)
    for k, v in _capi.A_OPERANDS.items():
        assert defs[f"SRBCRS_A_{k.upper()}"] == v
    for k, v in _capi.B_STAGES.items():
        assert defs[f"SRBCRS_B_{k.upper()}"] == v
    assert defs["SRBCRS_PACK_CONDENSED"] == _capi.PACKINGS["column_condensed_dense"]
    assert defs["SRBCRS_PACK_FIXED_BLOCKS"] == _capi.PACKINGS["active_fixed_blocks_dense"]
    assert (defs["SRBCRS_DUP_LAST"], defs["SRBCRS_DUP_SUM"]) == (_capi.DUPS["last"], _capi.DUPS["sum"])
    for name, hdr in (("identity", "IDENTITY"), ("row_rcm", "RCM"), ("first_col_sort", "FIRST_COL"),
                      ("jaccard_greedy", "JACCARD"), ("sparse_rows", "SPARSE_ROWS"), ("explicit", "EXPLICIT")):
        assert defs[f"SRBCRS_ORDER_{hdr}"] == _capi.ORDERS[name], name


@pytest.mark.parametrize("n_shards", [1, 2, 3, 8, 50])
def test_shard_windows_balanced_and_contiguous(n_shards):
    """Contiguous cover of the windows; each shard's cost (blocks + 1 per
    window) stays within one window of the ideal share; the cut points are
    the first windows whose prefix cost reaches s/n of the total."""
    rng = np.random.default_rng(n_shards)
    lens = rng.integers(0, 40, size=37)
    lens[5] = 300                                  # one heavy window
    soff = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    b = _capi.shard_windows(soff, n_shards)
    assert b[0] == 0 and b[-1] == lens.size and (np.diff(b) >= 0).all()
    cost = np.concatenate([[0], np.cumsum(lens + 1)])
    total = int(cost[-1])
    for s in range(1, n_shards):
        target = -(-total * s // n_shards)
        assert b[s] == int(np.searchsorted(cost, target, side="left"))   # first prefix cost >= target
    shard_cost = cost[b[1:]] - cost[b[:-1]]
    assert shard_cost.max() <= total / n_shards + (lens.max() + 1)


def test_shard_windows_rejects_bad_input():
    with pytest.raises(_capi.SrbcrsError, match="n_shards"):
        _capi.shard_windows(np.array([0, 1], np.int32), 0)
    with pytest.raises(_capi.SrbcrsError, match="non-decreasing"):
        _capi.shard_windows(np.array([0, 5, 2], np.int32), 2)


def test_bench_byte_model_and_traffic_lookup():
    """bench.py's algorithmic-bytes formula (SR-BCRS dataflow: metadata, A
    blocks, gathered B rows, C) and its profile lookup by launch settings."""
    import bench
    M, N, Mo, nb = 65536, 512, 4096, 131072
    assert bench.algorithmic_bytes(M, N, Mo, nb, 0, "srbcrs") == \
        4 * (Mo + 1) + nb * (8 * 4 + 128 * 4) + nb * 8 * N * 4 + M * N * 4
    assert bench.algorithmic_bytes(M, N, Mo, nb // 8, 0, "srbcrs", 32, 32) == \
        4 * (Mo + 1) + nb // 8 * (32 * 4 + 1024 * 4) + nb // 8 * 32 * N * 4 + M * N * 4
    assert bench.algorithmic_bytes(10, 64, 1, 1, 100, "csr") == 4 * 11 + 8 * 100 + 4 * 64 * 100 + 4 * 10 * 64
    knobs = dict(bench.PUBLISHED_KNOBS["banded-524288"], tile_b=0, b_stage="registers")
    got = bench.measured_profile("banded-524288", 512, "srbcrs", knobs)
    assert got is not None and got["l2_egress_bytes"] > 0 and got["file"].startswith("profiles/")
    assert bench.measured_profile("banded-524288", 512, "srbcrs", {**knobs, "depth": 3}) is None
    assert bench.measured_profile("banded-524288", 512, "csr", knobs) is None
    assert bench.measured_profile("banded-524288", 512, "srbcrs", knobs, "32x32") is None


def test_bench_reports_the_library_default_a_operand():
    """bench.a_operand_used mirrors srbcrs_run_ex's default A source: compact
    for sparse 16x8 plans, dense for full 16x8 plans and for any 32x32 plan."""
    import types
    import bench

    def plan(bh, bw, stored, blocks):
        return types.SimpleNamespace(blk_h=bh, blk_w=bw, total_blocks=blocks,
                                     desc=types.SimpleNamespace(stored_values=stored))

    assert bench.a_operand_used(plan(16, 8, 10, 4), "default") == "compact"     # 10 of 512 positions
    assert bench.a_operand_used(plan(16, 8, 400, 4), "default") == "dense"
    assert bench.a_operand_used(plan(16, 8, -1, 4), "default") == "dense"       # no compact copy
    assert bench.a_operand_used(plan(32, 32, 10, 4), "default") == "dense"
    assert bench.a_operand_used(plan(32, 32, 10, 4), "compact") == "compact"


def test_gcn_autograd_on_cpu_with_torch_spmm():
    """The GCN module's aggregation op on the CPU (torch.sparse.mm as the SpMM):
    loss and gradients equal a dense fp64 autograd model with the same weights,
    so the backward really runs A^T (a non-symmetric A catches a missing transpose)."""
    torch = pytest.importorskip("torch")
    from mask_amd import datasets
    from mask_amd.gcn import GCN, graph_from_csr, torch_spmm
    rowptr, colind, values = random_csr(60, 60, 0.08, seed=5)
    m = datasets.CSRMatrix("tiny", rowptr, colind, values, 60, 60, 8, "uniform", 0)
    g = graph_from_csr(m, 12, torch.device("cpu"), seed=1)
    model = GCN((12, 10, 5), spmm=torch_spmm, seed=3)
    y = torch.arange(60) % 5
    loss = torch.nn.functional.nll_loss(model(g), y)
    loss.backward()
    A = torch.zeros(60, 60, dtype=torch.float64)
    for r in range(60):
        for e in range(rowptr[r], rowptr[r + 1]):
            A[r, colind[e]] += float(values[e])
    assert not torch.equal(A, A.T)
    ws = [p.detach().double().clone().requires_grad_(True) for p in model.parameters()]
    h = g.x.double()
    for i, w in enumerate(ws):
        h = A @ (h @ w)
        if i < len(ws) - 1:
            h = torch.relu(h)
    ref = torch.nn.functional.nll_loss(torch.log_softmax(h, 1), y)
    ref.backward()
    assert abs(loss.item() - ref.item()) < 1e-5
    for p, w in zip(model.parameters(), ws):
        assert torch.allclose(p.grad.double(), w.grad, atol=1e-5, rtol=1e-4)


def test_operand_checks_raise_before_any_launch():
    """Plan.run / Plan.tune / GeneratedOperator.run validate dense and out
    with check_operand before handing a pointer to the GPU: a host tensor,
    a wrong dtype or a transposed view raise here, without a GPU."""
    torch = pytest.importorskip("torch")
    from mask_amd.SRBCRSSpMM import check_operand
    dev = torch.device("cuda", 0)
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        check_operand(torch.ones(4, 16), "dense", dev)
    with pytest.raises(RuntimeError, match="torch tensor"):
        check_operand(np.ones((4, 16), np.float32), "dense", dev)


def test_bench_roofline_is_bounded():
    """bench.roofline: frac is the compulsory bytes over the step time against
    the 8 TB/s peak (null above 1); the dataflow bytes are a rate only."""
    import bench
    t = 1e-3
    ok = bench.roofline(t, dataflow_bytes=9e9, compulsory_bytes=2e9, padded_flops=1e10, prof=None)
    assert ok["frac"] == 0.25 and ok["achieved"] == 2000.0 and ok["dataflow_gbs"] == 9000.0
    assert ok["basis"].startswith("compulsory")
    bad = bench.roofline(t, dataflow_bytes=9e9, compulsory_bytes=9e9, padded_flops=1e10, prof=None)
    assert bad["frac"] is None and bad["frac_rejected"] == 1.125


def test_bench_l2_egress_never_feeds_hbm_bytes():
    """A profile whose only byte figure is the L2-egress counters (TCC_EA0 *
    DRAM requests, which include memory-side-cache hits) must not become the
    HBM bytes: those come only from a memory-controller (UMC) measurement;
    without one the HBM bytes are the compulsory bytes, and the basis says so."""
    import bench
    t = 1e-3
    prof = {"file": "profiles/p.md", "l2_egress_bytes": 6_000_000_000, "traffic_bytes": 6_100_000_000}
    r = bench.roofline(t, 9e9, 2e9, 1e10, prof, bound="l2-miss gather path", gather_ceiling={"a": 7000.0, "b": 7500.0})
    assert r["hbm_bytes"] == 2_000_000_000 and r["hbm_basis"].startswith("compulsory")
    assert r["l2_egress_bytes"] == 6_000_000_000 and r["l2_egress_frac"] == 0.75
    assert r["gather_ceiling_gbs"] == 7500.0 and r["gather_frac"] == 0.8
    assert r["frac"] == 0.25 and r["bound"] == "l2-miss gather path"
    umc = bench.roofline(t, 9e9, 2e9, 1e10, dict(prof, hbm_bytes_umc=1_000_000_000))
    assert umc["hbm_bytes"] == 1_000_000_000 and "UMC" in umc["hbm_basis"] and umc["hbm_frac"] == 0.125
    assert umc["frac"] == 0.25   # the headline fraction keeps its compulsory basis


def test_committed_profiles_are_physical():
    """Every committed kernel profile's L2-egress and UMC-measured HBM bytes
    imply at most the 8 TB/s peak over its own kernel average, and bench.py
    finds the profile of each published launch setting."""
    import bench
    from pathlib import Path
    found = 0
    for path in sorted((Path(bench.ROOT) / "profiles").glob("spmm_*.md")):
        fields = dict(l.split(":", 1) for l in path.read_text().splitlines()
                      if l.startswith(("l2_egress_bytes:", "hbm_bytes_umc:", "kernel_avg_ns:")))
        for key in ("l2_egress_bytes", "hbm_bytes_umc"):
            if key in fields:
                found += 1
                gbs = int(fields[key]) / int(fields["kernel_avg_ns"])
                assert gbs <= bench.HBM_PEAK_GBS, (path.name, key, gbs)
    assert found >= 1
    for name, knobs in bench.PUBLISHED_KNOBS.items():
        k = dict({key: v for key, v in knobs.items() if key != "N"})
        k.setdefault("tile_b", 0)
        k.setdefault("b_stage", "registers")
        prof = bench.measured_profile(name, knobs.get("N", 512), "srbcrs", k)
        assert prof is not None and prof["l2_egress_bytes"] > 0, name
