#!/usr/bin/env python3
"""SR-BCRS 16x8 fp32 SpMM benchmark on one MI355X.

One "step" = one C = A * B over the whole workload (all launches of the
chosen schedule) with A (converted), B and C resident in HBM.  Conversion is
outside the timed region (the reference's kernel_only_post_conversion
contract).  Prints ONE JSON line.

Default workload: uniform-65536 at N = 512 (the metric's configuration).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, published
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix, published


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="uniform-65536",
                    choices=["uniform-4096", "uniform-65536", "banded-524288", "rmat-2^20", "gcn-232965"])
    ap.add_argument("--N", type=int, default=None, help="dense width (default: the workload's)")
    ap.add_argument("--mtx", default=None, help="a MatrixMarket file instead of a synthetic workload")
    ap.add_argument("--shard-sim", type=int, default=0,
                    help="time one GPU's share of a G-way row sharding and column sharding (one GPU, no communication)")
    ap.add_argument("--gcn-train", action="store_true",
                    help="GCN training step (GCN 512-256-64 + Adam) through the srbcrs_spmm drop-in")
    ap.add_argument("--gcn-forward", action="store_true",
                    help="time the GCN workload's two-layer forward instead of one SpMM")
    ap.add_argument("--row-order", default="identity",
                    choices=["identity", "row_rcm", "first_col_sort", "jaccard_greedy"],
                    help="pack rows in this order (inverse map fused into the kernel store)")
    ap.add_argument("--schedule", default="auto", help="row | split[:cap] | strict_lb[:w] | multi_bind | auto")
    ap.add_argument("--kernel", default="srbcrs", choices=["srbcrs", "csr"])
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the CPU baseline leg")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--sustained-s", type=float, default=2.0,
                    help="after the K timed steps, also time back-to-back steps for about this long "
                         "(reported apart as 'sustained'; 0 = skip)")
    ap.add_argument("--no-check", action="store_true")
    ap.add_argument("--depth", type=int, default=0, help="kernel knob: blocks in flight per wave (2/4/8)")
    ap.add_argument("--tile-b", type=int, default=0, help="kernel knob: 16/32/64")
    ap.add_argument("--wg-cols", type=int, default=0, help="kernel knob: columns per workgroup")
    ap.add_argument("--grid-order", type=int, default=0, help="kernel knob: 1 chunk-major, 2 window-major")
    ap.add_argument("--wpw", type=int, default=0, help="kernel knob: row windows streamed per wave")
    ap.add_argument("--blk", default="16x8", choices=["16x8", "32x32"],
                    help="SR-BCRS block shape (16x8: preprocess_gpu_16x8; 32x32: the base preprocess_gpu)")
    ap.add_argument("--tune", action="store_true",
                    help="run srbcrs_plan_tune (the one-time launch-setting search) before the warm-up instead of "
                         "the published setting of the workload")
    ap.add_argument("--no-tune", action="store_true",
                    help="GCN benches: skip the tuning on each plan's first call per width")
    ap.add_argument("--extra-off", action="store_true",
                    help="default run: skip the extra configurations (banded)")
    ap.add_argument("--b-stage", default="default", choices=["default", "registers", "lds"],
                    help="kernel knob: where the ring holds the gathered B rows")
    ap.add_argument("--a-operand", default="default", choices=["default", "compact", "dense"],
                    help="block-value copy the kernel reads (default: compact when blocks are at most half full)")
    ap.add_argument("--copy-seconds", type=float, default=0.0,
                    help="with --copy-calibration-mb: repeat the copy for this long")
    ap.add_argument("--lean", action="store_true",
                    help="profiling runs: skip the stream / gather probes and the library-tuned leg")
    ap.add_argument("--umc-seconds", type=float, default=0.0,
                    help="only measure HBM traffic at the memory controllers: amd-smi UMC activity sampled while a "
                         "1 GiB copy and then the workload (its published setting) run back to back this long each")
    ap.add_argument("--window-sharing", action="store_true",
                    help="host only: distinct (row window, column) pairs at window heights 16..256, i.e. how many "
                         "B-row gathers windows of more rows would share")
    ap.add_argument("--gather-study", action="store_true",
                    help="only time the gather probe on the workload's own B-row index stream: unit order vs "
                         "units of W windows merged by column, over grids and column-chunk widths")
    ap.add_argument("--sweep-crossover", action="store_true",
                    help="only time the nonzero sweep against the tuned MFMA kernels on 65536-row matrices of "
                         "16 values per row whose window columns are clustered to set the block fill (the "
                         "low-density dispatch threshold, SRBCRSSpMM.SWEEP_FILL)")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="only run an elementwise copy of this many MiB (5 launches) to calibrate "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE against a known byte count")
    return ap.parse_args()


def copy_calibration(mib, seconds=0.0):
    """Known-traffic reference kernel: out = in * 1 over mib MiB reads + writes,
    5 times, or back to back for `seconds` (a sustained copy load, the
    reference point for system-level memory-controller activity)."""
    import torch
    n = mib * (1 << 20) // 4
    a = torch.ones(n, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    reps, t0 = 0, time.time()
    while reps < 5 or time.time() - t0 < seconds:
        for _ in range(5 if seconds <= 0 else 50):
            torch.mul(a, 1.0, out=b)
            reps += 1
        torch.cuda.synchronize()
    el = time.time() - t0
    print(json.dumps({"copy_calibration_bytes_read": n * 4, "copy_calibration_bytes_written": n * 4,
                      "reps": reps, "gbs": round(2 * n * 4 * reps / el / 1e9, 1)}))


# Measurement probes of the library (mask_amd/csrc/srbcrs_probe.h): internal,
# not in the public C ABI, bound here only.
PROBE_SIGS = {
    "srbcrs_stream_probe": ("i32 vp vp i64 i32 vp"),
    "srbcrs_gather_probe": ("vp vp i32 i32 vp i64 i32 i32 vp vp"),
}


def probes():
    """The library with its probe entry points bound (ctypes)."""
    import ctypes
    from mask_amd import _capi
    L = _capi.lib()
    kinds = {"i32": ctypes.c_int32, "i64": ctypes.c_int64, "vp": ctypes.c_void_p}
    for name, sig in PROBE_SIGS.items():
        f = getattr(L, name)
        f.argtypes = [kinds[k] for k in sig.split()]
        f.restype = ctypes.c_int
    return L


def copy_bandwidth(mib=2048, reps=10):
    """What plain streaming kernels move on this box, as context for the
    SpMM's HBM-side rate: the library's float4 grid-stride probes
    (srbcrs_stream_probe) over mib MiB buffers -- copy (read + write, the mix
    of an SpMM that writes C), read-only, write-only -- each at a few grid
    sizes, best kept, HIP events on the launch stream.  GB/s of bytes moved."""
    import torch
    from mask_amd import _capi
    L = probes()
    n = mib * (1 << 20) // 4
    a = torch.ones(n, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    st = torch.cuda.current_stream().cuda_stream
    out = {}
    for kind, name, mult in ((0, "copy", 2), (1, "read", 1), (2, "write", 1)):
        best = 0.0
        for blocks in (1024, 4096, 65536):
            for _ in range(2):
                _capi.check(L.srbcrs_stream_probe(kind, a.data_ptr(), b.data_ptr(), n, blocks, st))
            e = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
            e[0].record()
            for _ in range(reps):
                _capi.check(L.srbcrs_stream_probe(kind, a.data_ptr(), b.data_ptr(), n, blocks, st))
            e[1].record()
            torch.cuda.synchronize()
            best = max(best, mult * n * 4 * reps / (e[0].elapsed_time(e[1]) / 1e3) / 1e9)
        out[name] = round(best, 1)
    del a, b
    torch.cuda.empty_cache()
    return out


def gather_time(rows, row_off, rpi, B, ldb, n_chunks, mapping, reps=20):
    """One srbcrs_gather_probe configuration, timed: (ms per launch, bytes
    gathered per launch).  rows / row_off are host arrays (int32 / int64);
    every row index is checked against B's rows before the upload."""
    import torch
    from mask_amd import _capi
    L = probes()
    n_rows_b = B.numel() // ldb
    rows = np.ascontiguousarray(rows, dtype=np.int32)
    row_off = np.ascontiguousarray(row_off, dtype=np.int64)
    assert rows.size == 0 or (int(rows.min()) >= 0 and int(rows.max()) < n_rows_b), "row index outside B"
    assert np.all(np.diff(row_off) % 8 == 0) and row_off[0] == 0 and row_off[-1] == rows.size
    seg = 256 // rpi
    assert n_chunks * seg <= ldb
    n_groups = row_off.size - 1
    d_rows = torch.from_numpy(rows).cuda()
    d_off = torch.from_numpy(row_off).cuda()
    nwg = (n_groups * n_chunks + 7) // 8 * 8
    out = torch.empty(nwg * 64, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    call = lambda: _capi.check(L.srbcrs_gather_probe(d_rows.data_ptr(), d_off.data_ptr(), n_groups, rpi,
                                                     B.data_ptr(), ldb, n_chunks, mapping, out.data_ptr(), st))
    for _ in range(3):
        call()
    e = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    e[0].record()
    for _ in range(reps):
        call()
    e[1].record()
    torch.cuda.synchronize()
    ms = e[0].elapsed_time(e[1]) / reps
    return ms, int(rows.size) * n_chunks * seg * 4


def gather_ceiling(n_lines=1 << 24, seed=7):
    """What gathers out of the L2 move on this box: n_lines uniformly random
    128-byte lines (eight per 1 KB load instruction) of a 134 MB buffer,
    which the 256 MB memory-side cache holds, and of a 2.1 GB buffer, which
    it does not; the same bytes as random 1 KB row segments of the 134 MB
    buffer; and as 1 KB segments read in address order (the path's streaming
    rate, the highest of the four).  One XCD's 4 MB L2 holds 3 % of the
    smaller buffer, so nearly every line leaves the L2: the rates are the
    L2-miss path's.  GB/s of gathered bytes (best of the XCD-blocked and
    dispatch-order grids)."""
    import torch
    rng = np.random.default_rng(seed)
    out = {}
    for name, mib, rpi in (("mall_128B", 128, 8), ("hbm_128B", 2048, 8), ("mall_1KB", 128, 1),
                           ("mall_seq_1KB", 128, 1)):
        seg = 256 // rpi
        B = torch.ones(mib * (1 << 20) // 4, device="cuda")
        n_rows_b = B.numel() // seg
        n = n_lines * 128 // (seg * 4)
        if name.startswith("mall_seq"):   # the same bytes read in address order: the L2-miss path's streaming rate
            rows = (np.arange(n, dtype=np.int64) % n_rows_b).astype(np.int32)
        else:
            rows = rng.integers(0, n_rows_b, size=n, dtype=np.int64).astype(np.int32)
        per = 2048 if rpi == 1 else 4096
        row_off = np.arange(0, n + 1, per, dtype=np.int64)
        best = 0.0
        for mapping in (0, 1):
            ms, nbytes = gather_time(rows, row_off, rpi, B, seg, 1, mapping)
            best = max(best, nbytes / (ms / 1e3) / 1e9)
        out[name] = round(best, 1)
        del B
        torch.cuda.empty_cache()
    return out


def gather_study(args):
    """Gather-only timings (srbcrs_gather_probe) of the workload's own B-row
    index stream at N = 512, printed as one JSON line.  Groups are row
    windows, or for the skewed graphs (R-MAT, GCN) segments of at most 64
    units of a window, as the split schedule cuts them; W consecutive groups
    go to one wave, in unit order or merged by first B-row index; column
    chunks of 32 to 256 columns; grids: dispatch-order chunk sweep (0), the
    XCD-blocked chunk-major grid (1), or chunks pinned to XCDs (2)."""
    import torch
    from mask_amd import _capi, datasets
    m = datasets.make_config(args.config)
    conv = _capi.convert_host(m.rowptr, m.colind, m.values, m.M)
    soff, sidx = conv["soff"].astype(np.int64), conv["sidx"].reshape(-1, 8)
    N = 512
    B = torch.from_numpy(m.dense(N)).cuda()
    nb = sidx.shape[0]
    skewed = m.name in ("rmat-2^20", "gcn-232965")
    win = np.repeat(np.arange(soff.size - 1), np.diff(soff))
    if skewed:   # segments of at most 64 units of one window
        pos = np.arange(nb) - soff[win]
        seg_key = win * 1_000_000 + pos // 64
        _, seg = np.unique(seg_key, return_inverse=True)
    else:
        seg = win
    if skewed:
        runs = [(1, False, 4, 0), (1, False, 4, 1), (1, False, 4, 2), (4, True, 4, 0), (8, True, 4, 0),
                (1, False, 8, 0), (1, False, 2, 0), (1, False, 1, 0), (1, False, 1, 1), (4, True, 4, 2)]
    else:
        runs = [(8, False, 1, 1), (8, False, 4, 2), (8, True, 1, 2), (8, True, 2, 2), (8, True, 4, 2),
                (4, True, 2, 2), (4, True, 4, 2), (16, True, 4, 2), (32, True, 4, 2), (1, False, 4, 2),
                (1, False, 1, 1)]
    res = []
    for W, merge, rpi, mapping in runs:
        grp = seg // W
        perm = np.lexsort((np.arange(nb), sidx[:, 0], grp)) if merge else np.arange(nb)
        rows = sidx[perm].ravel()
        row_off = np.zeros(grp.max() + 2, np.int64)
        np.add.at(row_off, grp + 1, 8)
        row_off = np.cumsum(row_off)
        n_chunks = N // (256 // rpi)
        if mapping == 2 and 8 % n_chunks and n_chunks % 8:
            continue
        ms, nbytes = gather_time(rows, row_off, rpi, B, N, n_chunks, mapping, reps=5 if skewed else 20)
        r = {"W": W, "merged": merge, "cols": 256 // rpi, "mapping": mapping, "ms": round(ms, 4),
             "gbs": round(nbytes / ms / 1e6, 1)}
        print("[gather-study]", r, file=sys.stderr, flush=True)
        res.append(r)
    print(json.dumps({"workload": m.name, "N": N, "gathered_bytes": int(nb * 8 * N * 4), "runs": res}), flush=True)


def gcn_forward_bench(args):
    """The GCN workload's two-layer forward alone (what the default run
    reports as extra_configs["gcn-232965-forward"]), after a 1 s settle.
    One JSON line."""
    res = gcn_forward_measure(args, settle_s=1.0)
    print(json.dumps({"metric": "GCN two-layer forward (gcn-232965, features 512, hidden 256, out 64)",
                      "higher_is_better": True, "n_gpus": 1, "dtype": "f32",
                      "data": "synthetic R-MAT graph + N(0,1) features (seeded)", **res}), flush=True)


def _find_key(obj, key):
    """The first value under `key` anywhere in a nested JSON object."""
    if isinstance(obj, dict):
        if key in obj:
            return obj[key]
        obj = list(obj.values())
    if isinstance(obj, list):
        for v in obj:
            r = _find_key(v, key)
            if r is not None:
                return r
    return None


def _pct(v):
    if isinstance(v, dict):
        v = v.get("value")
    try:
        return float(v)
    except (TypeError, ValueError):
        return None


def _clustered_rows(M, K, per_row, pool, seed):
    """M rows of per_row distinct sorted columns; the rows of each 16-row
    window draw them from one set of `pool` window columns (pool None: from
    all K), so the SR-BCRS 16x8 block fill is about per_row / pool."""
    rng = np.random.default_rng(seed)
    cols = np.empty((M, per_row), np.int64)
    for w in range(M // 16):
        src = rng.choice(K, pool, replace=False) if pool else None
        for r in range(16):
            cols[16 * w + r] = np.sort(rng.choice(src, per_row, replace=False) if pool
                                       else rng.choice(K, per_row, replace=False))
    rowptr = (np.arange(M + 1) * per_row).astype(np.int32)
    return rowptr, cols.reshape(-1).astype(np.int32), rng.uniform(-1, 1, M * per_row).astype(np.float32)


def sweep_crossover(args):
    """The nonzero sweep (grid order 5, default knobs) against the MFMA
    kernels at the setting srbcrs_plan_tune picks, on 65536 x 65536 matrices
    of 16 values per row at block fills from 0.06 to 0.5, N = 512: sustained
    ms per launch (--sustained-s of back-to-back launches each, after the
    tuning and 20 warm-up launches).  One JSON line."""
    import torch
    from mask_amd.SRBCRSSpMM import Plan
    M = K = 65536
    N = args.N or 512
    dev = torch.device("cuda", 0)
    B = torch.rand((K, N), device=dev) * 2 - 1
    C = torch.empty((M, N), device=dev)
    secs = args.sustained_s if args.sustained_s > 0 else 1.0

    def sustained(fn):
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        n = 0
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        while time.perf_counter() - t0 < secs:
            for _ in range(50):
                fn()
            n += 50
            torch.cuda.synchronize()
        e1.record()
        torch.cuda.synchronize()
        return round(e0.elapsed_time(e1) / n, 5)

    rows = []
    for pool in (None, 256, 128, 64, 32):
        rp, ci, vv = _clustered_rows(M, K, 16, pool, seed=5)
        plan = Plan(torch.from_numpy(rp).to(dev), torch.from_numpy(ci).to(dev), torch.from_numpy(vv).to(dev), M)
        fill = int(rp[-1]) / (plan.total_blocks * 128)
        tk = plan.tune(B, C, reps=3)
        ms_mfma = sustained(lambda: plan.run(B, C))
        ms_sweep = sustained(lambda: plan.run(B, C, grid_order=NZSWEEP))
        rows.append({"window_pool": pool, "block_fill": round(fill, 4), "mfma_tuned": tk, "mfma_ms": ms_mfma,
                     "sweep_ms": ms_sweep, "sweep_faster": ms_sweep < ms_mfma})
        print(f"[crossover] pool={pool} fill={fill:.3f} mfma={ms_mfma} sweep={ms_sweep}", file=sys.stderr,
              flush=True)
        del plan
        torch.cuda.empty_cache()
    print(json.dumps({"sweep_crossover": rows, "N": N, "rows_per_matrix": M, "values_per_row": 16}), flush=True)


def umc_measure(args):
    """HBM traffic of the workload's steady state, measured at the memory
    controllers: no per-kernel counter separates memory-side-cache (MALL)
    hits from HBM accesses, but the SMU's UMC activity sees only HBM.  A
    thread samples `amd-smi metric -u --json` (gfx and UMC activity, %)
    while, for args.umc_seconds each, a 1 GiB copy (torch.mul, known bytes)
    and then the workload at its published setting run back to back.  Only
    samples with gfx activity >= 99 % count.  The copy's bytes per second
    over its UMC activity give the GB/s of one UMC percent; the workload's
    HBM bytes per step = its activity x that scale x its step time.  One
    JSON line."""
    import subprocess
    import threading
    import torch
    from mask_amd import datasets
    from mask_amd.SRBCRSSpMM import Plan
    samples, stop = [], threading.Event()

    def sampler():
        while not stop.is_set():
            t = time.perf_counter()
            try:
                txt = subprocess.run(["amd-smi", "metric", "-u", "--json"], capture_output=True, text=True,
                                     timeout=20).stdout
                j = json.loads(txt[min(i for i in (txt.find("{"), txt.find("[")) if i >= 0):])
                g, u = _pct(_find_key(j, "gfx_activity")), _pct(_find_key(j, "umc_activity"))
                if g is not None and u is not None:
                    samples.append((t, g, u))
            except Exception as e:   # a missing or failing amd-smi leaves no samples; reported below
                samples.append((t, None, repr(e)[:200]))
                stop.wait(1.0)
            stop.wait(0.25)

    def phase(fn, seconds):
        t0 = time.perf_counter()
        n = 0
        while time.perf_counter() - t0 < seconds:
            for _ in range(20):
                fn()
            n += 20
            torch.cuda.synchronize()
        t1 = time.perf_counter()
        good = [u for (t, g, u) in samples if g is not None and t0 + 0.5 <= t <= t1 and g >= 99]
        return n, t1 - t0, good

    th = threading.Thread(target=sampler, daemon=True)
    th.start()
    a = torch.ones((1 << 30) // 4, device="cuda")
    b = torch.empty_like(a)
    n_c, s_c, u_c = phase(lambda: torch.mul(a, 1.0, out=b), args.umc_seconds)
    copy_gbs = 2 * a.numel() * 4 * n_c / s_c / 1e9
    del a, b
    m = datasets.make_config(args.config)
    k = dict(PUBLISHED_KNOBS[m.name])
    N = k.pop("N", 512)
    dev = torch.device("cuda", 0)
    t = lambda x: torch.from_numpy(x).to(dev)
    plan = Plan(t(m.rowptr), t(m.colind), t(m.values), m.M)
    sched = "split" if m.name in ("rmat-2^20", "gcn-232965") else "row"
    plan.set_schedule(sched, 0)
    B = t(m.dense(N))
    C = torch.empty((m.M, N), device=dev)
    for _ in range(5):
        plan.run(B, C, **k)
    n_w, s_w, u_w = phase(lambda: plan.run(B, C, **k), args.umc_seconds)
    stop.set()
    th.join(timeout=30)
    errors = sorted({u for (t, g, u) in samples if g is None})
    med = lambda v: float(np.median(v)) if v else None
    uc, uw = med(u_c), med(u_w)
    scale = copy_gbs / uc if uc else None
    ms = s_w / n_w * 1e3
    out = {"workload": m.name, "N": N, "knobs": k, "schedule": sched, "seconds_each": args.umc_seconds,
           "copy": {"gbs": round(copy_gbs, 1), "umc_pct": uc, "samples": len(u_c)},
           "workload_run": {"steps": n_w, "ms_per_step": round(ms, 5), "umc_pct": uw, "samples": len(u_w),
                            "umc_pct_values": sorted(set(u_w))},
           "gbs_per_umc_pct": round(scale, 2) if scale else None,
           "hbm_gbs": round(uw * scale, 1) if scale and uw is not None else None,
           "hbm_bytes_per_step": int(uw * scale * 1e9 * ms / 1e3) if scale and uw is not None else None,
           "sampler_errors": errors[:3]}
    print(json.dumps(out), flush=True)


def gcn_forward_measure(args, ceiling=None, settle_s=0.0):
    """BASELINE config 5 as one step: the GCN workload's two-layer forward
    relu(A (X W1)) -> A (H W2) on one GPU (X 232965 x 512, W1 512 x 256, W2
    256 x 64): dense GEMMs through torch (fp32, each on the faster of
    hipBLASLt and rocBLAS) and both SR-BCRS SpMMs (split schedule; N = 256
    at the published setting with the relu epilogue, N = 64 at the library's
    tuned choice), timed as one step with HIP events, then each part on its
    own.  Each SpMM carries its roofline block and the fp64
    oracle gate on a row sample of its own input.  Returns the result dict."""
    import torch
    from mask_amd import datasets
    from mask_amd.gcn import glorot_weights
    from mask_amd.SRBCRSSpMM import Plan
    dev = torch.device("cuda", 0)
    m = datasets.make_config("gcn-232965")
    gen = torch.Generator(device="cpu")
    gen.manual_seed(m.seed)
    X = torch.randn((m.M, 512), generator=gen).to(dev)
    w1, w2 = glorot_weights([512, 256, 64], seed=m.seed, device=dev)
    t = lambda a: torch.from_numpy(a).to(dev)
    plan = Plan(t(m.rowptr), t(m.colind), t(m.values), m.M)
    plan.set_schedule("split", 0)
    k256 = {k: v for k, v in PUBLISHED_KNOBS["gcn-232965"].items() if k != "N"}
    XW = torch.empty((m.M, 256), device=dev)
    H = torch.empty((m.M, 256), device=dev)
    HW = torch.empty((m.M, 64), device=dev)
    out = torch.empty((m.M, 64), device=dev)
    torch.mm(X, w1, out=XW)
    plan.run(XW, H, **k256)
    torch.relu_(H)
    torch.mm(H, w2, out=HW)
    k64 = plan.tune(HW, out)   # the N = 64 aggregation at the library's own choice
    # W2 kept as torch.nn.Linear keeps its weight (out x in, the GEMM reads it transposed): 0.112
    # against 0.137 ms for the 256 x 64 row-major operand
    w2t = w2.t().contiguous()
    # each GEMM on the faster of torch's two BLAS back ends for its shape (hipBLASLt / rocBLAS:
    # X W1 0.466 ms on rocBLAS against 0.522 on hipBLASLt, H W2 the other way round)
    blas = {"gemm_xw1": _faster_blas(lambda: torch.mm(X, w1, out=XW)),
            "gemm_hw2": _faster_blas(lambda: torch.mm(H, w2t.t(), out=HW))}
    on = torch.backends.cuda.preferred_blas_library
    blas_default = on()

    parts = {
        "gemm_xw1": lambda: (on(blas["gemm_xw1"]), torch.mm(X, w1, out=XW)),
        # relu(A (X W1)): the relu epilogue in the SpMM's stores (no pass of its own)
        "spmm_n256": lambda: plan.run(XW, H, relu=True, **k256),
        "gemm_hw2": lambda: (on(blas["gemm_hw2"]), torch.mm(H, w2t.t(), out=HW)),
        "spmm_n64": lambda: plan.run(HW, out),
    }

    def fwd():
        for f in parts.values():
            f()

    for _ in range(args.warmup):
        fwd()
    torch.cuda.synchronize()
    warm = args.warmup
    t_set = time.perf_counter()
    while time.perf_counter() - t_set < settle_s:
        for _ in range(10):
            fwd()
        warm += 10
        torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(args.steps):
        fwd()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    part_ms = {name: round(_time_ms(f, args.steps, 2), 5) for name, f in parts.items()}
    M, nnz = m.M, m.nnz
    flops = {"gemm_xw1": 2.0 * M * 512 * 256, "spmm_n256": 2.0 * nnz * 256, "gemm_hw2": 2.0 * M * 256 * 64,
             "spmm_n64": 2.0 * nnz * 64}
    nb, Mo = plan.total_blocks, plan.row_windows
    spmm = {}
    for name, N, knobs in (("spmm_n256", 256, dict(k256, tile_b=0)), ("spmm_n64", 64, dict(k64, tile_b=0))):
        knobs.setdefault("b_stage", "registers")
        ts = part_ms[name] / 1e3
        comp = nb * (8 * 4 + 128 * 4) + 4 * (Mo + 1) + m.K * N * 4 + M * N * 4
        prof = measured_profile(m.name, N, "srbcrs", knobs)
        spmm[name] = {"N": N, "ms": part_ms[name], "gflops": round(flops[name] / ts / 1e9, 1),
                      "knobs": {k: knobs[k] for k in ("depth", "wg_cols", "grid_order", "windows_per_wave",
                                                      "a_operand", "b_stage")},
                      "roofline": roofline(ts, algorithmic_bytes(M, N, Mo, nb, nnz, "srbcrs"), comp,
                                           2.0 * 16 * 8 * nb * N, prof, BOUND.get(m.name, "hbm"), ceiling)}
    parity = {}
    if not args.no_check:
        # the GEMMs as timed (their chosen back ends) against fp64 on a row sample: fp32 arithmetic,
        # no reduced-precision path (elementwise |err| <= 1e-5 (|X| |W|), the oracle gate's form)
        rows = torch.from_numpy(np.random.default_rng(m.seed).choice(m.M, 2048, replace=False)).to(dev)
        for name, a_, w_, c_ in (("gemm_xw1", X, w1, XW), ("gemm_hw2", H, w2, HW)):
            parts[name]()
            torch.cuda.synchronize()
            a64, w64 = a_[rows].double(), w_.double()
            err = (c_[rows].double() - a64 @ w64).abs()
            bound = a64.abs() @ w64.abs()
            parity[name] = {"max_ratio": float((err / bound.clamp_min(1e-30)).max()),
                            "rel_l2": float(err.norm() / (a64 @ w64).norm()),
                            "pass": bool((err <= 1e-5 * bound).all())}
        # the fused relu is torch.relu of the plain SpMM output, bit for bit
        parts["spmm_n256"]()
        fused = H.clone()
        plan.run(XW, H, **k256)
        parity["relu_epilogue"] = {"pass": bool(torch.equal(fused, torch.relu(H)))}
        # H now holds the SpMM's own output (no relu)
        parity["spmm_n256"] = parity_leg(m, XW.cpu().numpy(), H.cpu().numpy())
        plan.run(HW, out)
        parity["spmm_n64"] = parity_leg(m, HW.cpu().numpy(), out.cpu().numpy())
    on(blas_default)
    total = sum(flops.values())
    res = {"value": round(total / (ms / 1e3) / 1e9, 2), "unit": "GFLOP/s", "steps": args.steps, "warmup": warm,
           "ms_per_step": round(ms, 5),
           "config": {"workload": GCN_FORWARD, "nodes": M, "nnz": nnz, "features": 512, "hidden": 256, "out": 64,
                      "schedule": f"{plan.policy[0]}:{plan.policy[1]}", "seed": m.seed,
                      "flops": {k: int(v) for k, v in flops.items()},
                      "gemm": {k: f"torch.mm fp32 ({'hipBLASLt' if v == 'cublaslt' else 'rocBLAS'})"
                               for k, v in blas.items()},
                      "relu": "fused into the N = 256 SpMM's stores"},
           "parts_ms": part_ms, "spmm": spmm, "parity": parity}
    del plan, X, XW, H, HW, out
    torch.cuda.empty_cache()
    return res


def _faster_blas(gemm, reps=20):
    """The torch BLAS back end ("cublaslt" = hipBLASLt, "cublas" = rocBLAS on
    ROCm) that runs gemm faster, timed here; torch's default is restored."""
    import torch
    on = torch.backends.cuda.preferred_blas_library
    default = on()
    ms = {}
    for name in ("cublaslt", "cublas"):
        on(name)
        ms[name] = _time_ms(gemm, reps, 3)
    on(default)
    return min(ms, key=ms.get)


def _time_ms(fn, steps, warmup):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    e[0].record()
    for _ in range(steps):
        fn()
    e[1].record()
    torch.cuda.synchronize()
    return e[0].elapsed_time(e[1]) / steps


def shard_sim_bench(args):
    """One GPU's share of a G-way sharding of the workload, timed at its real
    shape on this GPU (communication excluded, one JSON line):
      rows:    srbcrs_shard_windows cuts the row windows into G ranges of
               near-equal cost; every shard's plan is tuned and timed; the
               critical path is the slowest shard;
      columns: every GPU holds all of A and N/G columns of B and C: the full
               plan at width N/G."""
    import torch
    from mask_amd import datasets
    from mask_amd.SRBCRSSpMM import Plan
    from mask_amd.sharding import RowShardedSpMM
    dev = torch.device("cuda", 0)
    G = args.shard_sim
    m = datasets.make_config(args.config)
    N = args.N or m.N
    t = lambda a: torch.from_numpy(a).to(dev)
    rp, ci, vv = t(m.rowptr), t(m.colind), t(m.values)
    B = t(m.dense(N))
    C = torch.empty((m.M, N), device=dev)
    sh = RowShardedSpMM(rp, ci, vv, m.M, G)
    sh.set_schedule("auto")
    row_ms = []
    for i, (r0, r1) in enumerate(sh.ranges):
        if sh.plans[i] is None:
            row_ms.append(0.0)
            continue
        sh.plans[i].tune(B, C[r0:r1])
        row_ms.append(_time_ms(lambda: sh.run_shard(i, B, C), args.steps, args.warmup))
    full = Plan(rp, ci, vv, m.M)
    full.set_schedule("auto")
    Nc = N // G if N % (16 * G) == 0 else 0
    col_ms = None
    if Nc:
        Bc = B[:, :Nc].contiguous()
        Cc = torch.empty((m.M, Nc), device=dev)
        full.tune(Bc, Cc)
        col_ms = _time_ms(lambda: full.run(Bc, Cc), args.steps, args.warmup)
    full.tune(B, C)
    one_ms = _time_ms(lambda: full.run(B, C), args.steps, args.warmup)
    flops = 2.0 * m.nnz * N
    mx = max(row_ms)
    print(json.dumps({
        "metric": f"simulated {G}-way sharding of the SpMM: one GPU's share timed on one MI355X (no communication)",
        "value": round(flops / mx / 1e6, 1), "unit": "GFLOP/s (row sharding, critical path)",
        "higher_is_better": True, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "dtype": "f32",
        "config": {"workload": m.name, "N": N, "shards": G},
        "one_gpu_ms": round(one_ms, 4),
        "rows": {"ranges": sh.ranges, "shard_ms": [round(x, 4) for x in row_ms], "max_ms": round(mx, 4),
                 "imbalance": round(mx / (sum(row_ms) / G), 3), "speedup_vs_one": round(one_ms / mx, 2)},
        "columns": None if col_ms is None else {
            "N_per_gpu": Nc, "ms": round(col_ms, 4), "speedup_vs_one": round(one_ms / col_ms, 2),
            "gflops": round(flops / col_ms / 1e6, 1)},
    }), flush=True)


def gcn_train_bench(args):
    """Full-batch GCN training steps on the GCN workload through the drop-in
    path the reference's GCN script uses (eva_gcn_sparsene.py:267-343): a
    two-layer GCN 512-256-64 (dropout 0.5) whose aggregations run through the
    srbcrs_spmm external backend (forward A @ X, backward A^T @ dY on the
    transposed CSR), log-softmax + NLL on synthetic labels, Adam.  Timed per
    SR-BCRS variant (16x8 and the 32x32 base) and, for comparison, with
    torch.sparse.mm on ROCm.  One JSON line."""
    import torch
    import torch.nn.functional as F
    from mask_amd import datasets
    from mask_amd.external_backend_spmm import reset_backend_state, srbcrs_spmm
    from mask_amd.gcn import GCN, graph_from_csr, torch_spmm
    dev = torch.device("cuda", 0)
    m = datasets.make_config("gcn-232965")
    graph = graph_from_csr(m, 512, dev, seed=m.seed)
    labels = torch.randint(0, 64, (m.M,), generator=torch.Generator().manual_seed(m.seed)).to(dev)
    if not args.no_tune:
        os.environ["SPARSENE_SRBCRS_AUTOTUNE"] = "1"   # tuned on each plan's first call per width
    results, losses = {}, {}
    for name in ("16x8", "base", "torch"):
        os.environ["SPARSENE_SRBCRS_VARIANT"] = "16x8" if name == "torch" else name
        reset_backend_state()
        torch.manual_seed(m.seed)
        model = GCN((512, 256, 64), dropout=0.5, spmm=torch_spmm if name == "torch" else srbcrs_spmm,
                    seed=m.seed).to(dev)
        opt = torch.optim.Adam(model.parameters(), lr=0.01)

        def step():
            opt.zero_grad(set_to_none=True)
            loss = F.nll_loss(model(graph), labels)
            loss.backward()
            opt.step()
            return loss

        t0 = time.time()
        step()   # conversion of A and A^T (and tuning) happens here, outside the timed steps
        torch.cuda.synchronize()
        setup_s = time.time() - t0
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        e = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        e[0].record()
        for _ in range(args.steps):
            loss = step()
        e[1].record()
        torch.cuda.synchronize()
        results[name] = {"ms_per_step": round(e[0].elapsed_time(e[1]) / args.steps, 4),
                         "first_step_s": round(setup_s, 3)}
        losses[name] = round(float(loss), 5)
    print(json.dumps({
        "metric": "GCN training step time (gcn-232965, GCN 512-256-64, Adam, full batch)",
        "value": results["16x8"]["ms_per_step"], "unit": "ms", "higher_is_better": False, "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "dtype": "f32",
        "data": "synthetic R-MAT graph, N(0,1) features, uniform labels (seeded)",
        "config": {"workload": m.name, "nodes": m.M, "nnz": m.nnz, "spmm": "srbcrs_spmm drop-in",
                   "autotune": not args.no_tune},
        "variants": results, "final_loss": losses,
    }), flush=True)


def tuned_knobs(t, tune_s):
    return {"depth": t["depth"], "tile_b": t.get("tile_b", 0), "wg_cols": t["wg_cols"], "grid_order": t["grid_order"],
            "windows_per_wave": t["windows_per_wave"], "a_operand": t["a_operand"], "b_stage": t["b_stage"],
            "tuned": True,
            "tune_s": round(tune_s, 3)}


def a_operand_used(plan, requested):
    """The block-value copy the SR-BCRS kernel reads (mirrors the library's
    default: for 16x8 blocks compact when at most half of the block positions
    are stored; 32x32 blocks read the dense array)."""
    if requested != "default":
        return requested
    stored = plan.desc.stored_values
    sparse = stored >= 0 and 2 * stored <= plan.total_blocks * plan.blk_h * plan.blk_w
    return "compact" if sparse and plan.blk_h == 16 else "dense"


def algorithmic_bytes(M, N, Mo, nb, nnz, kernel, bh=16, bw=8):
    """Dataflow bytes per launch.  SR-BCRS: metadata + A blocks + B rows
    gathered per block + C written (for 16x8 blocks: 4(Mo+1) + nb(8*4 +
    128*4) + nb*8*N*4 + M*N*4).  CSR: rowptr + (col, val) + B row per
    nonzero + C."""
    if kernel == "srbcrs":
        return 4 * (Mo + 1) + nb * (bw * 4 + bh * bw * 4) + nb * bw * N * 4 + M * N * 4
    return 4 * (M + 1) + 8 * nnz + 4 * N * nnz + 4 * M * N


# Launch settings the default run uses per workload (16x8 blocks, at N = the entry's "N", else 512).  They are
# the fastest settings of the on-GPU sweeps of srbcrs_plan_tune's candidate set, fixed here so that
# every run times the same kernel instantiation as the committed rocprofv3 profile of that workload;
# --tune times the candidates on the box instead.
PUBLISHED_KNOBS = {
    # the nonzero sweep: one B-row gather per stored value, 8 windows' values per 64-column wave in the
    # merged order, sub-batches of 32 values, 2 in flight
    "uniform-65536": {"depth": 2, "tile_b": 32, "wg_cols": 64, "grid_order": 5, "windows_per_wave": 8,
                      "a_operand": "compact"},
    "banded-524288": {"depth": 2, "wg_cols": 256, "grid_order": 1, "windows_per_wave": 1, "a_operand": "dense"},
    # B staged through LDS by direct-to-LDS loads
    "rmat-2^20": {"depth": 4, "wg_cols": 64, "grid_order": 3, "windows_per_wave": 1, "a_operand": "compact",
                  "b_stage": "lds"},
    # GCN aggregation at the workload's own width (N = 256), split schedule; depth 4 (1.517 ms
    # sustained against 1.595 at depth 2 and 1.521 with the LDS ring, interleaved on one box)
    "gcn-232965": {"N": 256, "depth": 4, "wg_cols": 64, "grid_order": 3, "windows_per_wave": 1, "a_operand": "compact"},
}
# What bounds each workload, from the measurements under profiles/: banded moves its compulsory
# bytes through HBM at 61 % memory-controller activity (umc_activity_*.md); the others run far below
# the HBM rate, bound by the gathers' requests out of the L2 (most served by the memory-side cache).
BOUND = {"banded-524288": "hbm", "uniform-65536": "l2-miss gather path", "rmat-2^20": "l2-miss gather path",
         "gcn-232965": "l2-miss gather path"}
NZSWEEP = 5   # grid order of the nonzero sweep
# the other large configurations (banded: the second north-star target; R-MAT and the GCN
# aggregation at N = 256), measured in the same invocation as the headline
EXTRA_CONFIGS = ("banded-524288", "rmat-2^20", "gcn-232965")
# ... and BASELINE config 5 as stated: the GCN workload's whole two-layer forward
GCN_FORWARD = "gcn-232965-forward"
# Each extra configuration warms for at least this long before its K timed steps (its "warmup"
# field gives the count): banded's clock boosts, dips and settles within the first ~20 ms of a
# new load, and K = 20 steps right after 5 warm-up steps land inside that dip.
EXTRA_SETTLE_S = 1.0


def window_sharing(args):
    """How many B-row gathers neighbouring row windows share (host only):
    the number of distinct (row // h, column) pairs of the workload for
    window heights h = 16 .. 256, against h = 16 (the SR-BCRS window, one
    gather per pair and column chunk).  One JSON line."""
    from mask_amd import datasets
    m = datasets.make_config(args.config)
    rows = np.repeat(np.arange(m.M, dtype=np.int64), np.diff(m.rowptr))
    cols = m.colind.astype(np.int64)
    out = {h: int(np.unique((rows // h) * (1 << 21) + cols).size) for h in (16, 32, 64, 128, 256)}
    print(json.dumps({"workload": m.name, "nnz": m.nnz, "distinct_pairs": out,
                      "ratio_to_16": {h: round(v / out[16], 4) for h, v in out.items()}}), flush=True)


def main():
    args = parse()
    if args.window_sharing:
        window_sharing(args)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(json.dumps({"error": "this benchmark measures one GPU; --gpus must be 1 "
                                   "(the SpMM path is single-GPU, sharding is design-only)"}))
        sys.exit(2)

    if args.copy_calibration_mb:
        copy_calibration(args.copy_calibration_mb, args.copy_seconds)
        return
    if args.gcn_train:
        gcn_train_bench(args)
        return
    if args.shard_sim > 1:
        shard_sim_bench(args)
        return
    if args.gcn_forward:
        gcn_forward_bench(args)
        return
    if args.gather_study:
        gather_study(args)
        return
    if args.sweep_crossover:
        sweep_crossover(args)
        return

    if args.umc_seconds > 0:
        umc_measure(args)
        return
    probes_out = {}

    def run_probes():
        # the stream and gather probes run after the workload's set-up, right
        # before its W warm-up steps: the GPU then enters the timed steps from
        # load, not from the idle time of the host-side generation and conversion
        probes_out["streams"] = copy_bandwidth()
        probes_out["ceiling"] = gather_ceiling()
        return probes_out["ceiling"]

    result = measure(args, args.config, mtx=args.mtx, before_warmup=None if args.lean else run_probes)
    ceiling = probes_out.get("ceiling")
    if not args.lean:
        result["roofline"]["stream_gbs"] = probes_out["streams"]
        result["roofline"]["gather_ceiling"] = ceiling
    default_run = (args.config == "uniform-65536" and not args.mtx and not args.extra_off and args.N in (None, 512)
                   and not explicit_knobs(args)
                   and args.kernel == "srbcrs" and args.blk == "16x8" and args.row_order == "identity")
    if default_run:
        result["extra_configs"] = {}
        for name in EXTRA_CONFIGS:
            extra = measure(args, name, cpu_seconds=max(3.0, args.cpu_seconds / 2), settle_s=EXTRA_SETTLE_S,
                            ceiling=ceiling)
            result["extra_configs"][name] = {k: extra[k] for k in (
                "value", "unit", "steps", "warmup", "ms_per_step", "ms_per_step_median", "config", "roofline",
                "sustained", "library_tuned", "parity", "cpu_baseline") if k in extra}
        result["extra_configs"][GCN_FORWARD] = gcn_forward_measure(args, ceiling, settle_s=EXTRA_SETTLE_S)
    print(json.dumps(result), flush=True)


def explicit_knobs(args):
    return bool(args.depth or args.tile_b or args.wg_cols or args.grid_order or args.wpw
                or args.a_operand != "default" or args.b_stage != "default")


def measure(args, config, mtx=None, cpu_seconds=None, settle_s=0.0, ceiling=None, before_warmup=None):
    """Time one workload (K steps after W warm-up steps, HIP events on the
    launch stream), check it against the oracle on a row sample and time the
    CPU baseline.  Returns the result dict."""
    import torch
    from mask_amd import datasets
    from mask_amd.SRBCRSSpMM import Plan, csr_spmm

    dev = torch.device("cuda", 0)
    t0 = time.time()
    m = datasets.from_mtx(mtx, N=args.N or 512) if mtx else datasets.make_config(config)
    N = args.N or m.N
    B_host = m.dense(N)
    print(f"[bench] workload {m.name} M={m.M} K={m.K} nnz={m.nnz} N={N} gen {time.time() - t0:.1f}s",
          file=sys.stderr, flush=True)

    rowptr_d = torch.from_numpy(m.rowptr).to(dev)
    colind_d = torch.from_numpy(m.colind).to(dev)
    values_d = torch.from_numpy(m.values).to(dev)
    B = torch.from_numpy(B_host).to(dev)
    C = torch.empty((m.M, N), dtype=torch.float32, device=dev)

    t0 = time.time()
    bh, bw = (int(x) for x in args.blk.split("x"))
    plan = Plan(rowptr_d, colind_d, values_d, m.M, bh, bw, row_order=args.row_order, K=m.K)
    conv_s = time.time() - t0
    nb, Mo = plan.total_blocks, plan.row_windows
    sched = args.schedule
    if sched == "auto":
        lens = np.diff(np.asarray(datasets_soff(plan)))
        sched = "split" if lens.size and lens.max() > max(64, 4 * max(1, int(np.percentile(lens, 95)))) else "row"
    name, _, param = sched.partition(":")
    plan.set_schedule(name, int(param) if param else 0)
    max_col = plan.max_col

    knob_args = {"depth": args.depth, "tile_b": args.tile_b, "wg_cols": args.wg_cols, "grid_order": args.grid_order,
                 "windows_per_wave": args.wpw, "a_operand": args.a_operand, "b_stage": args.b_stage}
    tuned, tune_s, knobs = None, 0.0, None
    if args.kernel == "srbcrs" and not explicit_knobs(args):
        if args.tune:
            t0 = time.time()
            tuned = plan.tune(B, C, nonzero_sweep=True)   # outside the timed region, like the conversion
            torch.cuda.synchronize()
            tune_s = time.time() - t0
            knobs = tuned_knobs(tuned, tune_s)
        elif (m.name in PUBLISHED_KNOBS and N == PUBLISHED_KNOBS[m.name].get("N", 512) and args.blk == "16x8"
              and args.row_order == "identity" and not mtx):
            knob_args.update({k: v for k, v in PUBLISHED_KNOBS[m.name].items() if k != "N"})
            knobs = {"depth": knob_args["depth"], "tile_b": knob_args["tile_b"], "wg_cols": knob_args["wg_cols"],
                     "grid_order": knob_args["grid_order"], "windows_per_wave": knob_args["windows_per_wave"],
                     "a_operand": knob_args["a_operand"],
                     "b_stage": "lds" if knob_args["b_stage"] == "lds" else "registers", "tuned": False,
                     "source": "bench.PUBLISHED_KNOBS"}
    if args.kernel == "srbcrs":
        step = lambda: plan.run(B, C, **knob_args)
    else:
        step = lambda: csr_spmm(rowptr_d, colind_d, values_d, B, m.M, max_col=max_col, out=C)

    n_warm = args.warmup
    if before_warmup is not None and n_warm > 0:
        # the first warm-up step prepares what the plan builds on first use
        # (the merged-window stream), then the probes run, then the rest
        step()
        torch.cuda.synchronize()
        n_warm -= 1
        ceiling = before_warmup()
    for _ in range(n_warm):
        step()
    torch.cuda.synchronize()
    warmup_done = args.warmup
    if settle_s > 0:
        # extra configurations only: keep warming until about settle_s of
        # back-to-back steps has run, so that the timed steps fall after the
        # clock's reaction to the new load, not inside it
        t_set = time.perf_counter()
        while time.perf_counter() - t_set < settle_s:
            for _ in range(10):
                step()
            warmup_done += 10
            torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    # The K timed steps run back to back between two events: a timing event
    # recorded between two steps waits for the first to drain before the
    # second starts, which would add a bubble per step to the timed region.
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    ev0.record(stream)
    for i in range(args.steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    total_ms = ev0.elapsed_time(ev1)
    ms_step = total_ms / args.steps
    # per-step times for the median: a separate pass of K steps, each between its own events
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    evs[0].record(stream)
    for i in range(args.steps):
        step()
        evs[i + 1].record(stream)
    torch.cuda.synchronize()
    per = np.array([evs[i].elapsed_time(evs[i + 1]) for i in range(args.steps)])  # ms
    t_s = ms_step / 1e3
    flops = 2.0 * m.nnz * N
    gflops = flops / t_s / 1e9

    if knobs is None:
        knobs = {"depth": args.depth or 2, "tile_b": args.tile_b, "wg_cols": args.wg_cols or 128,
                 "grid_order": args.grid_order or 1, "windows_per_wave": args.wpw or 1,
                 "a_operand": a_operand_used(plan, args.a_operand),
                 "b_stage": "lds" if args.b_stage == "lds" else "registers", "tuned": False}
    # the nonzero sweep reads (column, value) pairs and gathers one B row per value, as CSR does, and
    # does no MFMA work; the MFMA kernels read the blocks and gather BW rows per block
    vector = args.kernel == "csr" or knob_args.get("grid_order") == NZSWEEP
    ab = algorithmic_bytes(m.M, N, Mo, nb, m.nnz, "csr" if vector else "srbcrs", bh, bw)
    compulsory = (8 * m.nnz if vector else nb * (bw * 4 + bh * bw * 4) + 4 * (Mo + 1)) + m.K * N * 4 + m.M * N * 4
    padded_flops = 0.0 if vector else 2.0 * bh * bw * nb * N
    prof = None
    if args.kernel == "srbcrs" and args.schedule == "auto" and not args.tile_b and args.row_order == "identity" \
            and not mtx:
        prof = measured_profile(m.name, N, args.kernel, knobs, args.blk)

    sustained = None
    if args.sustained_s > 0:
        # The clock settles only after the power management has reacted to
        # the load (banded: boost, a dip, then a steady level), which a short
        # K-step window can catch anywhere; this times the steady rate apart.
        n_s = int(min(100000, max(args.steps, np.ceil(args.sustained_s * 1e3 / max(ms_step, 1e-3)))))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(n_s):
            step()
        e1.record(stream)
        torch.cuda.synchronize()
        ms_s = e0.elapsed_time(e1) / n_s
        rs = roofline(ms_s / 1e3, ab, compulsory, padded_flops, prof, BOUND.get(m.name, "hbm"), ceiling)
        sustained = {"steps": n_s, "seconds": round(ms_s * n_s / 1e3, 3), "ms_per_step": round(ms_s, 5),
                     "value": round(flops / (ms_s / 1e3) / 1e9, 2), "frac": rs["frac"],
                     "hbm_frac": rs["hbm_frac"]}
        if "gather_frac" in rs:
            sustained["gather_frac"] = rs["gather_frac"]

    result = {
        "metric": "SpMM GFLOP/s at N=512 fp32 on 1 MI355X; % of HBM roofline",
        "value": round(gflops, 2),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": warmup_done,
        "ms_per_step": round(ms_step, 5),
        "ms_per_step_median": round(float(np.median(per)), 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded numpy, see mask_amd/datasets.py)",
        "config": {"workload": m.name, "M": m.M, "K": m.K, "N": N, "nnz": m.nnz, "blocks": nb,
                   "block": args.blk, "block_fill": round(m.nnz / (bh * bw * max(nb, 1)), 4),
                   "kernel": args.kernel,
                   "schedule": f"{plan.policy[0]}:{plan.policy[1]}", "seed": m.seed, "row_order": args.row_order,
                   "conversion_s": round(conv_s, 3), "meta": m.meta,
                   "knobs": knobs},
        "roofline": roofline(t_s, ab, compulsory, padded_flops, prof, BOUND.get(m.name, "hbm"), ceiling),
        "wall_s_timed": round(wall, 4),
    }
    if sustained is not None:
        result["sustained"] = sustained

    if knobs.get("source") == "bench.PUBLISHED_KNOBS" and not args.lean:
        # beside the published setting: what the library picks for itself on
        # this plan (srbcrs_plan_tune_ex with the nonzero sweep admitted: the
        # drop-in's autotune under SPARSENE_ALLOW_CSR_FALLBACK=1), timed the same way
        t0 = time.time()
        tk = plan.tune(B, C, nonzero_sweep=True)
        torch.cuda.synchronize()
        tune_s = time.time() - t0
        ms_t = _time_ms(lambda: plan.run(B, C), args.steps, args.warmup)
        same = all(str(tk[k]) == str(knobs[k]) for k in ("depth", "wg_cols", "grid_order", "windows_per_wave",
                                                          "a_operand", "b_stage")) \
            and (tk["grid_order"] != NZSWEEP or tk["tile_b"] == knobs.get("tile_b"))
        result["library_tuned"] = {"knobs": tk, "tune_s": round(tune_s, 3), "ms_per_step": round(ms_t, 5),
                                   "value": round(flops / (ms_t / 1e3) / 1e9, 2), "same_as_published": same}

    budget = args.cpu_seconds if cpu_seconds is None else cpu_seconds
    if not (args.no_check and args.no_cpu):
        parity, base = cpu_baseline_leg(m, B_host, N, budget, None if args.no_check else C.cpu().numpy(),
                                        time_baseline=not args.no_cpu)
        if parity is not None:
            result["parity"] = parity
        if base is not None:
            result["cpu_baseline"] = base
    del plan, B, C
    torch.cuda.empty_cache()
    return result


def roofline(t_s, dataflow_bytes, compulsory_bytes, padded_flops, prof, bound="hbm", gather_ceiling=None):
    """The roofline block of a result.

    frac = achieved / peak with achieved = compulsory bytes per step (A as
    stored, B once, C once: the bytes any schedule must move) / step time,
    against the 8 TB/s HBM peak.  Beside it, each from its own source:
      hbm_bytes       bytes that reached HBM, measured at the memory
                      controllers (amd-smi UMC activity) for this launch
                      setting (prof "hbm_bytes_umc"), else the compulsory
                      bytes; hbm_basis names which;
      l2_egress_bytes requests out of the L2 toward the memory side
                      (TCC_EA0_*_DRAM counters, prof "l2_egress_bytes"):
                      memory-side-cache hits included, so never an HBM figure;
      traffic         FETCH_SIZE + WRITE_SIZE of the same profile (also L2
                      egress);
      gather_frac     L2-egress rate / the gather ceiling (random line
                      gathers out of the L2 on the same box, gather_ceiling());
      dataflow_gbs    every gathered B row per block over the step time: a
                      rate only (the L2 serves part of it).
    A compulsory fraction above 1 would mean the byte model is wrong: frac is
    then null and frac_rejected holds it."""
    achieved = compulsory_bytes / t_s / 1e9
    frac = achieved / HBM_PEAK_GBS
    prof = prof or {}
    if prof.get("hbm_bytes_umc"):
        hbm, hbm_basis = prof["hbm_bytes_umc"], f"memory-controller (UMC) activity: {prof['file']}"
    else:
        hbm, hbm_basis = compulsory_bytes, "compulsory bytes (no memory-controller measurement of this setting)"
    out = {"bound": bound, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
           "frac": round(frac, 4) if frac <= 1.0 else None,
           "basis": "compulsory bytes (A as stored + B once + C once) / step time",
           "traffic": prof.get("traffic_bytes"),
           "traffic_basis": ("FETCH_SIZE + WRITE_SIZE, copy-calibrated: bytes leaving the L2, memory-side-cache "
                             f"hits included ({prof['file']})") if prof.get("traffic_bytes") else None,
           "compulsory_bytes": int(compulsory_bytes),
           "hbm_bytes": int(hbm), "hbm_basis": hbm_basis,
           "hbm_frac": round(hbm / t_s / 1e9 / HBM_PEAK_GBS, 4),
           "dataflow_bytes": int(dataflow_bytes), "dataflow_gbs": round(dataflow_bytes / t_s / 1e9, 1),
           "mfma_padded_tflops": round(padded_flops / t_s / 1e12, 3),
           "mfma_frac": round(padded_flops / t_s / 1e12 / FP32_MFMA_PEAK_TFLOPS, 4)}
    if frac > 1.0:
        out["frac_rejected"] = round(frac, 4)
    if prof.get("l2_egress_bytes"):
        eg = prof["l2_egress_bytes"] / t_s / 1e9
        out.update({"l2_egress_bytes": int(prof["l2_egress_bytes"]), "l2_egress_gbs": round(eg, 1),
                    "l2_egress_frac": round(eg / HBM_PEAK_GBS, 4),
                    "l2_egress_basis": f"TCC_EA0_RDREQ_DRAM_32B + TCC_EA0_WRREQ_WRITE_DRAM_32B, copy-calibrated "
                                       f"({prof['file']})"})
        if gather_ceiling:
            c = max(gather_ceiling.values())
            out["gather_ceiling_gbs"] = c
            out["gather_frac"] = round(eg / c, 4)
    if prof.get("kernel_avg_ms"):
        out["profile_kernel_avg_ms"] = prof["kernel_avg_ms"]
    return out


def measured_profile(workload, N, kernel, knobs, blk="16x8"):
    """The committed rocprofv3 summary of this workload whose "knobs:" line
    (block shape included; 16x8 when the line names none) matches the launch
    settings of this run: {"file", "l2_egress_bytes", "traffic_bytes",
    "kernel_avg_ms", "hbm_bytes_umc" (when measured)}, or None when there is
    none or it lacks an l2_egress_bytes line."""
    if kernel != "srbcrs" or knobs is None:
        return None
    want = {k: str(knobs[k]) for k in ("depth", "wg_cols", "grid_order", "windows_per_wave", "a_operand")}
    want["tile_b"] = str(knobs.get("tile_b", 0) or 0)
    want["blk"] = blk
    want["b_stage"] = str(knobs.get("b_stage", "registers"))
    for path in sorted((ROOT / "profiles").glob(f"spmm_*_{workload.replace('^', '')}_N{N}*.md")):
        fields, prof_knobs = {}, None
        for line in path.read_text().splitlines():
            key, _, val = line.partition(":")
            if key in ("traffic_bytes", "l2_egress_bytes", "hbm_bytes_umc"):
                fields[key] = int(val)
            elif key == "kernel_avg_ns":
                fields["kernel_avg_ms"] = round(int(val) / 1e6, 5)
            elif key == "knobs":
                prof_knobs = dict(kv.split("=") for kv in val.split())
        if prof_knobs and {"windows_per_wave": "1", "blk": "16x8", "b_stage": "registers", "tile_b": "0",
                           **prof_knobs} == want \
                and "l2_egress_bytes" in fields:
            return {"file": f"profiles/{path.name}", "traffic_bytes": fields.get("traffic_bytes"), **fields}
    return None


def datasets_soff(plan):
    import torch
    n = plan.row_windows + 1
    t = torch.empty(n, dtype=torch.int32, device=plan.device)
    from mask_amd import _capi
    _capi.check(_capi.lib().srbcrs_plan_export_index(plan.handle, t.data_ptr(), n, None, 0,
                                                     torch.cuda.current_stream(plan.device).cuda_stream))
    return t.cpu().numpy()


def _row_sample(m, rows):
    rp = m.rowptr
    counts = rp[rows + 1] - rp[rows]
    sub_rp = np.zeros(rows.size + 1, np.int64)
    sub_rp[1:] = np.cumsum(counts)
    idx = np.concatenate([np.arange(rp[r], rp[r + 1]) for r in rows]) if rows.size else np.zeros(0, np.int64)
    return sub_rp.astype(np.int32), m.colind[idx], m.values[idx]


def _check_sample(oracle, m, B_host, C, n_rows=4096):
    """Correctness gate on a seeded row sample against the fp64 oracle."""
    rng = np.random.default_rng(0)
    rows = np.sort(rng.choice(m.M, size=min(n_rows, m.M), replace=False))
    rp, ci, vv = _row_sample(m, rows)
    C64, absAB = oracle.csr_spmm_f64(rp, ci, vv, B_host, rows.size, with_abs=True)
    met = oracle.error_metrics(C[rows], C64, absAB)
    met["rows_checked"] = int(rows.size)
    met["pass"] = bool(met["finite"] and met["max_ratio"] <= 1e-4 and met["ref_gate"])
    return met


def parity_leg(m, B_host, C):
    """The correctness gate of one SpMM result C (host array, all rows) with
    dense input B_host against the fp64 oracle on a seeded row sample (the
    CPU leg's checker, for results that have no CPU-baseline timing)."""
    from oracle import oracle
    return _check_sample(oracle, m, B_host, C)


def cpu_baseline_leg(m, B_host, N, budget_s, C=None, time_baseline=True):
    """The CPU leg: the only place bench.py touches oracle/.  Returns
    (parity, cpu_baseline): the fp64 oracle as the checker of the GPU result
    C on a seeded row sample (None when C is None), and the timed CPU
    baseline (None unless time_baseline)."""
    from oracle import oracle
    parity = _check_sample(oracle, m, B_host, C) if C is not None else None
    return parity, (cpu_baseline(oracle, m, B_host, N, budget_s) if time_baseline else None)


def cpu_baseline(oracle, m, B_host, N, budget_s):
    """The oracle's fp32 CSR SpMM (csr_spmm_value_kernel's arithmetic) on the
    host cores over a bounded row sample, repeated within the time budget."""
    cores = len(os.sched_getaffinity(0))
    # sample sized for ~1 s per repetition at ~1 GFLOP/s per core
    target_flops = 1e9 * cores
    rows_needed = int(target_flops / max(1.0, 2.0 * N * m.nnz / m.M))
    rows = np.arange(min(m.M, max(16, rows_needed)))
    rp, ci, vv = _row_sample(m, rows)
    oracle.csr_spmm_f32(rp, ci, vv, B_host, rows.size, nthreads=cores)  # warmup
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t = time.perf_counter()
        oracle.csr_spmm_f32(rp, ci, vv, B_host, rows.size, nthreads=cores)
        times.append(time.perf_counter() - t)
        if len(times) >= 5000:   # the time budget governs; this only bounds tiny samples
            break
    t_med = float(np.median(times))
    nnz_s = int(rp[-1])
    flops = 2.0 * nnz_s * N
    # beside the baseline, on the same sample: the fp64 oracle (the checker, one run) and CPU
    # torch.sparse.mm (the reference's torch fallback, external_backend_spmm.py:115-124)
    t = time.perf_counter()
    oracle.csr_spmm_f64(rp, ci, vv, B_host, rows.size)
    t_f64 = time.perf_counter() - t
    import torch
    import warnings
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")   # "sparse CSR support is in beta"
        A = torch.sparse_csr_tensor(torch.from_numpy(rp.astype(np.int64)), torch.from_numpy(ci.astype(np.int64)),
                                    torch.from_numpy(vv), size=(rows.size, B_host.shape[0]))
    Bt = torch.from_numpy(B_host)
    torch.sparse.mm(A, Bt)
    tt = []
    for _ in range(3):
        t = time.perf_counter()
        torch.sparse.mm(A, Bt)
        tt.append(time.perf_counter() - t)
    t_torch = float(np.median(tt))
    return {"value": round(flops / t_med / 1e9, 3), "unit": "GFLOP/s", "cores": cores, "kind": "port",
            "sample": f"first {rows.size} rows ({nnz_s} nnz) of {m.name} at N={N}, median of {len(times)} runs, "
                      f"fp32 row-parallel CSR (oracle/srbcrs_oracle.c)",
            "median_s": round(t_med, 5),
            "oracle_f64_s": round(t_f64, 5),
            "torch_sparse_cpu": {"value": round(flops / t_torch / 1e9, 3), "unit": "GFLOP/s",
                                 "threads": torch.get_num_threads(), "median_s": round(t_torch, 5)}}


if __name__ == "__main__":
    main()
