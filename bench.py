#!/usr/bin/env python3
"""Benchmark of the MI355X proximity hot path (one GPU).

Workload (the headline configuration, C3): N=100,000
samples, T=500 trees, int32 leaf ids drawn uniformly from 2,048 leaves per
tree, OOB bits Bernoulli(0.368) iid; output = the uint8-quantized normalised
OOB proximity upper triangle (N(N+1)/2 = 5,000,050,000 bytes) with the
reference quantizer's min/max rule for min 0, max 1: scale = (1-0)/255,
zp = -0/scale.  One step = rfxp_set_forest (bucket index over all trees)
+ rfxp_upper (counting + normalise + quantize + store) from device-resident
inputs to the completed device output.

Metric: pair-tree comparisons per second = C(N,2)*T / step time.
Prints one JSON line (see the driver contract).  `--gpus N` with N > 1
exits: this build runs on one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "rfx-fuse_amd"))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published

CONFIGS = {
    "c3": dict(workload="C3 quantized uint8 upper triangle", n=100_000, t=500, nleaf=2048,
               leaves=(2048, 2048), p_oob=0.368, fmt="u8", seed=20261201 + 3),
    # mid-size fp32 triangle (C2): a measurement case
    "c2": dict(workload="C2 fp32 upper triangle", n=20_000, t=500, nleaf=4096,
               leaves=(1000, 4096), p_oob=0.368, fmt="f32", seed=20261201 + 2),
    # top-K retrieval of new queries over all trees (C5): a parity/measurement case,
    # not the driver's bench line
    "c5": dict(workload="C5 top-K retrieval", n=1_000_000, q=100_000, t=500, nleaf=2048, k=20,
               seed=20261201 + 5),
    # low-rank one-hot SpMM and subspace iteration (C4): measurement case
    "c4": dict(workload="C4 low-rank P V and rank-32 subspace iteration", n=1_000_000, t=500, nleaf=4096,
               r=32, iters=5, zipf=1.1, seed=20261201 + 4),
    # the reference's live GPU low-rank sequence (growtree: per tree an FP16
    # triangle + the class's incremental add, then finalize), at the size of
    # the reference README's largest GPU run (59,047 samples), 100 of its
    # 1,000 trees; opt-in (--config cs2), not part of the default run
    "cs2": dict(workload="CS2 growtree low-rank class sequence", n=59_047, t=100, nleaf=2000, level=1,
                seed=20261201 + 6),
}

# Kernel sources whose rocprofv3 traffic summary (profiles/k_tri_<cfg>_traffic.md)
# stays valid only as long as they are unchanged.
TRI_SOURCES = ("rfx-fuse_amd/csrc/rfxp_triangle.hip", "rfx-fuse_amd/csrc/rfxp_pack.hip",
               "rfx-fuse_amd/csrc/rfxp_forest.hpp", "rfx-fuse_amd/csrc/rfxp_device.hpp")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default=None, choices=sorted(CONFIGS),
                    help="one config only; by default C3 is the bench line and C2, C5, C4 are added "
                         "to it as sub-records")
    ap.add_argument("--no-sub", action="store_true", help="default run without the C2/C5/C4 sub-records")
    ap.add_argument("--n", type=int, default=None, help="override N (smaller smoke runs)")
    ap.add_argument("--q", type=int, default=None, help="override the query count (c5)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=16.0,
                    help="target CPU time of the bounded CPU-baseline sample")
    ap.add_argument("--calibrate", action="store_true",
                    help="only time the triangle's two traffic streams on synthetic data of its shape: "
                         "random run gathers, the N(N+1)/2-byte streaming store, each alone and both in "
                         "one kernel (rfx-fuse_amd/calib/rfxc_calib.hip)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB a few times (the reference "
                         "point that scales rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes)")
    return ap.parse_args()


def kernel_source_sha(paths=TRI_SOURCES):
    """SHA-256 (first 16 hex digits) of the kernel sources, in order."""
    import hashlib

    h = hashlib.sha256()
    for p in paths:
        with open(os.path.join(REPO, p), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def traffic_from_profile(config):
    """HBM bytes per triangle launch measured with rocprofv3 --pmc FETCH_SIZE
    and WRITE_SIZE (each scaled by the copy-kernel calibration), read from the
    committed summary profiles/k_tri_<config>_traffic.md.  None when the file
    is absent or was measured on other kernel sources than the ones built
    now (its `kernel_source_sha` line differs)."""
    path = os.path.join(REPO, "profiles", f"k_tri_{config}_traffic.md")
    vals = {}
    try:
        with open(path) as f:
            for line in f:
                line = line.strip().strip("`")
                for key in ("traffic_bytes_per_launch", "kernel_source_sha"):
                    if line.startswith(key) and "=" in line:
                        vals[key] = line.split("=", 1)[1].strip().strip("`")
    except OSError:
        return None
    if vals.get("kernel_source_sha") != kernel_source_sha() or "traffic_bytes_per_launch" not in vals:
        return None
    return float(vals["traffic_bytes_per_launch"])


def host_cpu():
    """(CPU model, logical CPUs of the host, threads this process may use).
    The threads are the OpenMP setting of the environment (on the GPU box:
    the CPU share granted to one GPU), else every CPU of the host."""
    model, ncpu = "unknown", os.cpu_count() or 1
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or ncpu
    except ValueError:
        threads = ncpu
    return model, ncpu, max(1, min(threads, ncpu))


def copy_calibration(mib):
    import torch

    n = mib * (1 << 20)
    src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n, "launches": 5}), flush=True)


def calibrate(args):
    """Floor of the bucketed triangle's traffic on this GPU.  Synthetic
    records of C3's shape (N rows, T random runs of 0..24 ids per row, ids
    at uniform places of an id array), one workgroup per row as in k_tri:
      gather  -- records, run loads and LDS counting, no output;
      store   -- the N(N+1)/2-byte triangle streamed from LDS, no run loads;
      both    -- both in one kernel, in k_tri's order.
    The id array's size is swept to show where the runs are served from
    (L2: a few MB; Infinity Cache: up to 256 MB; HBM beyond).  Times are HIP
    events around single launches on one stream (median of 5)."""
    import ctypes as C
    import statistics

    import torch

    lib = C.CDLL(os.path.join(REPO, "rfx-fuse_amd", "lib", "librfxcalib.so"))
    vp, i64, i32 = C.c_void_p, C.c_int64, C.c_int32
    lib.rfxc_setup.argtypes = [vp, i64, C.c_int, vp, vp, i64, i32, i64, C.c_uint32, vp]
    lib.rfxc_run.argtypes = [C.c_int, C.c_int, vp, vp, vp, i64, i32, i64, vp, vp, vp]
    cfg = CONFIGS["c3"]
    n = args.n or cfg["n"]
    t = cfg["t"]
    ldr = (t + 15) // 16 * 16
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream().cuda_stream
    roff = torch.empty(n * ldr, dtype=torch.int32, device=dev)
    rlen = torch.empty(n * ldr, dtype=torch.int16, device=dev)
    out = torch.empty(n * (n + 1) // 2, dtype=torch.uint8, device=dev)
    sink = torch.empty(n, dtype=torch.int32, device=dev)
    runs = n * t
    res = {"workload": "calibration of the C3 triangle's traffic", "N": n, "T": t, "runs": runs,
           "store_bytes": n * (n + 1) // 2, "cases": []}

    def timed(mode, idb, mem):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ms = []
        for k in range(7):
            ev[0].record()
            rc = lib.rfxc_run(mode, idb, mem.data_ptr(), roff.data_ptr(), rlen.data_ptr(), ldr, t, n,
                              out.data_ptr(), sink.data_ptr(), stream)
            ev[1].record()
            torch.cuda.synchronize()
            if rc != 0:
                raise RuntimeError(f"rfxc_run mode {mode} idb {idb}: hip error {rc}")
            if k >= 2:
                ms.append(ev[0].elapsed_time(ev[1]))
        return statistics.median(ms)

    # mode bits: 1 gather, 2 store, 4 records by one vector load per group
    # (else by scalar loads)
    for idb, mem_mb, modes in ((4, 200, (2, 1, 3, 5, 7)), (4, 2, (5, 7)), (4, 32, (5,)), (4, 1024, (5, 7)),
                               (2, 100, (5, 7))):
        mem_bytes = mem_mb << 20
        mem = torch.empty(mem_bytes + 4096, dtype=torch.uint8, device=dev)
        rc = lib.rfxc_setup(mem.data_ptr(), mem_bytes, idb, roff.data_ptr(), rlen.data_ptr(), n, t, ldr, 7, stream)
        torch.cuda.synchronize()
        if rc != 0:
            raise RuntimeError(f"rfxc_setup: hip error {rc}")
        for mode in modes:
            ms = timed(mode, idb, mem)
            case = {"kind": {1: "gather", 2: "store", 3: "both"}[mode & 3], "id_bytes": idb, "id_array_MB": mem_mb,
                    "records": "vector" if mode & 4 else "scalar", "ms": ms}
            if mode & 1:
                case["runs_per_s"] = runs / (ms / 1e3)
            if mode & 2:
                case["store_GBps"] = n * (n + 1) // 2 / (ms / 1e3) / 1e9
            res["cases"].append(case)
            print(json.dumps(case), flush=True)
        del mem
    print(json.dumps(res), flush=True)


def make_inputs(cfg, n, device):
    """Seeded synthetic forest on the device: per tree a leaf count L_t drawn
    from cfg["leaves"] (inclusive), labels uniform on [0, L_t), OOB bits
    Bernoulli(p_oob) iid."""
    import torch

    import rfxprox as R

    g = torch.Generator(device=device)
    g.manual_seed(cfg["seed"])
    t = cfg["t"]
    lo, hi = cfg["leaves"]
    if lo == hi:
        leaf = torch.randint(0, lo, (t, n), generator=g, device=device, dtype=torch.int32)
    else:
        lt = torch.randint(lo, hi + 1, (t, 1), generator=g, device=device, dtype=torch.int64)
        leaf = (torch.rand((t, n), generator=g, device=device, dtype=torch.float64) * lt).to(torch.int32)
    oob = torch.rand((t, n), generator=g, device=device) < cfg["p_oob"]
    words = R.pack_oob_bits(oob)
    return leaf, oob, words


def _rows_rate(idx, O, fmt, n, scale, zp, target_s, threads, seed, chunk=16):
    """Pairs per second of the oracle's row pass on random chunks of rows
    until ~target_s of wall time is spent."""
    import numpy as np

    rng = np.random.default_rng(seed)
    pairs_done, t_rows, nchunk = 0, 0.0, 0
    while t_rows < target_s and nchunk < n // chunk:
        r0 = int(rng.integers(0, n - chunk))
        t0 = time.perf_counter()
        idx.rows(fmt, r0, r0 + chunk, scale, zp, threads=threads)
        t_rows += time.perf_counter() - t0
        pairs_done += sum(n - 1 - i for i in range(r0, r0 + chunk))
        nchunk += 1
    return pairs_done / t_rows, nchunk, pairs_done, t_rows


def cpu_baseline(cfg, leaf_tn, oob_tn, n, fmt, scale, zp, target_s):
    """The oracle (our OpenMP C restatement of the reference algorithm:
    per-tree leaf bucketing, OOB x in-bag co-occurrence, finishprox
    normalisation, quantize) on bounded samples of rows, extrapolated to the
    whole triangle, on the GPU box's host cores.  Three runs on every thread
    this process may use (median reported), then one single-thread run."""
    import statistics

    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O

    t = cfg["t"]
    model, ncpu, threads = host_cpu()
    ofmt = {"u8": O.FMT_U8, "f32": O.FMT_F32}[fmt]
    # bucketing of all trees is paid once per triangle
    t0 = time.perf_counter()
    idx = O.RowIndex(leaf_tn, oob_tn, cfg["nleaf"], threads=threads)
    t_bucket = time.perf_counter() - t0
    total_pairs = n * (n - 1) // 2
    per_run = target_s / 4.0
    runs = []
    for k in range(3):
        rate, nchunk, pairs, secs = _rows_rate(idx, O, ofmt, n, scale, zp, per_run, threads, cfg["seed"] + k)
        runs.append((rate, nchunk, pairs, secs))
    rate1, nchunk1, pairs1, secs1 = _rows_rate(idx, O, ofmt, n, scale, zp, per_run, 1, cfg["seed"] + 9)
    idx.close()
    med = statistics.median(r[0] for r in runs)
    est_s = t_bucket + total_pairs / med
    est1_s = t_bucket * threads + total_pairs / rate1
    return {
        "value": total_pairs * t / est_s,
        "unit": "pair-tree comparisons/s",
        "cores": threads,
        "kind": "port",
        "cpu_model": model,
        "host_cpus": ncpu,
        "single_thread_value": total_pairs * t / est1_s,
        "runs": [total_pairs * t / (t_bucket + total_pairs / r[0]) for r in runs],
        "sample": (f"median of 3 runs on {threads} threads, each {runs[0][1]}-{max(r[1] for r in runs)} "
                   f"chunks of 16 rows at random offsets (~{per_run:.0f} s each), plus one full bucketing "
                   f"pass ({t_bucket:.2f} s), extrapolated to the full triangle; single thread: "
                   f"{nchunk1} chunks ({secs1:.1f} s)"),
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs the proximity path on one GPU; "
                                   f"--gpus {args.gpus} is not supported (multi-GPU sharding is "
                                   "a design note only)"}))
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.calibrate:
        calibrate(args)
        return
    name = args.config or "c3"
    rec = RUNNERS[name](args, name)
    if args.config is None and not args.no_sub:
        rec["sub_records"] = sub_records(args)
    print(json.dumps(rec), flush=True)


def sub_records(args):
    """C2, C5 and C4 measured in the same process after the C3 line, at
    their full sizes, with the same step counts.  A failure in one of them
    is reported in its record and never stops the others or the C3 line."""
    import copy
    import gc

    import torch

    out = {}
    for name in ("c2", "c5", "c4"):
        sub = copy.copy(args)
        sub.n = sub.q = None
        try:
            gc.collect()
            torch.cuda.empty_cache()
            out[name] = RUNNERS[name](sub, name)
        except Exception as e:  # reported, not raised: the C3 line must still print
            out[name] = {"config": CONFIGS[name]["workload"], "error": f"{type(e).__name__}: {e}"}
    return out


def run_triangle(args, name):
    """C3 (default) and C2: one step = rfxp_set_forest (bucket index over all
    trees) + rfxp_upper (counting, normalisation, quantisation, stores).
    Returns the record."""
    import torch

    import rfxprox as R

    cfg = CONFIGS[name]
    n = args.n or cfg["n"]
    t = cfg["t"]
    dev = torch.device("cuda:0")
    torch.cuda.init()
    leaf, oob, words = make_inputs(cfg, n, dev)
    fmt = cfg["fmt"]
    if fmt == "u8":
        scale = float(torch.tensor(1.0, dtype=torch.float32) / 255.0)      # (max-min)/255
        zp = float(-torch.tensor(0.0, dtype=torch.float32) / scale)         # -min/scale
    else:
        scale, zp = 1.0, 0.0
    rfmt = R.FMT_NAMES[fmt]
    esz = {"u8": 1, "f32": 4}[fmt]
    nbytes = R.upper_nbytes(rfmt, n)
    out = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    ctx = R.Context(0)
    ctx.use_torch_stream()

    def step():
        ctx.set_forest(leaf, words, n, t, cfg["nleaf"])
        ctx.upper(rfmt, out, 0, n, scale=scale, zp=zp)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ctx.set_timing(True)
    ctx.reset_timing()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_step = ev0.elapsed_time(ev1) / args.steps
    tri_ms, tri_n = ctx.kernel_time("tri")
    pack_names = ("rr_init", "pack_hist", "pack_scan", "pack_scatter", "records", "nout_final")
    pack_each = {k: ctx.kernel_time(k)[0] / args.steps for k in pack_names}
    pack_ms = sum(pack_each.values()) * args.steps
    tri_avg = tri_ms / max(tri_n, 1)
    pairs = n * (n - 1) // 2
    value = pairs * t / (ms_step / 1e3)
    # algorithmic bytes of one triangle launch: the output entries written
    # + 6 B per (sample, tree) record slot read (4 B offset, 2 B length; rows
    # padded to ldr = T rounded up to 16) + 8 B per sample of 1/nout
    ldr = (t + 15) // 16 * 16
    tri_bytes = nbytes + n * ldr * 6 + n * 8
    achieved = tri_bytes / (tri_avg / 1e3) / 1e9
    # compulsory HBM bytes of the step: the output once, the int32 leaf
    # matrix, the OOB bits and nout once each
    compulsory = nbytes + n * t * 4 + n * t // 8 + n * 4
    rec = {
        "metric": f"pair-tree comparisons/sec at N={n // 1000}k,T={t} ({fmt} OOB proximity triangle)",
        "value": value,
        "unit": "pair-tree comparisons/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": fmt,
        "data": (f"synthetic ({cfg['leaves'][0]}-{cfg['leaves'][1]} uniform leaves per tree, "
                 f"Bernoulli({cfg['p_oob']}) OOB, seeded)"),
        "config": {"workload": cfg["workload"], "N": n, "T": t, "leaves_per_tree": list(cfg["leaves"]),
                   "output_bytes": nbytes, "format": fmt, "scale": scale, "zp": zp},
        "output_GBps": nbytes / (ms_step / 1e3) / 1e9,
        "kernels_ms": {"tri_avg": tri_avg, "pack_per_step": pack_ms / args.steps,
                       **{f"{k}_per_step": v for k, v in pack_each.items()}},
        # row segments the last step recounted with 16-bit counters (wrapped 8-bit counts)
        "tri_recounts": ctx.upper_recounts(),
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "alg_bytes_per_launch": tri_bytes,
                     "traffic": traffic_from_profile(name) if n == cfg["n"] else None,
                     "kernel_source_sha": kernel_source_sha(),
                     # the same against the config's compulsory bytes: the triangle
                     # kernel alone, and the whole timed step (packing included)
                     "compulsory_bytes": compulsory,
                     "frac_compulsory_kernel": compulsory / (tri_avg / 1e3) / 1e9 / HBM_PEAK_GBS,
                     "frac_compulsory_step": compulsory / (ms_step / 1e3) / 1e9 / HBM_PEAK_GBS},
        "wall_s": wall,
    }
    ctx.set_timing(False)
    if fmt == "u8":
        # the reference quantizer rule on this forest's data, outside the
        # timed region: min and max of the fp32 triangle (rfxp_upper_minmax)
        # and the scale / zero point they give, against the ones used above
        try:
            mn, mx = ctx.upper_minmax()
            dscale, dzp = R.quant_scale(mn, mx)
            rec["quantizer"] = {"min": mn, "max": mx, "scale": dscale, "zp": dzp,
                                "matches_the_scale_used": dscale == scale and dzp == zp}
        except Exception as e:  # reported in the record, never fatal to the line
            rec["quantizer"] = {"error": f"{type(e).__name__}: {e}"}
    if not args.no_cpu_baseline:
        leaf_np = leaf.cpu().numpy()
        oob_np = oob.to(torch.uint8).cpu().numpy()
        rec["cpu_baseline"] = cpu_baseline(cfg, leaf_np, oob_np, n, fmt, scale, zp, args.cpu_seconds)
    else:
        rec["cpu_baseline"] = None
    ctx.close()
    return rec


def cpu_baseline_topk(cfg, ref_tn, q_qt, k, target_s):
    """The oracle's top-K (OpenMP over queries, a dense count scan per query
    like python/randomforest_py.cpp:2534-2558) on bounded query samples:
    median of three runs on every thread this process may use, then one
    single-thread run."""
    import statistics

    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O

    model, ncpu, threads = host_cpu()
    t, n = ref_tn.shape
    nq_all = q_qt.shape[0]

    def rate(nth, budget, seed_off):
        # queries [lo, lo + n_q) of the set: a first run of one query per
        # thread sizes the timed run to the budget
        lo = min(seed_off, max(0, nq_all - nth))
        n_q = min(nth, nq_all - lo)
        t0 = time.perf_counter()
        O.topk_all(ref_tn, q_qt[lo:lo + n_q], k, threads=nth)
        dt = time.perf_counter() - t0
        if dt < budget:
            n_q = min(nq_all - lo, max(n_q, int(n_q * budget / max(dt, 1e-3)) // nth * nth))
            t0 = time.perf_counter()
            O.topk_all(ref_tn, q_qt[lo:lo + n_q], k, threads=nth)
            dt = time.perf_counter() - t0
        return n_q * n * t / dt, n_q, dt

    per_run = target_s / 4.0
    runs = [rate(threads, per_run, 64 * j) for j in range(3)]
    r1 = rate(1, per_run, 256)
    return {
        "value": statistics.median(r[0] for r in runs),
        "unit": "pair-tree comparisons/s",
        "cores": threads,
        "kind": "port",
        "cpu_model": model,
        "host_cpus": ncpu,
        "single_thread_value": r1[0],
        "runs": [r[0] for r in runs],
        "sample": (f"median of 3 runs on {threads} threads of {runs[0][1]}-{max(r[1] for r in runs)} queries "
                   f"against all {n} references (~{per_run:.0f} s each); single thread: {r1[1]} queries "
                   f"({r1[2]:.1f} s); linear in the query count"),
    }


def run_c5(args, name="c5"):
    """Top-K of K=20 references per query for Q queries against N references
    over T trees (all trees, zeros included, ties by lower index).  The
    reference index (rfxp_set_reference) is built once outside the timed
    region; one step = rfxp_topk over all Q queries.  Returns the record."""
    import numpy as np
    import torch

    import rfxprox as R

    cfg = CONFIGS["c5"]
    n = args.n or cfg["n"]
    q = args.q or cfg["q"]
    t, nleaf, k = cfg["t"], cfg["nleaf"], cfg["k"]
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(cfg["seed"])
    ref = torch.randint(0, nleaf, (t, n), generator=g, device=dev, dtype=torch.int32)
    qs = torch.randint(0, nleaf, (q, t), generator=g, device=dev, dtype=torch.int32)
    ctx = R.Context(0)
    ctx.use_torch_stream()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ctx.set_reference(ref, n, t, nleaf)
    torch.cuda.synchronize()
    index_ms = (time.perf_counter() - t0) * 1e3
    for _ in range(args.warmup):
        ctx.topk(qs, k)
    torch.cuda.synchronize()
    ctx.set_timing(True)
    ctx.reset_timing()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(args.steps):
        ctx.topk(qs, k)
    ev1.record()
    torch.cuda.synchronize()
    ms_step = ev0.elapsed_time(ev1) / args.steps
    kms, kn = ctx.kernel_time("topk")
    k_avg = kms / max(kn, 1)
    # algorithmic bytes of one launch: every member id of the query's T
    # buckets (N/nleaf per bucket on average, 4 B) + the query labels + outputs
    alg = q * t * (n / nleaf) * 4 + q * t * 4 + q * k * 6
    achieved = alg / (k_avg / 1e3) / 1e9
    # compulsory HBM bytes: the reference leaf matrix and the queries once
    # (int16 labels, as the survey counts them) and the outputs
    compulsory = n * t * 2 + q * t * 2 + q * k * 6
    rec = {
        "metric": "pair-tree comparisons/sec (C5 top-K retrieval, Q x N x T)",
        "value": q * n * t / (ms_step / 1e3),
        "unit": "pair-tree comparisons/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u16",
        "data": "synthetic (uniform 2048-leaf assignment, seeded)",
        "config": {"workload": cfg["workload"], "N": n, "Q": q, "T": t, "leaves_per_tree": nleaf, "K": k},
        "queries_per_s": q / (ms_step / 1e3),
        "index_build_ms": index_ms,
        "kernels_ms": {"topk_avg": k_avg},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "alg_bytes_per_launch": alg, "traffic": None,
                     "compulsory_bytes": compulsory,
                     "frac_compulsory_step": compulsory / (ms_step / 1e3) / 1e9 / HBM_PEAK_GBS},
    }
    ctx.set_timing(False)
    if not args.no_cpu_baseline:
        rec["cpu_baseline"] = cpu_baseline_topk(cfg, ref.cpu().numpy(), qs.cpu().numpy(), k, args.cpu_seconds)
    else:
        rec["cpu_baseline"] = None
    ctx.close()
    return rec


def run_c4(args, name="c4"):
    """One step = rfxp_lowrank_pv (Y = A (A^T V) / T) on an N x 32 block;
    also reported: the 5-iteration subspace run to a rank-32 factor.  The
    reference index (rfxp_set_reference) is built once outside the timed
    region.  Returns the record."""
    import numpy as np
    import torch

    import rfxprox as R

    cfg = CONFIGS["c4"]
    n = args.n or cfg["n"]
    t, nleaf, r = cfg["t"], cfg["nleaf"], cfg["r"]
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(cfg["seed"])
    p = 1.0 / torch.arange(1, nleaf + 1, dtype=torch.float64) ** cfg["zipf"]
    p = (p / p.sum()).to(dev)
    leaf = torch.empty((t, n), dtype=torch.int32, device=dev)
    for k in range(t):
        perm = torch.randperm(nleaf, generator=g, device=dev).to(torch.int32)
        leaf[k] = perm[torch.multinomial(p, n, replacement=True, generator=g)]
    V = torch.randn((n, r), generator=g, device=dev, dtype=torch.float32)
    ctx = R.Context(0)
    ctx.use_torch_stream()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ctx.set_reference(leaf, n, t, nleaf)
    ctx.lowrank_pv(V)            # also builds the piece index
    torch.cuda.synchronize()
    index_ms = (time.perf_counter() - t0) * 1e3
    for _ in range(args.warmup):
        ctx.lowrank_pv(V)
    torch.cuda.synchronize()
    ctx.set_timing(True)
    ctx.reset_timing()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(args.steps):
        ctx.lowrank_pv(V)
    ev1.record()
    torch.cuda.synchronize()
    ms_step = ev0.elapsed_time(ev1) / args.steps
    w_ms = ctx.kernel_time("lr_w")[0] / args.steps
    y_ms = ctx.kernel_time("lr_y")[0] / args.steps
    ctx.set_timing(False)
    t0 = time.perf_counter()
    Q, B = ctx.lowrank_subspace(V, cfg["iters"])
    torch.cuda.synchronize()
    sub_ms = (time.perf_counter() - t0) * 1e3
    # compulsory HBM bytes of one P V: the member lists once (A^T V, k_lr_w),
    # the leaf labels once (A W, k_lr_y), V and Y once, W written once and
    # read once per (tree, leaf); the per-(sample, tree) row gathers of V
    # and W (2 N T r 4 B) are served from L2 / Infinity Cache and reported
    # separately as the gather rate
    alg = n * t * 4 + n * t * 4 + 2 * n * r * 4 + 2 * t * nleaf * r * 4
    gather = 2 * n * t * r * 4
    achieved = alg / (ms_step / 1e3) / 1e9
    rec = {
        "metric": "one-hot SpMM P V throughput (C4, N x T x r multiply-adds)",
        "value": 2 * n * t * r / (ms_step / 1e3),
        "unit": "multiply-adds/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (Zipf(1.1) leaf sizes, per-tree label permutation, V ~ N(0,1), seeded)",
        "config": {"workload": cfg["workload"], "N": n, "T": t, "leaves_per_tree": nleaf, "r": r,
                   "iters": cfg["iters"]},
        "kernels_ms": {"lr_w": w_ms, "lr_y": y_ms},
        "subspace_ms": sub_ms,
        "index_build_ms": index_ms,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "alg_bytes_per_step": alg, "traffic": None,
                     "compulsory_bytes": alg,
                     "frac_compulsory_step": alg / (ms_step / 1e3) / 1e9 / HBM_PEAK_GBS},
        "gather_GBps": gather / (ms_step / 1e3) / 1e9,
        "ritz_top": float(np.max(np.linalg.eigvalsh((B + B.T) / 2))),
    }
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(REPO, "oracle"))
        import oracle as O

        # the oracle's SpMM on a tree subset at full N, scaled to T trees:
        # median of three runs on every thread this process may use, then
        # one single-thread run
        import statistics

        model, ncpu, threads = host_cpu()
        tt = 8
        lf = leaf[:tt].cpu().numpy()
        Vd = V.cpu().numpy().astype(np.float64)

        def one(nth):
            c0 = time.perf_counter()
            O.lowrank_pv(lf, nleaf, Vd, threads=nth)
            return 2 * n * t * r / ((time.perf_counter() - c0) * t / tt)

        runs = [one(threads) for _ in range(3)]
        rec["cpu_baseline"] = {"value": statistics.median(runs), "unit": "multiply-adds/s", "cores": threads,
                               "kind": "port", "cpu_model": model, "host_cpus": ncpu,
                               "single_thread_value": one(1), "runs": runs,
                               "sample": f"{tt} of {t} trees at full N, scaled linearly; median of 3 runs"}
    else:
        rec["cpu_baseline"] = None
    ctx.close()
    return rec


# the C++ program that calls the class through the reference's signatures
LRDRIVER = os.path.join(REPO, "tests", "compat", "lowrank_driver")


def run_cs2(args, name="cs2"):
    """The class sequence of cuda/rf_growtree.cu:5219-5410 through the
    reference's own C++ signatures (tests/compat/lowrank_driver, mode
    "measure", a separate process linked against librfxprox.so): per tree
    cudaMalloc + memset of the N(N+1)/2 FP16 triangle,
    gpu_proximity_upper_triangle_fp16 from host nodestatus / nodextr / nin,
    add_tree_contribution_incremental_upper_triangle_fp16, free; then
    finalize_accumulation(T, true), get_lowrank_factors_host and
    compute_mds_from_factors_host.  One step = one tree.  The forest is
    synthetic: nleaf terminal nodes per tree with skewed sizes, bootstrap
    multiplicities for nin.  Returns the record."""
    import statistics
    import subprocess
    import tempfile

    import numpy as np

    cfg = CONFIGS["cs2"]
    n = args.n or cfg["n"]
    t, nleaf, level = cfg["t"], cfg["nleaf"], cfg["level"]
    drv = LRDRIVER
    if not os.path.exists(drv):
        raise RuntimeError("tests/compat/lowrank_driver is not built (make -C rfx-fuse_amd driver)")
    rng = np.random.default_rng(cfg["seed"])
    nnode = 2 * nleaf - 1
    w = 1.0 / np.arange(1, nleaf + 1) ** 0.8
    w /= w.sum()
    with tempfile.TemporaryDirectory() as tmp:
        inp, outp = os.path.join(tmp, "in.bin"), os.path.join(tmp, "out.bin")
        nout = np.zeros(n, np.int32)
        with open(inp, "wb") as f:
            np.array([n, t, 0], np.int32).tofile(f)
            for _ in range(t):
                ns = np.ones(nnode, np.int32)
                term = rng.choice(nnode, nleaf, replace=False)
                ns[term] = -1
                nx = term[rng.permutation(nleaf)[rng.choice(nleaf, n, p=w)]].astype(np.int32)
                nin = np.bincount(rng.integers(0, n, n), minlength=n).astype(np.int32)
                nout += nin == 0
                np.array([nnode], np.int32).tofile(f)
                ns.tofile(f)
                nx.tofile(f)
                nin.tofile(f)
            nout.tofile(f)
        wall0 = time.perf_counter()
        r = subprocess.run(["timeout", "-k", "10", "900", drv, inp, outp, "measure", str(level)],
                           capture_output=True, text=True)
        wall = time.perf_counter() - wall0
        if r.returncode != 0:
            raise RuntimeError(f"lowrank_driver exited {r.returncode}: {(r.stdout + r.stderr)[-400:]}")
        raw = np.fromfile(outp, np.uint8)
    rank = int(raw[:4].view(np.int32)[0])
    # skip the sections before the measurements (layout in the driver's header)
    off = 12 + 2 * 8 * n * rank
    nc = int(raw[off:off + 8].view(np.int64)[0])
    off += 8 + 8 * nc
    rec_flag = int(raw[off:off + 4].view(np.int32)[0])
    off += 4 + (8 * n * n if rec_flag else 0)
    mem = raw[off:off + 32].view(np.uint64)
    off += 32 + 8 + 16 + 8
    tt = int(raw[off:off + 4].view(np.int32)[0])
    off += 4
    times = raw[off:off + 24 * tt].view(np.float64).reshape((tt, 3))
    off += 24 * tt
    used = raw[off:off + 8 * tt].view(np.uint64).astype(np.int64)
    off += 8 * tt
    used0 = int(raw[off:off + 8].view(np.uint64)[0])
    fin_ms, fac_ms, mds_ms = (float(x) for x in raw[off + 8:off + 32].view(np.float64))
    step_ms = float(statistics.median(times[:, 2]))
    ne = n * (n + 1) // 2
    # compulsory HBM bytes of one tree: the caller's memset of the FP16
    # triangle and one read of it by the add
    compulsory = 2 * ne * 2
    return {
        "metric": "trees/s of the growtree low-rank sequence (CS2)",
        "value": 1e3 / step_ms,
        "unit": "trees/s",
        "n_gpus": 1,
        "steps": tt,
        "warmup": 0,
        "ms_per_step": step_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": (f"synthetic ({nleaf} terminal nodes per tree, sizes ~ 1/k^0.8, bootstrap nin, seeded); "
                 "one step = one tree, median over the trees"),
        "config": {"workload": cfg["workload"], "N": n, "T": t, "leaves_per_tree": nleaf, "level": level,
                   "rank": rank},
        "kernels_ms": {"triangle_median": float(np.median(times[:, 0])),
                       "add_median": float(np.median(times[:, 1])),
                       "step_first": float(times[0, 2]), "step_max": float(times[:, 2].max())},
        "finalize_ms": fin_ms,
        "factors_copy_ms": fac_ms,
        "mds_ms": mds_ms,
        "device_bytes_after_add": {"first": int(used[0] - used0), "last": int(used[-1] - used0),
                                   "max": int(used.max() - used0)},
        "get_memory_usage": [int(x) for x in mem],
        "driver_wall_s": wall,
        "roofline": {"bound": "hbm", "achieved": compulsory / (step_ms / 1e3) / 1e9, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": compulsory / (step_ms / 1e3) / 1e9 / HBM_PEAK_GBS,
                     "compulsory_bytes": compulsory, "traffic": None},
        # the reference has no CPU form of this class; nothing to time beside it
        "cpu_baseline": None,
    }


RUNNERS = {"c3": run_triangle, "c2": run_triangle, "c5": run_c5, "c4": run_c4, "cs2": run_cs2}


if __name__ == "__main__":
    main()
