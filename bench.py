"""Benchmark: histogram GB/s + seconds per 100 trees, 10.5M x 28 quantized-grad, 1 MI355X.

One step = one boosting iteration of BASELINE.json configs[1] (binary logloss,
num_leaves 255, max_bin 63, int8 gradients with 4 quantization bins and stochastic
rounding) with every input resident in HBM: objective -> quantize -> grow the tree
(histogram, split scan, partition for all 254 splits) -> score update.  The raw
table is binned by the library (BinMapper on a 200k-row sample on the host, then
ValueToBin on the device) before the timed region; the binning kernel and a batch
prediction with the trained trees are reported as secondary lines (`next_rows`).

Prints ONE JSON line.  `value` is seconds per 100 trees (lower is better) over the
timed iterations 0 .. K-1 (default K = 100: the metric's first 100 trees), the first
of `--repeats` timed runs (their median is reported beside it).  `roofline` is the
dominant kernel at the survey's algorithmic bytes, timed with HIP events on the
library's own stream; `hist_GBps` is every ConstructHistogram of the iterations at
those bytes over the kernels that perform them.  `cpu_baseline` times the CPU
restatement of the reference learner (oracle/) on a bounded sample of the same
workload and bins (all cores and one thread), and `parity` compares the device's
first iterations with that run's trees and scores, bit for bit.

`--workload config2|config3|config4` instead times BASELINE.json configs[2] (1M x 2000
sparse LogNormal features, L2 regression, f32 gradients, feature_fraction 0.8, 127
leaves), configs[3] (2M x 100 with 20 categorical features, softmax over 10 classes:
10 trees per iteration, f32 gradients, 127 leaves) or configs[4] (2M x 700,
lambdarank over query groups, quantized, 255 leaves) on the wide row layout, as a secondary line with the roofline of its dominant kernel
(k_hist_wide) and the CPU restatement timed on its first iteration; the default
`config1` is the headline above.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def traffic_for(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc summary.

    profiles/traffic_config1_10.5Mx28.md holds, per kernel, the FETCH_SIZE and
    WRITE_SIZE readings of two counter runs of this script, each already scaled
    by what the same counter reads for a device copy of known size (the
    --copy-probe-mib kernel), as lines `traffic <kernel> <bytes per launch>`.
    Returns None when no such measurement exists."""
    path = os.path.join(ROOT, "profiles", "traffic_config1_10.5Mx28.md")
    try:
        with open(path) as f:
            for line in f:
                parts = line.strip().strip("`").split()
                if len(parts) == 3 and parts[0] == "traffic" and parts[1] == kernel:
                    return float(parts[2])
    except OSError:
        pass
    return None


def _line(kernel, ms, launches, bytes_per_launch, workload, walks=None):
    """A secondary kernel's per-launch time and algorithmic bandwidth (HIP events on
    the library's stream)."""
    if launches <= 0 or ms <= 0:
        return None
    us = ms * 1e3 / launches
    gbs = bytes_per_launch / (us * 1e-6) / 1e9
    out = {"kernel": kernel, "workload": workload, "avg_launch_us": round(us, 2),
           "bytes_per_launch": int(bytes_per_launch), "achieved_GBps": round(gbs, 1),
           "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
    if walks is not None:
        out["row_trees_per_s"] = float(f"{walks / (ms * 1e-3):.4g}")
    return out


def cpu_info():
    """(CPU model name, physical cores) of this host from /proc/cpuinfo."""
    model, cores = None, set()
    try:
        phys = core = None
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "model name" and model is None:
                model = v
            elif k == "physical id":
                phys = v
            elif k == "core id":
                core = v
            elif not k and phys is not None:
                cores.add((phys, core))
                phys = core = None
        if phys is not None:
            cores.add((phys, core))
    except OSError:
        pass
    return model, (len(cores) or None)


def compare_iterations(trees, scores, otrees, oscores, init):
    """The device's first iterations vs the CPU baseline's: every tree field and every
    training score bit-exact (the oracle's first tree carries Tree::add_bias(init))."""
    import numpy as np
    z = float(np.float32(1e-35))

    def mrz(v):
        return np.where((v >= -z) & (v <= z), 0.0, v)

    bad = []
    for i, (t, o) in enumerate(zip(trees, otrees)):
        t = dict(t)
        if i == 0 and init != 0.0:
            t["leaf_value"] = mrz(t["leaf_value"] + init)
            t["internal_value"] = mrz(t["internal_value"] + init)
        if t["num_leaves"] != o["num_leaves"]:
            bad.append(f"tree {i} num_leaves")
            continue
        for k in o:
            if k == "num_leaves":
                continue
            a, b = np.ascontiguousarray(t[k]), np.ascontiguousarray(o[k])
            if a.shape != b.shape or a.tobytes() != b.tobytes():
                bad.append(f"tree {i} {k}")
    same_scores = bool(np.ascontiguousarray(scores).tobytes() ==
                       np.ascontiguousarray(oscores).tobytes())
    # the tree structure (what splits where, and the partition counts)
    structural = ("num_leaves", "split_feature", "threshold_in_bin", "threshold",
                  "decision_type", "left_child", "right_child", "leaf_count",
                  "internal_count", "leaf_depth", "leaf_parent", "cat_boundaries",
                  "cat_threshold", "num_cat")
    return {"iterations": len(trees), "trees_bit_exact": not bad, "mismatches": bad[:8],
            "structure_equal": not any(m.split()[-1] in structural for m in bad),
            "scores_bit_exact": same_scores,
            "leaves": [int(t["num_leaves"]) for t in trees]}


def secondary(args):
    """configs[2] / [3] / [4]: the wide row layout's paths (column sampling and L2
    regression with f32 gradients; softmax over 10 classes with categorical splits and
    f32 gradients; lambdarank with quantized gradients)."""
    import numpy as np
    from lightgbm_rs_amd import GainConfig, HipBackend, boost_from_score, feature_meta
    from lightgbm_rs_amd.synth import (config2_raw_host, config3_mappers, config3_raw_host,
                                       config4_raw_host, sample_mappers)

    t0 = time.perf_counter()
    K, cat = 1, []  # trees per iteration, categorical features
    if args.workload == "config3":
        n, K = 2_000_000, 10
        X, y, cat = config3_raw_host(n, num_class=K)
        F = X.shape[0]
        obj, nl, ff, qbins, qb = "multiclass", 127, 1.0, 0, None
        workload = ("configs[3]: softmax, 10 classes, 2M rows x 100 features (80 N(0,1), "
                    "20 categorical of 32 levels), max_bin 255, num_leaves 127, categorical "
                    "splits, f32 gradients, one step = one iteration = 10 trees")
        dtype = "f32 grad/hess, 64-bit fixed-point histogram, f64 split math"
    elif args.workload == "config2":
        n, F = 1_000_000, 2000
        X, y = config2_raw_host(n, F=F)
        obj, nl, ff, qbins, qb = "regression", 127, 0.8, 0, None
        workload = ("configs[2]: L2 regression, 1M rows x 2000 sparse LogNormal features, "
                    "max_bin 255, num_leaves 127, feature_fraction 0.8, f32 gradients")
        dtype = "f32 grad/hess, 64-bit fixed-point histogram, f64 split math"
    else:
        n, F = 2_000_000, 700
        X, y, groups = config4_raw_host(n, F=F)
        qb = np.concatenate([[0], np.cumsum(groups)]).astype(np.int32)
        obj, nl, ff, qbins = "lambdarank", 255, 1.0, 4
        workload = ("configs[4]: lambdarank, 2M rows x 700 features in query groups, "
                    "max_bin 255, num_leaves 255, quantized int8 grads (4 bins, stochastic)")
        dtype = "int8 grad/hess, int32 histogram, f64 split math"
    if cat:
        mappers, meta, ub = config3_mappers(X, cat)
    else:
        mappers = sample_mappers(X, 255)
        meta = [feature_meta(m.num_bin, m.most_freq_bin, m.missing_type, m.default_bin, f)
                for f, m in enumerate(mappers)]
        ub = np.concatenate([m.upper_bounds for m in mappers])
    log(f"{args.workload}: data + mappers {time.perf_counter() - t0:.1f}s")
    if K > 1:  # BoostFromAverage per class (gbdt.rs:691-1373), classes that need trees
        k_eps = float(np.float32(1e-15))
        prior = np.bincount(y.astype(np.int64), minlength=K) / n
        init_k = np.log(np.maximum(prior, k_eps))
        init_k = np.where(np.abs(init_k) > k_eps, init_k, 0.0)
        need = [0 if (p <= k_eps or p >= 1.0 - k_eps) else 1 for p in prior]
        init = 0.0
    else:
        init = boost_from_score(obj, y)
        init = init if abs(init) > 1e-15 else 0.0
    cfg = GainConfig.make(min_data_in_leaf=20)
    be = HipBackend(0)
    be.upload_raw(X, mappers, col_major=True)
    del X
    cpu_iters = min(args.cpu_iters, 1)
    bins = be.get_bins() if cpu_iters > 0 else None  # the CPU baseline's input

    def start():
        if K > 1:
            be.set_labels_multiclass(y, K, init_k)
            return
        be.set_labels(y, init)
        if obj == "lambdarank":
            be.set_lambdarank(qb)
        else:
            be.set_objective(obj)
        if ff < 1.0:
            be.set_col_sampler(ff, 1.0, 2)

    def step(i):  # one boosting iteration: its K trees, read back
        if K > 1:
            return be.train_iter_multiclass(i, cfg, nl, -1, 0.1, qbins, True, need)
        return [be.train_iter(i, cfg, nl, -1, 0.1, qbins, True)]

    # configs[3] times its first iterations from a fresh score (at most 10 = 100 trees):
    # the reference's categorical child seeding (learner.rs:4191-4229, kept bit for bit)
    # hands a child its sibling's sums whenever the SplitInfo and partition counts order
    # the two differently, which on this data drives the softmax scores to saturation and
    # a class's root sum_hessian to 0 (InvalidLeafHessian, learner.rs:1331-1334) after
    # about 14 iterations, in the CPU restatement as on the device
    steps = min(args.steps, 10) if K > 1 else args.steps
    first = 0 if K > 1 else args.warmup
    start()
    for i in range(max(args.warmup, 1)):
        step(i)
    if K > 1:
        start()
    t1 = time.perf_counter()
    for i in range(first, first + steps):
        step(i)
    elapsed = time.perf_counter() - t1
    if K > 1:
        start()
    be.set_timing(True)
    p0 = 0 if K > 1 else first + steps
    for i in range(p0, p0 + max(args.prof_steps, 1)):
        step(i)
    tm = be.timing()
    be.set_timing(False)
    gpu_first = None
    if cpu_iters > 0:  # the parity leg's device iterations, from a fresh start
        start()
        gpu_first = [t for i in range(cpu_iters) for t in step(i)]
        gpu_scores = be.scores()
        if K > 1:  # the first iteration's trees carry the class's init (add_bias)
            z = float(np.float32(1e-35))
            for k, t in enumerate(gpu_first[:K]):
                if abs(init_k[k]) > 0.0 and t["num_leaves"] > 1:
                    for key in ("leaf_value", "internal_value"):
                        v = t[key] + init_k[k]
                        t[key] = np.where((v >= -z) & (v <= z), 0.0, v)
    be.close()
    ps = max(args.prof_steps, 1)
    ms = elapsed / steps * 1e3
    # k_hist_wide, the dominant kernel: the survey's algorithmic bytes, u8 bins (F per
    # row), the pair (2 B quantized, 8 B f32) and the row index of a child build
    w_gh = 2 if qbins else 8
    cell_b = 8 if qbins else 16
    hist_bytes = (tm["root_rows"] * (F + w_gh) + tm["hist_child_rows"] * (F + w_gh + 4)
                  + (tm["hist_launches"] + tm["partition_launches"]) * tm["cells"] * cell_b)
    hist_launches = tm["hist_launches"] + tm["partition_launches"]
    hist_gbs = hist_bytes / (tm["hist_ms"] * 1e-3) / 1e9 if tm["hist_ms"] > 0 else 0.0
    cpu, parity = None, None
    if cpu_iters > 0:
        from oracle import oracle
        env_threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
        threads = oracle.set_threads(args.cpu_threads or env_threads or len(os.sched_getaffinity(0)))
        okind = oracle.OBJECTIVE_LAMBDARANK if obj == "lambdarank" else oracle.OBJECTIVE_REGRESSION
        tc = time.perf_counter()
        if K > 1:
            oscores, otrees = oracle.train_multiclass(bins, meta, ub, y, K, cfg, nl, -1,
                                                      cpu_iters, 0.1)
        else:
            oscores, otrees = oracle.train(bins, meta, ub, y, cfg, okind, nl, -1, cpu_iters,
                                           0.1, quantized=qbins > 0, feature_fraction=ff,
                                           feature_fraction_seed=2, query_boundaries=qb)
        cs = time.perf_counter() - tc
        log(f"cpu: {cs:.1f}s for {cpu_iters} iteration(s) on {threads} threads")
        model_name, phys = cpu_info()
        cpu = {"value": round(cs / (cpu_iters * K) * 100.0, 3), "unit": "s/100 trees",
               "cores": threads,
               "kind": "port",
               "sample": f"the first {cpu_iters} boosting iteration(s) ({cpu_iters * K} trees) "
                         f"of the same workload and "
                         f"bins (C++ restatement of the reference CpuBackend learner, OpenMP, "
                         f"{threads} threads: {cs:.1f}s), scaled to 100 trees",
               "cpu_model": model_name, "physical_cores": phys,
               "gpu_speedup": round((cs / cpu_iters) / (elapsed / steps), 1)}
        parity = compare_iterations(gpu_first, gpu_scores, otrees, oscores, init)
        if not qbins:  # f32 gradients: fixed-point cells vs the f64 fold (stated bar 1e-5)
            parity["scores_max_rel_diff"] = float(
                np.max(np.abs(gpu_scores - oscores) / np.maximum(np.abs(oscores), 1e-300)))
            # the tree structure must match exactly; the f64 values within the bar
            parity["within_1e-5"] = bool(parity["structure_equal"] and
                                         parity["scores_max_rel_diff"] <= 1e-5)
        log(f"parity: {parity}")
    print(json.dumps({
        "metric": f"sec per 100 trees, {args.workload} (wide row layout), 1 MI355X",
        "value": round(ms / K / 10.0, 4), "unit": "s/100 trees", "n_gpus": 1, "steps": steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": dtype,
        "data": "synthetic (BASELINE.json recipe), binned by the library's BinMapper",
        "config": {"workload": workload, "rows": n, "features": F, "num_leaves": nl},
        "phase_ms_per_step": {k: round(v / ps, 4) for k, v in tm.items()
                              if k.endswith("_ms")},
        "trees_per_step": K,
        "rounds_per_tree": round(tm["rounds"] / max(tm["trees"], 1.0), 1),
        "roofline": {"bound": "hbm", "achieved": round(hist_gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(hist_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "k_hist_wide (ConstructHistogram, root and child builds)",
                     "bytes_per_launch": round(hist_bytes / max(hist_launches, 1), 1),
                     "launches": int(hist_launches),
                     "avg_launch_us": round(tm["hist_ms"] * 1e3 / max(hist_launches, 1), 3)},
        "cpu_baseline": cpu, "parity": parity}), flush=True)


def lds_probe(args):
    """LDS-atomic ceiling of the quantized histogram adds (lgbm_hip_probe_lds_atomics):
    one packed-cell add per (row, feature) into 28 x 64 LDS cells, with nothing else in
    the loop, on configs[1]-shaped bins; prints one JSON line of lane adds per CU-cycle
    per mode and the root build's LDS-only floor at that rate."""
    import ctypes as C
    import numpy as np
    from lightgbm_rs_amd import load_library
    from lightgbm_rs_amd.synth import config1_like

    lib = load_library()
    n = 262_144  # one row per thread of the probe's 2 x 256 blocks x 512 threads
    bins, _, _, _ = config1_like(n)
    bins = np.ascontiguousarray(bins, np.uint8)
    F = bins.shape[0]
    modes = {"u32 distinct": 0, "u32 config1 bins": 1, "u32 one address": 2,
             "u64 distinct": 4, "u64 config1 bins": 5, "u64 one address": 6,
             "u32 wave-private distinct": 8, "u32 wave-private config1 bins": 9}
    rows = {}
    for name, mode in modes.items():
        out = (C.c_double * 5)()
        rc = lib.lgbm_hip_probe_lds_atomics(C.c_int(0), bins.ctypes.data_as(C.c_void_p),
                                            C.c_int64(n), C.c_int32(F), C.c_int32(mode),
                                            C.c_int32(args.probe_reps), out)
        if rc != 0:
            sys.exit(f"lds probe mode {mode}: status {rc}")
        rows[name] = {"ms": round(out[0], 4), "lane_adds": int(out[1]),
                      "lane_adds_per_cu_cycle": round(out[2], 3)}
        clock_mhz, cus = out[3], int(out[4])
        log(f"lds probe {name}: {out[2]:.3f} lane adds / CU-cycle ({out[0]:.3f} ms)")
    root_adds = 10_500_000 * 28
    floor = {k: round(root_adds / (v["lane_adds_per_cu_cycle"] * cus * clock_mhz * 1e6) * 1e6, 1)
             for k, v in rows.items()}
    print(json.dumps({"probe": "lds atomics", "rows_per_launch": n, "features": F,
                      "reps": args.probe_reps, "clock_mhz": clock_mhz, "cus": cus,
                      "modes": rows,
                      "root_build_lds_floor_us (10.5M rows x 28 adds)": floor}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--rows", type=int, default=10_500_000)
    ap.add_argument("--num-leaves", type=int, default=255)
    ap.add_argument("--cpu-iters", type=int, default=5,
                    help="boosting iterations of the all-core CPU baseline sample, also "
                         "replayed on the device for the parity check (0 disables both)")
    ap.add_argument("--cpu-iters-1t", type=int, default=3,
                    help="boosting iterations of the 1-thread CPU baseline sample")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="all-core thread count (default: OMP_NUM_THREADS, else usable CPUs)")
    ap.add_argument("--repeats", type=int, default=3,
                    help="timed loops of --steps iterations; value is the first, the median "
                         "of all is reported beside it")
    ap.add_argument("--prof-steps", type=int, default=3,
                    help="extra iterations timed per kernel with HIP events")
    ap.add_argument("--workload", default="config1",
                    choices=["config1", "config2", "config3", "config4"],
                    help="config1: the headline; config2 / config3 / config4: a secondary "
                         "wide-layout line")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="after the run, copy a buffer of this many MiB device-to-device "
                         "(3 times): the known-size kernel that scales rocprofv3 "
                         "FETCH_SIZE/WRITE_SIZE readings to bytes")
    ap.add_argument("--lds-probe", action="store_true",
                    help="measure the LDS-atomic ceiling of the histogram adds instead")
    ap.add_argument("--probe-reps", type=int, default=64)
    args = ap.parse_args()
    if args.lds_probe:
        return lds_probe(args)
    if args.gpus != 1:
        print(f"bench.py runs on exactly one GPU (--gpus {args.gpus} requested): this build "
              "has no multi-GPU path (rows would shard by range, one all-reduce of each "
              "round's built integer histograms; not built).", file=sys.stderr)
        sys.exit(2)
    if args.workload != "config1":
        return secondary(args)

    import numpy as np
    import torch

    from lightgbm_rs_amd import (BinMapper, GainConfig, HipBackend, Model,
                                 binary_boost_from_score, sample_indices)
    from lightgbm_rs_amd.synth import config1_raw

    n, nl = args.rows, args.num_leaves
    t0 = time.perf_counter()
    dev = torch.device("cuda:0") if torch.cuda.is_available() else None
    if dev is None:
        sys.exit("bench.py needs a HIP device")
    # raw table generated on the device by torch, then handed to the library as host
    # memory (torch and the library each bring their own HIP runtime)
    Xd, y = config1_raw(n, device=dev)
    idx = torch.from_numpy(sample_indices(n, 200000, 1).astype(np.int64)).to(dev)
    sampled = Xd[:, idx].double().cpu().numpy()
    X = Xd.cpu().numpy()  # [28, n] float32, one feature per row
    del Xd, idx
    torch.cuda.empty_cache()
    mappers = [BinMapper.from_sampled_column(sampled[f], n, max_bin=63) for f in range(28)]
    log(f"data: {n} x 28, num_bin {max(m.num_bin for m in mappers)}, "
        f"gen + mappers {time.perf_counter()-t0:.1f}s")
    init = binary_boost_from_score(y)
    cfg = GainConfig.make(min_data_in_leaf=20, min_sum_hessian_in_leaf=1e-3)
    lr = 0.1

    be = HipBackend(0)
    t1 = time.perf_counter()
    be.upload_raw(X, mappers, col_major=True)  # first binning: fresh allocations
    # a job that hands the raw table over from host memory pays this once: PCIe copy
    # of 10.5M x 28 f32 plus the device binning (reported beside `value`, never in it)
    t_up = time.perf_counter()
    be.upload_raw(X, mappers, col_major=True)
    upload_s = time.perf_counter() - t_up
    be.set_timing(True)
    be.upload_raw(X, mappers, col_major=True)
    bin_tm = be.timing()
    be.set_timing(False)
    be.set_labels(y, init)
    bins = be.get_bins() if args.cpu_iters > 0 else None  # the CPU baseline's input
    log(f"upload + device binning {time.perf_counter()-t1:.2f}s "
        f"(kernel {bin_tm['bin_ms']:.3f} ms)")
    # the host reads each tree while the device already computes the next
    # iteration's gradients and quantization (results unchanged)
    be.set_lookahead(True)
    for i in range(args.warmup):
        be.train_iter_binary(i, cfg, nl, -1, lr, 4, True, want_tree=False)
    torch.cuda.synchronize() if dev is not None else None
    # Timed: iterations 0 .. K-1 of the boosting run (the score is reset to the init
    # score before each repeat, so every repeat does the same work as a fresh run of
    # the first K iterations; the warmup only captured the per-tree graph).
    leaves, trees = [], []
    runs = []
    for rep in range(max(args.repeats, 1)):
        be.set_labels(y, init)
        torch.cuda.synchronize() if dev is not None else None
        t2 = time.perf_counter()
        for i in range(args.steps):
            t = be.train_iter_binary(i, cfg, nl, -1, lr, 4, True, want_tree=True)
            if rep == 0:
                leaves.append(t["num_leaves"])
                trees.append(t)
        torch.cuda.synchronize() if dev is not None else None
        runs.append(time.perf_counter() - t2)
    elapsed = runs[0]
    it = args.steps
    # the metric's first 100 trees when the timed window is shorter (later trees need
    # more rounds than the first ones)
    full100 = None
    if args.steps < 100:
        be.set_labels(y, init)
        torch.cuda.synchronize() if dev is not None else None
        t3 = time.perf_counter()
        for i in range(100):
            be.train_iter_binary(i, cfg, nl, -1, lr, 4, True, want_tree=False)
        torch.cuda.synchronize() if dev is not None else None
        full100 = time.perf_counter() - t3
        it = 100
    # Per-kernel device time: HIP events around every launch on the library's stream.
    # The per-tree sequence then runs as individual launches (no graph), so this pass
    # measures kernel durations, not the timed loop's wall clock.
    be.set_lookahead(False)
    be.set_timing(True)
    it0 = it
    for i in range(it0, it0 + args.prof_steps):
        be.train_iter_binary(i, cfg, nl, -1, lr, 4, True, want_tree=False)
    tm = be.timing()
    # parity leg (outside the timed region): the first cpu_iters iterations again from
    # the initial score, for the bit-exact comparison with the CPU baseline's trees
    gpu_iters = None
    if args.cpu_iters > 0:
        be.set_labels(y, init)
        gpu_iters = [be.train_iter_binary(i, cfg, nl, -1, lr, 4, True, want_tree=True)
                     for i in range(args.cpu_iters)]
        gpu_scores = be.scores()
    # secondary: batch prediction of the timed iterations' trees on the first
    # `pred_rows` rows (row-major f32, as the predictor reads them)
    model = Model.create(num_class=1, max_feature_idx=27, objective="binary sigmoid:1")
    for t in trees:
        model.add_tree(t, shrinkage=lr)
    pred_rows = min(n, 2_000_000)
    Xp = np.ascontiguousarray(X[:, :pred_rows].T)
    be.predict(model, Xp, "raw")  # first call: loads the kernel, sizes the buffers
    be.set_timing(True)
    for _ in range(3):
        be.predict(model, Xp, "raw")
    pred_tm = be.timing()
    be.close()
    del Xp
    if args.copy_probe_mib > 0 and dev is not None:
        nb = args.copy_probe_mib << 20
        src = torch.ones(nb // 4, dtype=torch.int32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy probe: {nb} bytes read + {nb} bytes written per launch")
        del src, dst
    tsteps = max(args.prof_steps, 1)
    ms_per_step = elapsed / args.steps * 1e3
    s_per_100 = elapsed / args.steps * 100.0
    F, cells, rec = tm["features"], tm["cells"], tm["record_bytes"]
    # Algorithmic bytes (the survey's per-unit figures; u8 bins, packed int8 g/h, u32
    # row index, int32 histogram cells):
    #   root ConstructHistogram: rows x (F + 2) + cells x 2 x 4 per launch;
    #   a split's DataPartition: parent rows x (4 + 1 + 4) (index in, bin, index out);
    #   its smaller child's ConstructHistogram: rows x (F + 2 + 4) + cells x 2 x 4.
    # k_partition does both for every split of a round.  The bytes it actually moves
    # (records of `rec` bytes + 2 B g/h, read and written) are reported as `design`.
    hist_w = cells * 8
    root_bytes = tm["root_rows"] * (F + 2) + tm["hist_launches"] * hist_w
    part_bytes = (tm["partition_rows"] * 9 + tm["hist_child_rows"] * (F + 6)
                  + tm["partition_jobs"] * hist_w)
    # record_bytes: what a partition pass reads per row (record + separately stored pair)
    design_bytes = tm["partition_rows"] * 2 * rec + tm["partition_jobs"] * hist_w
    root_gbs = root_bytes / (tm["hist_ms"] * 1e-3) / 1e9 if tm["hist_ms"] > 0 else 0.0
    part_gbs = part_bytes / (tm["partition_ms"] * 1e-3) / 1e9 if tm["partition_ms"] > 0 else 0.0
    design_gbs = design_bytes / (tm["partition_ms"] * 1e-3) / 1e9 if tm["partition_ms"] > 0 else 0.0
    # every ConstructHistogram of the iterations (root + each split's child) over the
    # time of the kernels that perform them (the child builds are fused into k_partition)
    build_bytes = root_bytes + tm["hist_child_rows"] * (F + 6) + tm["partition_jobs"] * hist_w
    build_ms = tm["hist_ms"] + tm["partition_ms"]
    hist_gbs = build_bytes / (build_ms * 1e-3) / 1e9 if build_ms > 0 else 0.0
    launches = tm["partition_launches"]
    if tm["partition_ms"] >= tm["hist_ms"]:
        dom = ("k_partition (DataPartition + smaller-child ConstructHistogram, fused)", part_gbs,
               part_bytes, launches, tm["partition_ms"])
    else:
        dom = ("k_hist_jobs (ConstructHistogram, root)", root_gbs, root_bytes, tm["hist_launches"],
               tm["hist_ms"])
    log(f"gpu: {ms_per_step:.2f} ms/step (repeats {[round(r / args.steps * 1e3, 3) for r in runs]}),"
        f" leaves {min(leaves)}..{max(leaves)}, timing {tm}")

    cpu, parity = None, None
    if args.cpu_iters > 0:
        from oracle import oracle
        from lightgbm_rs_amd import feature_meta
        meta = [feature_meta(m.num_bin, m.most_freq_bin, m.missing_type, m.default_bin, f)
                for f, m in enumerate(mappers)]
        ub = np.concatenate([m.upper_bounds for m in mappers])
        env_threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
        want = args.cpu_threads or env_threads or len(os.sched_getaffinity(0))
        threads = oracle.set_threads(want)
        tc = time.perf_counter()
        oscores, otrees = oracle.train_binary(bins, meta, ub, y, cfg, nl, -1, args.cpu_iters, lr,
                                              boost_from_average=True, quantized=True,
                                              quant_bins=4, stochastic=True, want_trees=True)
        cs = time.perf_counter() - tc
        log(f"cpu: {cs:.1f}s for {args.cpu_iters} iters on {threads} threads")
        one = None
        if args.cpu_iters_1t > 0:
            oracle.set_threads(1)
            t1c = time.perf_counter()
            oracle.train_binary(bins, meta, ub, y, cfg, nl, -1, args.cpu_iters_1t, lr,
                                boost_from_average=True, quantized=True, quant_bins=4,
                                stochastic=True, want_trees=False)
            one = time.perf_counter() - t1c
            oracle.set_threads(threads)
            log(f"cpu: {one:.1f}s for {args.cpu_iters_1t} iters on 1 thread")
        model_name, phys = cpu_info()
        cpu = {"value": round(cs / args.cpu_iters * 100.0, 3), "unit": "s/100 trees",
               "cores": threads, "kind": "port",
               "sample": f"the first {args.cpu_iters} boosting iterations of the same "
                         f"{n}x28 workload and bins (C++ restatement of the reference "
                         f"CpuBackend learner, OpenMP, {threads} threads: {cs:.1f}s), scaled "
                         f"to 100 trees",
               "one_thread": None if one is None else {
                   "value": round(one / args.cpu_iters_1t * 100.0, 3), "unit": "s/100 trees",
                   "sample": f"the first {args.cpu_iters_1t} iterations on 1 thread: "
                             f"{one:.1f}s"},
               "cpu_model": model_name, "physical_cores": phys,
               "usable_cpus": len(os.sched_getaffinity(0)),
               "gpu_speedup": round((cs / args.cpu_iters) / (elapsed / args.steps), 1)}
        parity = compare_iterations(gpu_iters, gpu_scores, otrees, oscores, init)
        log(f"parity: {parity}")

    out = {
        "metric": "histogram GB/s + sec per 100 trees, 10.5M x 28 quantized-grad, 1 MI355X",
        "value": round(s_per_100, 4),
        "unit": "s/100 trees",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 grad/hess, int32 histogram, f64 split math",
        "data": "synthetic (BASELINE.json configs[1] recipe), binned by the library's "
                "BinMapper (200k-row sample, max_bin 63)",
        "config": {"workload": "configs[1]: binary, 10.5M rows x 28 features, max_bin 63, "
                               "num_leaves 255, quantized int8 grads (4 bins, stochastic)",
                   "rows": n, "features": 28, "num_leaves": nl, "learning_rate": lr,
                   "timed_iterations": f"0-{args.steps - 1}"},
        "s_per_100_trees_iter0_99": (round(full100, 4) if full100 is not None
                                     else round(s_per_100, 4)),
        "pcie_inclusive": {
            "upload_s": round(upload_s, 4),
            "s_per_100_trees": round((full100 if full100 is not None else s_per_100)
                                     + upload_s, 4),
            "what": "iterations 0-99 plus one hand-over of the raw f32 table from host "
                    "memory (lgbm_hip_upload_raw: PCIe copy and device binning)"},
        "ms_per_step_median": round(sorted(runs)[len(runs) // 2] / args.steps * 1e3, 4),
        "ms_per_step_runs": [round(r / args.steps * 1e3, 4) for r in runs],
        "hist_GBps": round(hist_gbs, 2),
        "hist_GBps_root": round(root_gbs, 2),
        "roofline": {"bound": "hbm", "achieved": round(dom[1], 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(dom[1] / HBM_PEAK_GBS, 4),
                     "traffic": traffic_for(dom[0].split()[0]),
                     "kernel": dom[0],
                     "bytes_per_launch": round(dom[2] / max(dom[3], 1), 1),
                     "launches": int(dom[3]),
                     "avg_launch_us": round(dom[4] * 1e3 / max(dom[3], 1), 3),
                     "design_bytes_per_launch": round(design_bytes / max(launches, 1), 1),
                     "design_GBps": round(design_gbs, 2)},
        "parity": parity,
        "phase_ms_per_step": {k: round(tm[k] / tsteps, 4) for k in
                              ("hist_ms", "partition_ms", "scan_ms", "quant_ms", "objective_ms")},
        "cpu_baseline": cpu,
        "next_rows": {
            "binning": _line("k_bin_records (ValueToBin + record packing, f32 column-major "
                             "input)", bin_tm["bin_ms"], bin_tm["bin_launches"],
                             n * (28 * 4 + int(rec)), f"{n} rows x 28 features"),
            "predict": _line("k_predict (raw scores)", pred_tm["predict_ms"],
                             pred_tm["predict_launches"], pred_rows * (28 * 4 + 8),
                             f"{pred_rows} rows x {len(trees)} trees of {nl} leaves",
                             walks=pred_tm["predict_walks"]),
        },
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
