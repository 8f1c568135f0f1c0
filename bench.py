"""Benchmark: histogram GB/s + seconds per 100 trees, 10.5M x 28 quantized-grad, 1 MI355X.

One step = one boosting iteration of BASELINE.json configs[1] (binary logloss,
num_leaves 255, max_bin 63, int8 gradients with 4 quantization bins and stochastic
rounding) with every input resident in HBM: objective -> quantize -> grow the tree
(histogram, split scan, partition for all 254 splits) -> score update.  The raw
table is binned by the library (BinMapper on a 200k-row sample on the host, then
ValueToBin on the device) before the timed region; the binning kernel and a batch
prediction with the trained trees are reported as secondary lines (`next_rows`).

Prints ONE JSON line.  `value` is seconds per 100 trees (lower is better); the
histogram bandwidth of the dominant kernel is reported in `roofline`, timed with HIP
events on the library's own stream.  `cpu_baseline` times the CPU restatement of the
reference learner (oracle/) on a bounded sample of the same workload.
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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--rows", type=int, default=10_500_000)
    ap.add_argument("--num-leaves", type=int, default=255)
    ap.add_argument("--cpu-iters", type=int, default=2,
                    help="boosting iterations of the CPU baseline sample (0 disables)")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--prof-steps", type=int, default=3,
                    help="extra iterations timed per kernel with HIP events")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="after the run, copy a buffer of this many MiB device-to-device "
                         "(3 times): the known-size kernel that scales rocprofv3 "
                         "FETCH_SIZE/WRITE_SIZE readings to bytes")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on exactly one GPU (--gpus {args.gpus} requested): this build "
              "has no multi-GPU path; see DESIGN.md for how the path would shard.",
              file=sys.stderr)
        sys.exit(2)

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
    leaves, trees = [], []
    t2 = time.perf_counter()
    for i in range(args.warmup, args.warmup + args.steps):
        t = be.train_iter_binary(i, cfg, nl, -1, lr, 4, True, want_tree=True)
        leaves.append(t["num_leaves"])
        trees.append(t)
    torch.cuda.synchronize() if dev is not None else None
    elapsed = time.perf_counter() - t2
    # Per-kernel device time: HIP events around every launch on the library's stream.
    # The per-tree sequence then runs as individual launches (no graph), so this pass
    # measures kernel durations, not the timed loop's wall clock.
    be.set_lookahead(False)
    be.set_timing(True)
    it0 = args.warmup + args.steps
    for i in range(it0, it0 + args.prof_steps):
        be.train_iter_binary(i, cfg, nl, -1, lr, 4, True, want_tree=False)
    tm = be.timing()
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
    # Algorithmic bytes.  Root ConstructHistogram: rows x (F bin bytes + 2 B packed
    # g/h) + cells x 2 x 4 B written.  Partition round (also builds one child's
    # histogram per split): rows x (record + 2 B g/h) read and written + cells x 2 x
    # 4 B per split.
    root_bytes = tm["root_rows"] * (F + 2) + tm["hist_launches"] * cells * 8
    part_bytes = tm["partition_rows"] * 2 * (rec + 2) + tm["partition_jobs"] * cells * 8
    root_gbs = root_bytes / (tm["hist_ms"] * 1e-3) / 1e9 if tm["hist_ms"] > 0 else 0.0
    part_gbs = part_bytes / (tm["partition_ms"] * 1e-3) / 1e9 if tm["partition_ms"] > 0 else 0.0
    if tm["partition_ms"] >= tm["hist_ms"]:
        dom = ("k_partition (DataPartition + smaller-child ConstructHistogram, fused)", part_gbs,
               part_bytes, tm["partition_launches"], tm["partition_ms"])
    else:
        dom = ("k_hist_jobs (ConstructHistogram, root)", root_gbs, root_bytes, tm["hist_launches"],
               tm["hist_ms"])
    log(f"gpu: {ms_per_step:.2f} ms/step, leaves {min(leaves)}..{max(leaves)}, timing {tm}")

    cpu = None
    if args.cpu_iters > 0:
        from oracle import oracle
        from lightgbm_rs_amd import feature_meta
        meta = [feature_meta(m.num_bin, m.most_freq_bin, m.missing_type, m.default_bin, f)
                for f, m in enumerate(mappers)]
        ub = np.concatenate([m.upper_bounds for m in mappers])
        threads = args.cpu_threads or (os.cpu_count() or 1)
        threads = oracle.set_threads(threads)
        tc = time.perf_counter()
        oracle.train_binary(bins, meta, ub, y, cfg, nl, -1, args.cpu_iters, lr,
                            boost_from_average=True, quantized=True, quant_bins=4,
                            stochastic=True, want_trees=False)
        cs = time.perf_counter() - tc
        cpu = {"value": cs / args.cpu_iters * 100.0, "unit": "s/100 trees", "cores": threads,
               "kind": "port",
               "sample": f"{args.cpu_iters} boosting iterations of the same {n}x28 workload "
                         f"(C++ restatement of the reference CpuBackend learner, OpenMP), "
                         f"extrapolated to 100 trees; {cs:.1f}s measured"}
        log(f"cpu: {cs:.1f}s for {args.cpu_iters} iters on {threads} threads")

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
                   "rows": n, "features": 28, "num_leaves": nl, "learning_rate": lr},
        "hist_GBps_root": round(root_gbs, 2),
        "partition_hist_GBps": round(part_gbs, 2),
        "roofline": {"bound": "hbm", "achieved": round(dom[1], 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(dom[1] / HBM_PEAK_GBS, 4),
                     "traffic": traffic_for(dom[0].split()[0]),
                     "kernel": dom[0],
                     "bytes_per_launch": round(dom[2] / max(dom[3], 1), 1),
                     "launches": int(dom[3]),
                     "avg_launch_us": round(dom[4] * 1e3 / max(dom[3], 1), 3)},
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
