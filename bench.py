"""Benchmark of the MI355X oblivious-tree training path (headline config 2).

Workload: Logloss, 10M rows x 200 features (100 N(0,1) + 100 lognormal(0,1)), 254
borders (u8 bins, 4 per u32 word), depth 6, Bayesian bootstrap T=1, synthetic seeded
data.  A step is one boosting iteration (one tree) through the C-ABI
(``cbt_step`` -> ``cbh_session_grow``); the bins, target and approximant are resident in
HBM before the timed region starts.  Each step ends with a stream synchronisation (the
tree is copied back), so wall time around the steps is the device time of the steps.

Reported next to the GPU figure:
  * roofline of the dominant kernel (histogram fill): algorithmic bytes per launch
    (V rows x (W*4 + 8*(K+1) + 4) + histogram bytes) / average launch time from HIP events
    recorded on the session stream, against MI355X's 8 TB/s;
  * cpu_baseline: the CPU restatement of the reference algorithm (oracle/) timed on the
    host cores for a few trees of the same data.

Usage: python bench.py [--gpus 1] [--steps 200] [--warmup 3] [--rows N] [--cpu-trees 2]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = ("histogram rows·features/s + HBM GB/s; boosting iters/s at 10M×200, depth 6")
HBM_PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _profiled_traffic(n, F):
    """HBM bytes per fill launch measured by rocprofv3 (FETCH_SIZE + WRITE_SIZE, copy-calibrated)
    for this workload shape, read from the committed profile summary; None if absent."""
    path = os.path.join(ROOT, "profiles", "fill_kernel_config2.md")
    if n != 10_000_000 or F != 200 or not os.path.exists(path):
        return None
    import re

    m = re.search(r"mean per dispatch: fetch ([0-9.]+) GB write ([0-9.]+) GB", open(path).read())
    return round((float(m.group(1)) + float(m.group(2))) * 1e9) if m else None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--rows", type=int, default=10_000_000)
    ap.add_argument("--features", type=int, default=200)
    ap.add_argument("--cpu-trees", type=int, default=2)
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calib", type=int, default=0,
                    help="only copy this many bytes device-to-device (counter calibration)")
    args = ap.parse_args()
    if args.copy_calib:
        import torch

        a = torch.empty(args.copy_calib, dtype=torch.uint8, device="cuda:0")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        log(f"copied {args.copy_calib} bytes x3")
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the multi-GPU "
              "row-parallel (integer histogram all-reduce) design is not built in this library.", file=sys.stderr)
        sys.exit(2)

    import numpy as np

    import catboost_rs_amd as cb
    from catboost_rs_amd import datagen

    cb.load()
    t0 = time.perf_counter()
    data = datagen.config2(n_rows=args.rows, n_features=args.features)
    bins, nb, y = data["bins"], data["n_borders"], data["target"]
    P = data["params"]
    F, n = bins.shape
    n_bins = int(nb.max()) + 1
    log(f"data: {n} x {F}, max borders {int(nb.max())}, generated in {time.perf_counter() - t0:.1f}s")

    t0 = time.perf_counter()
    tr = cb.Trainer(bins, n_bins, y, loss=P["loss"], depth=P["depth"], learning_rate=P["learning_rate"],
                    l2_leaf_reg=P["l2_leaf_reg"], score=P["score"], leaf_method=P["leaf_method"],
                    bootstrap_type=P["bootstrap_type"], bagging_temperature=P["bagging_temperature"],
                    boost_from_average=P["boost_from_average"], random_seed=P["random_seed"],
                    real_folds=nb + 1, profile=True)
    log(f"session open (upload + pack) {time.perf_counter() - t0:.2f}s")
    for _ in range(args.warmup):
        tr.step()
    tr.reset_stats()
    t0 = time.perf_counter()
    gpu_splits = []
    for _ in range(args.steps):
        s, _, _ = tr.step()
        gpu_splits.append(s)
    wall = time.perf_counter() - t0
    st = tr.stats()
    tr.close()
    iters_per_s = args.steps / wall
    ms_per_step = 1000.0 * wall / args.steps
    fill_s = st["fill_ms"] / 1000.0
    achieved = st["fill_bytes"] / 1e9 / fill_s if fill_s > 0 else 0.0
    log(f"gpu: {iters_per_s:.2f} iters/s, {ms_per_step:.3f} ms/tree; stage ms/tree: " +
        ", ".join(f"{k[:-3]} {st[k] / args.steps:.3f}" for k in
                  ("fill_ms", "derive_ms", "score_ms", "partition_ms", "leaf_ms", "prepare_ms")))
    log(f"fill: {st['fill_launches']} launches, avg {st['fill_ms'] / max(1, st['fill_launches']):.4f} ms, "
        f"{achieved:.1f} GB/s algorithmic")

    # LDS-atomic roofline of the fill: every visited (row, feature) adds K+1 64-bit integer
    # cells; the cap is the scattered 64-bit LDS atomic rate measured on this GPU
    lds = None
    lane_atomics = st["fill_row_features"] * 2
    probe = os.path.join(ROOT, "catboost_rs_amd", "lds_atomic_rate")
    if os.path.exists(probe):
        import subprocess

        r = subprocess.run([probe], capture_output=True, text=True, timeout=120)
        rates = dict((l.split()[0], float(l.split()[1])) for l in r.stdout.splitlines() if len(l.split()) == 2)
        if "scattered_u64" in rates and fill_s > 0:
            ach = lane_atomics / fill_s
            lds = {"achieved_lane_atomics_per_s": round(ach, 1),
                   "cap_scattered_u64_per_s": rates["scattered_u64"],
                   "cap_contiguous_u64_per_s": rates.get("contiguous_u64"),
                   "frac_of_scattered_cap": round(ach / rates["scattered_u64"], 4)}
            log(f"fill LDS atomics: {ach:.3e}/s = {100 * ach / rates['scattered_u64']:.1f}% of the "
                f"measured scattered-u64 cap {rates['scattered_u64']:.3e}/s")
    traffic = _profiled_traffic(n, F)

    cpu = None
    if not args.no_cpu and args.cpu_trees > 0:
        from oracle import oracle as O

        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        t0 = time.perf_counter()
        exp = O.train(bins, nb, y, loss=P["loss"], depth=P["depth"], iterations=args.cpu_trees,
                      learning_rate=P["learning_rate"], l2_leaf_reg=P["l2_leaf_reg"], score=P["score"],
                      leaf_method=P["leaf_method"], bootstrap_type=P["bootstrap_type"],
                      bagging_temperature=P["bagging_temperature"],
                      boost_from_average=P["boost_from_average"], random_seed=P["random_seed"],
                      n_threads=threads)
        cpu_wall = time.perf_counter() - t0
        cpu = {"value": round(args.cpu_trees / cpu_wall, 6), "unit": "iters/s", "cores": threads,
               "kind": "port",
               "sample": f"first {args.cpu_trees} trees of the same {n}x{F} workload "
                         f"(CPU restatement of the reference algorithm, OpenMP over features)"}
        log(f"cpu: {args.cpu_trees} trees in {cpu_wall:.1f}s on {threads} threads")
        # the CPU trees must be the GPU run's first trees (parity on the full-size workload)
        tr2 = cb.Trainer(bins, n_bins, y, loss=P["loss"], depth=P["depth"], learning_rate=P["learning_rate"],
                         l2_leaf_reg=P["l2_leaf_reg"], score=P["score"], leaf_method=P["leaf_method"],
                         bootstrap_type=P["bootstrap_type"], bagging_temperature=P["bagging_temperature"],
                         boost_from_average=P["boost_from_average"], random_seed=P["random_seed"],
                         real_folds=nb + 1)
        first, _ = tr2.fit(args.cpu_trees)
        tr2.close()
        cpu["splits_match_gpu"] = bool(np.array_equal(first, exp["splits"]))

    out = {
        "metric": METRIC,
        "value": round(iters_per_s, 4),
        "unit": "iters/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8 bins, int64 fixed-point sums, f64 scores",
        "data": "synthetic (seeded; datagen.config2)",
        "config": {"workload": "config2: Logloss, Bayesian bootstrap T=1, depth 6, 254 borders",
                   "rows": n, "features": F, "depth": P["depth"], "parallelism": "single GPU"},
        "hist_rows_features_per_s": round(st["fill_row_features"] / fill_s, 1) if fill_s else None,
        "hist_rows_features_per_s_logical": round(n * F * P["depth"] * args.steps / fill_s, 1) if fill_s else None,
        "stage_ms_per_tree": {k[:-3]: round(st[k] / args.steps, 4) for k in
                              ("fill_ms", "derive_ms", "score_ms", "partition_ms", "leaf_ms", "prepare_ms")},
        "roofline": {"bound": "hbm", "kernel": "fill_kernel", "achieved": round(achieved, 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "launches": st["fill_launches"],
                     "avg_launch_ms": round(st["fill_ms"] / max(1, st["fill_launches"]), 5),
                     "algorithmic_bytes_per_launch": round(st["fill_bytes"] / max(1, st["fill_launches"]))},
        "lds_atomic_roofline": lds,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
