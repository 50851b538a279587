"""Benchmark of the MI355X oblivious-tree training path.

Default workload (the headline metric): config 2 -- Logloss, 10M rows x 200 features
(100 N(0,1) + 100 lognormal(0,1)), 254 borders (u8 bins, 4 per u32 word), depth 6,
Bayesian bootstrap T=1, synthetic seeded data.  ``--config 1|3|4|5`` measures the other
configs of the scope the same way (config 3 = PairLogit over query groups with pairs,
``--pairwise`` for PairLogitPairwise; config 4 = RMSE over 30 floats + 20 categorical
columns as online CTR columns built on the device; config 5 = MultiClass K=10, depth 8,
4096 features).

A step is one boosting iteration (one tree) through the C-ABI (``cbt_step`` ->
``cbh_session_grow``); the bins, target and approximant are resident in HBM before the
timed region starts.  Each step ends with a stream synchronisation (the tree is copied
back), so wall time around the steps is the device time of the steps.  After the first
tree, a tree replays one recorded launch sequence (HIP graph); a short profiled
continuation of the same fit then runs eager trees with HIP events around every stage
for the stage breakdown and the fill roofline.

Reported next to the GPU figure:
  * roofline of the dominant kernel (histogram fill): algorithmic bytes per launch
    (V rows x (W*4 + S + 4) + histogram bytes, S = bytes of a row's statistics: 8 for the
    packed and count-packed fills, 8*ceil((K+1)/2) for the packed multi-channel fills,
    8*(K+1) otherwise) / average launch time from HIP events
    recorded on the session stream, against MI355X's 8 TB/s; HBM traffic per launch from
    the copy-calibrated rocprofv3 FETCH_SIZE / WRITE_SIZE summary in profiles/;
  * the fill's LDS-atomic rate against the measured conflict-free 64-bit LDS atomic cap;
  * cpu_baseline: the CPU restatement of the reference algorithm (oracle/) timed on the
    host cores for the first trees of the same data, with a check that its splits equal
    the GPU's;
  * reference_published_cells (config 2): the reference's own published speed cells (a
    whole fit of 30 trees from a row-major f32 matrix, then a 1024-row prediction) timed on
    this GPU, next to the seconds the reference publishes for them on a Tesla P100.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 2] [--rows N]
"""
from __future__ import annotations

import argparse
import json
import os
import re
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "histogram rows·features/s + HBM GB/s; boosting iters/s at 10M×200, depth 6"
HBM_PEAK_GBS = 8000.0
DEFAULT_STEPS = {1: 100, 2: 200, 3: 100, 4: 200, 5: 20}
DEFAULT_CPU_TREES = {1: 5, 2: 5, 3: 3, 4: 3, 5: 1}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _profile_facts(config, n, F, kernel):
    """(traffic, limiter) of the fill kernel from the committed profile summary of the same
    kernel on the same bench command: HBM bytes per launch measured by rocprofv3 (FETCH_SIZE +
    WRITE_SIZE, copy-calibrated; its last 120 fill dispatches are the 20 profiled trees this
    line's avg_launch_ms and algorithmic bytes come from) and the bound its SQ counters show;
    (None, None) if absent or of another kernel or shape."""
    path = os.path.join(ROOT, "profiles", "fill_kernel_config2.md")
    if config != 2 or n != 10_000_000 or F != 200 or not os.path.exists(path):
        return None, None
    text = open(path).read()
    k = re.search(r"^kernel: (\S+)", text, re.M)
    m = re.search(r"mean per dispatch: fetch ([0-9.]+) GB write ([0-9.]+) GB", text)
    lim = re.search(r"^limiter: (.+)$", text, re.M)
    if not k or k.group(1) != kernel or not m:
        return None, None
    return round((float(m.group(1)) + float(m.group(2))) * 1e9), (lim.group(1).strip() if lim else None)


def _lds_rates():
    probe = os.path.join(ROOT, "catboost_rs_amd", "lds_atomic_rate")
    if not os.path.exists(probe):
        return {}
    r = subprocess.run([probe], capture_output=True, text=True, timeout=120)
    return dict((l.split()[0], float(l.split()[1])) for l in r.stdout.splitlines() if len(l.split()) == 2)


def _workload(args):
    from catboost_rs_amd import datagen

    if args.config == 1:
        return datagen.config1(scale=args.rows / 100_000 if args.rows else 1.0)
    if args.config == 2 and args.quantile_borders:
        return datagen.config2(n_rows=args.rows or 10_000_000, n_features=args.features or 200)
    if args.config == 2:
        return _config2_raw(args.rows or 10_000_000, args.features or 200)
    if args.config == 3:
        return datagen.config3(n_rows=args.rows or 1_000_000, n_features=args.features or 100,
                               loss="PairLogitPairwise" if args.pairwise else "PairLogit")
    if args.config == 4:
        return _config4(args.rows or 2_000_000)
    if args.config == 5:
        return datagen.config5(n_rows=args.rows or 1_000_000, n_features=args.features or 4096)
    raise SystemExit(f"--config {args.config}: configs 1 to 5 are measured")


def _config2_raw(n, F):
    """Config 2 as a user feeds it: raw f32 columns, 254 GreedyLogSum borders selected on the
    device (cbh_select_borders), the session opened over the raw float channel (the device
    quantizes the columns).  Border selection is timed here, outside the boosting steps."""
    import numpy as np

    import catboost_rs_amd as cb
    from catboost_rs_amd import datagen

    d = datagen.config2_raw(n_rows=n, n_features=F)
    P = d["params"]
    t0 = time.perf_counter()
    borders = cb.select_borders(d["floats"], P["border_count"], "Min", P["border_type"])
    d["borders_s"] = time.perf_counter() - t0
    d["borders"] = borders
    d["n_borders"] = np.array([b.size for b in borders], np.uint32)
    return d


def _config4(n):
    """Config 4 with its categorical columns as Borders CTR columns (prior 0.5, 16 bins) built
    on the device over the learn permutation: the reference-legal all-CTR variant."""
    import numpy as np

    import catboost_rs_amd as cb
    from catboost_rs_amd import datagen

    d = datagen.config4(n_rows=n)
    P = d["params"]
    # learn permutation S and averaging permutation Q = S[P_avg] off one seeded stream
    two = cb.shuffled_indices(n, P["random_seed"], count=2)
    perm, avg_perm = two[0], two[0][two[1]]
    t0 = time.perf_counter()
    ctr, counts = cb.ctr_bin_columns(d["cat_keys"], perm, d["target_class"], [P["ctr"]], P["ctr_border_count"])
    avg, _ = cb.ctr_bin_columns(d["cat_keys"], avg_perm, d["target_class"], [P["ctr"]], P["ctr_border_count"])
    buckets = np.stack([cb.perfect_hash(k)[0] for k in d["cat_keys"]])
    ctr_s = time.perf_counter() - t0
    bc = P["ctr_border_count"]
    d["bins"] = np.concatenate([d["bins"], ctr], 0)
    d["n_borders"] = np.concatenate([d["n_borders"], np.full(ctr.shape[0], bc, np.uint32)])
    d["ctr"] = dict(avg_bins=avg, bucket_count=counts.astype(np.uint32),
                    group=np.arange(len(counts), dtype=np.uint32), cat_buckets=buckets,
                    cat_bucket_count=counts.astype(np.uint32), model_size_reg=0.5)
    d["ctr_s"] = ctr_s
    log(f"config 4 CTR columns: {ctr.shape[0]} x 2 permutations built on the device in {ctr_s:.3f}s "
        f"(bucket counts {counts.min()}..{counts.max()})")
    return d


def _train_kwargs(P):
    return dict(loss=P["loss"], depth=P["depth"], learning_rate=P["learning_rate"],
                l2_leaf_reg=P["l2_leaf_reg"], score=P["score"], leaf_method=P["leaf_method"],
                bootstrap_type=P["bootstrap_type"], bagging_temperature=P.get("bagging_temperature", 1.0),
                subsample=P.get("subsample", 0.66), boost_from_average=P["boost_from_average"],
                random_seed=P.get("random_seed", 0), approx_dim=P.get("approx_dim", 1))


def prep_bench(args):
    """Float-feature preparation at config 2's size (10M x 200 f32 columns, 254 GreedyLogSum
    borders): device border selection (host subset gather, device NaN drop + segmented
    radix sort, host greedy heap) and the raw-channel session open (PCIe upload + device
    quantize + row packing).  The quantize kernel's roofline comes from HIP events around
    its launches (algorithmic bytes: 4 read + 1 written per value)."""
    import numpy as np

    import catboost_rs_amd as cb
    from catboost_rs_amd import datagen

    n, F = args.rows or 10_000_000, args.features or 200
    t0 = time.perf_counter()
    X = datagen.config2_floats(n, F)
    y = np.zeros(n)
    log(f"prep data: {n} x {F} f32 generated in {time.perf_counter() - t0:.1f}s")
    cb.select_borders(X[:2, :1000], 254)  # load the library / first-use costs
    sel = []
    for _ in range(3):
        t0 = time.perf_counter()
        borders = cb.select_borders(X, 254, "Min")
        sel.append(time.perf_counter() - t0)
    sel_s = min(sel)
    log(f"select_borders: {', '.join(f'{v:.3f}' for v in sel)} s")
    opens, st = [], None
    for _ in range(2):
        t0 = time.perf_counter()
        tr = cb.Trainer.from_floats(X, borders, y, loss="Logloss", depth=6, profile=True)
        opens.append(time.perf_counter() - t0)
        st = tr.stats()
        tr.close()
    open_s = min(opens)
    q_s = st["quantize_ms"] / 1000.0
    q_gbs = st["quantize_bytes"] / 1e9 / q_s if q_s > 0 else 0.0
    log(f"raw open: {', '.join(f'{v:.3f}' for v in opens)} s; quantize {st['quantize_launches']} launches, "
        f"{st['quantize_ms']:.3f} ms, {q_gbs:.1f} GB/s algorithmic")
    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O

        k = 4
        t0 = time.perf_counter()
        cpu_b = [O.select_borders(X[f], 254, bool(np.isnan(X[f]).any())) for f in range(k)]
        for f in range(k):
            O.quantize(X[f], cpu_b[f])
        cpu_s = time.perf_counter() - t0
        cpu = {"value": round(k / cpu_s, 4), "unit": "columns/s", "cores": 1, "kind": "port",
               "sample": f"borders + quantize of the first {k} of the same {n}-row columns "
                         "(CPU restatement: greedy borders over the 200000-row subset, bin_of)",
               "borders_match_gpu": all(np.array_equal(a, b) for a, b in zip(cpu_b, borders[:k]))}
        log(f"cpu: {k} columns in {cpu_s:.1f}s")
    out = {
        "metric": "float feature preparation (greedy borders + quantize + pack), columns/s",
        "value": round(F / (sel_s + open_s), 3), "unit": "columns/s", "n_gpus": 1,
        "higher_is_better": True, "dtype": "f32 values, f64 borders, u8 bins",
        "data": "synthetic (seeded; datagen.config2_floats)",
        "config": {"workload": "config2 float columns", "rows": n, "features": F, "border_count": 254},
        "select_borders_s": round(sel_s, 4), "raw_open_s_pcie_inclusive": round(open_s, 4),
        "roofline": {"bound": "hbm", "kernel": "quantize_kernel", "achieved": round(q_gbs, 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(q_gbs / HBM_PEAK_GBS, 4),
                     "traffic": None, "launches": st["quantize_launches"],
                     "avg_launch_ms": round(st["quantize_ms"] / max(1, st["quantize_launches"]), 5),
                     "algorithmic_bytes_per_launch": round(st["quantize_bytes"] / max(1, st["quantize_launches"]))},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--pairwise", action="store_true", help="config 3 with PairLogitPairwise")
    ap.add_argument("--quantile-borders", action="store_true",
                    help="config 2 from host bins over quantile borders instead of raw floats")
    ap.add_argument("--steps", type=int, default=0)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--rows", type=int, default=0)
    ap.add_argument("--features", type=int, default=0)
    ap.add_argument("--cpu-trees", type=int, default=-1)
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-published", action="store_true",
                    help="config 2: leave out the reference's published speed cells")
    ap.add_argument("--bootstrap", default="",
                    help="override the config's bootstrap type (a measurement option; the line then names it)")
    ap.add_argument("--prep", action="store_true",
                    help="measure float-feature preparation (borders, quantize) instead of boosting")
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
              "row-parallel (integer histogram all-reduce) design is not built in this library.",
              file=sys.stderr)
        sys.exit(2)
    if args.prep:
        prep_bench(args)
        return
    steps = args.steps or DEFAULT_STEPS.get(args.config, 50)
    cpu_trees = args.cpu_trees if args.cpu_trees >= 0 else DEFAULT_CPU_TREES.get(args.config, 1)

    import numpy as np

    import catboost_rs_amd as cb

    cb.load()
    t0 = time.perf_counter()
    data = _workload(args)
    raw = "floats" in data
    bins, nb, y = data.get("bins"), data["n_borders"], data["target"]
    P = data["params"]
    if args.bootstrap:
        P = dict(P, bootstrap_type=args.bootstrap)
    F, n = (data["floats"] if raw else bins).shape
    n_bins = int(nb.max()) + 1
    kw = _train_kwargs(P)
    pairs, go = data.get("pairs"), data.get("group_offsets")
    log(f"data: config {args.config} {P['loss']}: {n} x {F}, max borders {int(nb.max())}"
        + (f", {len(pairs[0])} pairs" if pairs is not None else "")
        + (f", {P['border_type']} borders selected on the device in {data['borders_s']:.3f}s" if raw else "")
        + f", generated in {time.perf_counter() - t0:.1f}s")

    t0 = time.perf_counter()
    ctr = data.get("ctr")

    def open_trainer(profile):
        if raw:   # raw f32 columns: the device quantizes them
            return cb.Trainer.from_floats(data["floats"], data["borders"], y, profile=profile, **kw)
        return cb.Trainer(bins, n_bins, y, real_folds=nb + 1, profile=profile, pairs=pairs, group_offsets=go,
                          ctr=ctr, **kw)

    tr = open_trainer(False)
    log(f"session open (upload{' + device quantize' if raw else ''} + pack) {time.perf_counter() - t0:.2f}s")
    for _ in range(args.warmup):
        tr.step()
    # timed region: trees as a caller runs them (after the first, each tree replays one
    # recorded launch sequence)
    t0 = time.perf_counter()
    for _ in range(steps):
        tr.step()
    wall = time.perf_counter() - t0
    # profiled continuation of the same fit: eager launches with HIP events around every
    # stage on the session stream, for the stage breakdown and the fill roofline
    prof_steps = max(3, min(steps, 20))
    tr.set_profile(True)
    tr.step()
    tr.reset_stats()
    t1 = time.perf_counter()
    for _ in range(prof_steps):
        tr.step()
    prof_wall = time.perf_counter() - t1
    st = tr.stats()
    tr.close()
    iters_per_s = steps / wall
    ms_per_step = 1000.0 * wall / steps
    fill_s = st["fill_ms"] / 1000.0
    achieved = st["fill_bytes"] / 1e9 / fill_s if fill_s > 0 else 0.0
    stages = ("fill_ms", "derive_ms", "score_ms", "partition_ms", "leaf_ms", "prepare_ms")
    log(f"gpu: {iters_per_s:.2f} iters/s, {ms_per_step:.3f} ms/tree (profiled eager trees: "
        f"{1000.0 * prof_wall / prof_steps:.3f} ms/tree); stage ms/tree: " +
        ", ".join(f"{k[:-3]} {st[k] / prof_steps:.3f}" for k in stages))
    log(f"fill: {st['fill_launches']} launches, avg {st['fill_ms'] / max(1, st['fill_launches']):.4f} ms, "
        f"{achieved:.1f} GB/s algorithmic")

    # LDS-atomic roofline of the fill: every (row, feature) entry the fill adds costs one 64-bit
    # LDS atomic (packed and count-packed fills: both channels in one word), ceil((K+1)/2)
    # (packed multi-channel fills: two channels per word, one fewer at level 0 when the weight's
    # plane comes from its cache) or K+1 (two-channel / channel-split fills); the library counts
    # the lane atomics issued (cbh_stats.fill_lane_atomics) over the profiled trees, with the
    # dominant-bin skip over the issued entries only (bins other than the feature's dominant
    # bin).  The cap is the contiguous (conflict-free) 64-bit LDS atomic rate measured on this
    # GPU, the pattern the fills' rotated lane layouts reach
    lds = None
    rates = _lds_rates()
    if "contiguous_u64" in rates and fill_s > 0:
        entries = st["fill_entries"] if st["skip_features"] else st["fill_row_features"]
        issued = st["fill_lane_atomics"]
        per_pair = round(issued / entries, 4) if entries else 0.0
        ach = issued / fill_s
        lds = {"achieved_lane_atomics_per_s": round(ach, 1),
               "atomics_per_entry": per_pair,
               "lane_atomics": issued,
               "entries": entries,
               "counted_as": "all (row, feature) pairs" if not st["skip_features"] else
               f"issued: the {entries} (row, feature) entries whose bin is not the feature's dominant bin, "
               f"of {st['fill_row_features']} visited pairs ({st['skip_features']} of {F} features skip "
               f"their dominant bin)",
               "cap_contiguous_u64_per_s": rates["contiguous_u64"],
               "frac_of_contiguous_cap": round(ach / rates["contiguous_u64"], 4)}
        log(f"fill LDS atomics: {ach:.3e}/s ({per_pair} per entry, {entries} entries) = "
            f"{100 * ach / rates['contiguous_u64']:.1f}% of the measured conflict-free 64-bit cap "
            f"{rates['contiguous_u64']:.3e}/s")

    cpu = None
    if not args.no_cpu and cpu_trees > 0:
        from oracle import oracle as O

        # the host threads this process may use (nproc), capped by the box's CPU share when the
        # environment states one (OMP_NUM_THREADS: 16 per GPU on the GPU boxes)
        nproc = len(os.sched_getaffinity(0))
        threads = args.cpu_threads or min(nproc, int(os.environ.get("OMP_NUM_THREADS") or nproc))
        if raw:   # the oracle's bins: the same borders, quantized on the host (bin_of)
            from catboost_rs_amd import datagen

            bins = datagen.quantize_columns(data["floats"], data["borders"])
        t0 = time.perf_counter()
        exp = O.train(bins, nb, y, iterations=cpu_trees, n_threads=threads, pairs=pairs, ctr=ctr, **kw)
        cpu_wall = time.perf_counter() - t0
        cpu = {"value": round(cpu_trees / cpu_wall, 6), "unit": "iters/s", "cores": threads, "nproc": nproc,
               "kind": "port",
               "sample": f"first {cpu_trees} trees of the same {n}x{F} workload "
                         f"(CPU restatement of the reference algorithm, OpenMP over features)"}
        log(f"cpu: {cpu_trees} trees in {cpu_wall:.1f}s on {threads} threads")
        # the CPU trees must be the GPU run's first trees (parity on the full-size workload)
        tr2 = open_trainer(False)
        first, _ = tr2.fit(cpu_trees)
        tr2.close()
        cpu["splits_match_gpu"] = bool(np.array_equal(first, exp["splits"]))
        if args.config == 1:   # the single-core leg of the CPU baseline (the whole fit)
            t0 = time.perf_counter()
            O.train(bins, nb, y, iterations=P["iterations"], n_threads=1, pairs=pairs, ctr=ctr, **kw)
            one = time.perf_counter() - t0
            cpu["single_core"] = {"value": round(P["iterations"] / one, 4), "unit": "iters/s", "cores": 1,
                                  "sample": f"all {P['iterations']} trees of the same workload"}
            log(f"cpu: {P['iterations']} trees in {one:.1f}s on 1 thread")

    traffic, limiter = None, None   # (set below from the committed profile)
    fill_kernel = {0: "fill_kernel", 1: "fill_packed_kernel", 2: "fill_exact_kernel",
                   3: "fill_pkk_kernel", 4: "fill_pks_kernel", 5: "fill_packed_kernel"}[st["fill_mode"]]
    traffic, limiter = _profile_facts(args.config, n, F, fill_kernel)
    names = {1: "config1: RMSE, no bootstrap, depth 6, 128 borders",
             2: ("config2: Logloss, Bayesian bootstrap T=1, depth 6, 254 GreedyLogSum borders selected on the "
                 "device from the raw f32 columns, quantized on the device" if raw else
                 "config2: Logloss, Bayesian bootstrap T=1, depth 6, 254 quantile borders (host bins)"),
             3: f"config3: {P['loss']}, groups of 20, ~10 pairs per group, depth 6, 254 borders",
             4: "config4: RMSE, Bernoulli 0.66, depth 6, 30 float (254 borders) + 20 categorical as "
                "Borders CTR columns (prior 0.5, 16 bins; model_size_reg 0.5, averaging-permutation leaves), "
                "max_ctr_complexity=1 (single-feature CTR projections; the reference's default 4 also scores "
                "feature combinations)",
             5: "config5: MultiClass K=10, depth 8, 64 borders, 70% zeros"}
    out = {
        "metric": METRIC,
        "value": round(iters_per_s, 4),
        "unit": "iters/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": (f"u8 bins; int64 fixed-point histogram sums, a row's value v entering as round(v * 2^S): "
                  f"S = {st['score_shift_der']} (der), {st['score_shift_w']} (weight) in the last tree "
                  f"(the reference: 2^30); f64 scores"
                  if st["fill_mode"] in (0, 2) else
                  f"u8 bins; int64 fixed-point histogram sums: der rows as round(v * 2^{st['score_shift_der']}) "
                  f"(the reference: 2^30), integer weights exact; f64 scores"
                  if st["fill_mode"] == 5 else
                  f"u8 bins; int64 sums of rows rounded to {st['fill_pack_bits']}-bit fields of the tree's "
                  f"largest row (coarser than the reference's 2^-30); f64 scores"),
        "fill": {0: "generic 32-feature tiles (one 64-bit atomic per channel, full fixed-point scale)", 1: f"packed 64-feature tiles ({st['fill_pack_bits']}-bit rows)",
                 2: "tiled exact 32-feature tiles (one 64-bit atomic per channel, full fixed-point scale)",
                 3: f"packed multi-channel 32-feature tiles (two channels per word, {st['fill_pack_bits']}-bit rows)",
                 4: f"packed multi-channel 32-feature tiles over sparse entries (a row per 16-lane DPP row, "
                    f"two channels per word, {st['fill_pack_bits']}-bit rows)",
                 5: "count-packed 64-feature tiles (der at >= 2^-30 and the integer weight in one 64-bit atomic)",
                 }[st["fill_mode"]],
        "data": f"synthetic (seeded; datagen.config{args.config}{'_raw' if raw else ''})",
        "config": {"workload": names[args.config] + (f" (bootstrap overridden: {args.bootstrap})"
                                                     if args.bootstrap else ""),
                   "rows": n, "features": F, "depth": P["depth"],
                   "parallelism": "single GPU"},
        "hist_rows_features_per_s": round(st["fill_row_features"] / fill_s, 1) if fill_s else None,
        "hist_rows_features_per_s_logical": round(n * F * P["depth"] * prof_steps / fill_s, 1) if fill_s else None,
        "stage_ms_per_tree": {k[:-3]: round(st[k] / prof_steps, 4) for k in stages},
        "profiled_trees": prof_steps,
        "ms_per_step_profiled_eager": round(1000.0 * prof_wall / prof_steps, 4),
        "roofline": {"bound": "hbm", "kernel": fill_kernel, "achieved": round(achieved, 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "traffic_source": "rocprofv3 FETCH_SIZE + WRITE_SIZE (copy-calibrated) of the last 120 fill "
                                       "dispatches of this command, profiles/fill_kernel_config2.md"
                                       if traffic else None,
                     "limiter": limiter,
                     "launches": st["fill_launches"],
                     "avg_launch_ms": round(st["fill_ms"] / max(1, st["fill_launches"]), 5),
                     "algorithmic_bytes_per_launch": round(st["fill_bytes"] / max(1, st["fill_launches"]))},
        "lds_atomic_roofline": lds,
        "cpu_baseline": cpu,
    }
    if "ctr_s" in data:
        out["ctr_columns_s"] = round(data["ctr_s"], 4)
    if raw:
        out["select_borders_s"] = round(data["borders_s"], 4)
    if args.config == 2 and not args.no_published:
        try:
            out["reference_published_cells"] = _reference_cells()
        except Exception as e:   # an informational block: it never voids the measurement
            out["reference_published_cells"] = {"error": repr(e)}
    print(json.dumps(out), flush=True)


# The reference's published GPU fit wall-clock (seconds per fit, median of 3, Tesla P100;
# bench/full_param_gpu_speed/kaggle-output-260808-r6/report.md:13,17,29,33): catboost_rs and
# official CatBoost 1.2.10 with task_type GPU, for the SymmetricTree cells without weights or CTRs.
REFERENCE_CELLS = (("RMSE", 300_000, 0.435, 1.223), ("Logloss", 300_000, 0.460, 1.434),
                   ("RMSE", 1_000_000, 0.992, 1.661), ("Logloss", 1_000_000, 0.987, 1.838))


def _reference_cells():
    """The reference's published speed cells on this GPU, timed as its grid times them
    (bench/full_param_gpu_speed/bench.py:51-62,545-572): fit(X, y) from a row-major f32 X in
    host memory -- the columns of X, 32 GreedyLogSum borders per feature, the session open
    (upload, device quantization), 30 depth-6 trees (L2 score, Gradient leaves, no bootstrap,
    no boost from average, learning rate 0.1, L2 3.0) -- plus a prediction of the first 1024
    rows; one untimed warm fit (whose predictions are checked against the training
    approximant), then the median of 3.  Other hardware than the reference's numbers (a
    Tesla P100), the same recipe."""
    import numpy as np

    import catboost_rs_amd as cb
    from catboost_rs_amd import datagen

    cells = []
    for loss, n, ref_s, off_s in REFERENCE_CELLS:
        X, y = datagen.reference_speed_cell(n, 50, classification=loss == "Logloss")

        def fit_once(check=False):
            t = [time.perf_counter()]
            cols = cb.columns_from_rows(X)
            t.append(time.perf_counter())
            borders = cb.select_borders(cols, 32, "Min", "GreedyLogSum")
            t.append(time.perf_counter())
            tr = cb.Trainer.from_floats(cols, borders, y, loss=loss, depth=6, learning_rate=0.1,
                                        l2_leaf_reg=3.0, score="L2", leaf_method="Gradient",
                                        bootstrap_type="No", boost_from_average=False)
            t.append(time.perf_counter())
            try:
                splits, leaves = tr.fit(30)
                approx = tr.approx()[0, :1024] if check else None
            finally:
                tr.close()
            t.append(time.perf_counter())
            sf = np.concatenate([sp[:, 0] for sp in splits]).astype(np.uint32)
            sb = np.array([borders[f][b] for sp in splits for f, b in sp], np.float64)
            so = np.arange(0, 6 * len(splits) + 1, 6, dtype=np.uint32)
            lv = np.concatenate([lvs[0] for lvs in leaves]).astype(np.float64)
            lo = np.arange(0, 64 * len(splits) + 1, 64, dtype=np.uint32)
            pred = cb.apply_oblivious(cols[:, :1024], sf, sb, so, lv, lo)
            t.append(time.perf_counter())
            if check and not np.allclose(pred[0], approx, rtol=1e-12, atol=1e-12):
                raise RuntimeError(f"{loss} {n}: predictions differ from the training approximant")
            return t[-1] - t[0], [t[i + 1] - t[i] for i in range(5)]

        fit_once(check=True)
        runs = [fit_once() for _ in range(3)]
        order = sorted(range(3), key=lambda i: runs[i][0])
        med = runs[order[1]]
        cells.append({"cell": f"SymmetricTree|{loss}|unw|noctr|{n // 1000}k", "rows": n, "features": 50,
                      "fit_s": round(med[0], 4), "fit_s_all": [round(r[0], 4) for r in runs],
                      "stages_s": dict(zip(("columns", "borders", "open", "trees", "predict"),
                                           (round(v, 4) for v in med[1]))),
                      "reference_catboost_rs_p100_s": ref_s, "official_catboost_gpu_p100_s": off_s,
                      "speedup_vs_reference_p100": round(ref_s / med[0], 2)})
        log(f"published cell {cells[-1]['cell']}: {med[0]:.3f} s per fit "
            f"(reference on a P100: {ref_s} s; stages {cells[-1]['stages_s']})")
    return cells


if __name__ == "__main__":
    main()
