"""Extract the reference's own golden vectors into small committed fixtures.

Run in the build container (where the reference checkout is mounted):

    python tests/golden/make_golden.py /root/reference

Everything written here is DATA taken from the reference's test fixtures (inputs and
expected outputs); no reference source is copied.  Sources:

* ``rng_kat.json``        -- known answers quoted in crates/cb-core/src/rng_test.rs:15-32
                             (fast_ut.cpp Test3 / Test2).
* ``fast_logf.txt``       -- the ``fast_logf`` rows of
                             crates/cb-train/tests/fixtures/fast_approx_ref.txt.
* ``depth6.npz/.json``    -- bench/fixtures/cindex_small.npy + expected_depth6_tree.json
                             + expected_depth1_tree.json.
* ``upstream_*.npz``      -- catboost 1.2.10 fits under crates/cb-oracle/fixtures/
                             (inputs, used borders, per-tree splits and leaf values, staged
                             approx, predictions).
* ``upstream_ranking.npz`` -- catboost 1.2.10 PairLogit / PairLogitPairwise fits over the
                             12-document ranking corpus (inputs, pairs, used borders, splits,
                             leaf values, staged approx, predictions).
* ``upstream_one_hot_*``  -- catboost 1.2.10 one-hot fits (one_hot_train/*): float inputs,
                             categorical columns as first-seen bins, used borders, splits
                             (one-hot values as bins), leaf values, predictions.
* ``borders.npz/.json``   -- catboost 1.2.10 standalone quantization borders
                             (Pool.quantize().save_quantization_borders()) of the greedy
                             border types: border_types/<dataset>.bc<k>.Greedy* and
                             borders_quant/numeric_{tiny,nan} (border_count 254), with the
                             input matrices they were computed from.
* ``categorical.npz``     -- catboost 1.2.10 learn permutations and per-object online CTR
                             anchors (good / total counts, values) of plain_ctr,
                             ordered_ctr, tensor_ctr and one_hot_cat, and the cat_hash
                             category hashes with their first-seen bins.
* ``upstream_ctr_fits.npz`` -- catboost 1.2.10 CTR fits ctr_device_{counter,btmv,mixed,buckets}:
                             float inputs, categorical codes, labels, the full float border
                             set, per-tree splits (float feature / CTR target border index,
                             value-space border) and leaf values.
"""
from __future__ import annotations

import json
import os
import re
import shutil
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

UPSTREAM = ["bootstrap/no", "bootstrap/bayesian", "bootstrap/bernoulli", "regression_skeleton",
            "binclf_skeleton", "multiclass_softmax"]


def rng_kat(ref):
    src = open(os.path.join(ref, "crates/cb-core/src/rng_test.rs")).read()
    seed17 = int(re.search(r"from_seed\(17\);\s*assert_eq!\(rng\.gen_rand\(\),\s*([\d_]+)_u64",
                           src).group(1).replace("_", ""))
    arr = re.search(r"const EXPECTED: \[u64; 20\] = \[(.*?)\];", src, re.S).group(1)
    seq = [int(x) for x in arr.replace("\n", " ").split(",") if x.strip()]
    json.dump({"from_seed_17_first_gen_rand": seed17, "new_0_1_2_3_uniform_100": seq},
              open(os.path.join(HERE, "rng_kat.json"), "w"), indent=1)


def fast_logf(ref):
    rows = [l for l in open(os.path.join(ref, "crates/cb-train/tests/fixtures/fast_approx_ref.txt"))
            if l.startswith("fast_logf ")]
    open(os.path.join(HERE, "fast_logf.txt"), "w").writelines(rows)


def depth6(ref):
    fx = os.path.join(ref, "bench/fixtures")
    np.savez_compressed(os.path.join(HERE, "depth6.npz"),
                        cindex=np.load(os.path.join(fx, "cindex_small.npy")).astype(np.uint8))
    shutil.copy(os.path.join(fx, "expected_depth6_tree.json"), os.path.join(HERE, "depth6.json"))
    shutil.copy(os.path.join(fx, "expected_depth1_tree.json"), os.path.join(HERE, "depth1.json"))


def upstream(ref, scen):
    fx = os.path.join(ref, "crates/cb-oracle/fixtures")
    cfg = json.load(open(os.path.join(fx, scen, "config.json")))
    model = json.load(open(os.path.join(fx, scen, "model.json")))
    ds = cfg["input_dataset"]
    X = np.load(os.path.join(fx, "inputs", ds, "X.npy"))
    y = np.load(os.path.join(fx, "inputs", ds, "y.npy"))
    feats = model["features_info"]["float_features"]
    borders = [np.asarray(f["borders"], np.float64) for f in feats]
    nb = np.array([len(b) for b in borders], np.int64)
    flat_b = np.concatenate(borders) if len(borders) else np.zeros(0)
    trees = model["oblivious_trees"]
    depth = len(trees[0]["splits"])
    split_f = np.array([[s["float_feature_index"] for s in t["splits"]] for t in trees], np.int64)
    split_b = np.array([[s["border"] for s in t["splits"]] for t in trees], np.float64)
    leaves = np.array([t["leaf_values"] for t in trees], np.float64)
    staged = np.load(os.path.join(fx, scen, "staged.npy"))
    preds = np.load(os.path.join(fx, scen, "predictions.npy"))
    name = "upstream_" + scen.replace("/", "_")
    np.savez_compressed(os.path.join(HERE, name + ".npz"), X=X, y=y, borders=flat_b, n_borders=nb,
                        split_feature=split_f, split_border=split_b, leaf_values=leaves,
                        staged=staged, predictions=preds,
                        bias=np.array(model["scale_and_bias"][1], np.float64))
    meta = {"scenario": scen, "loss_function": cfg.get("loss_function"), "params": cfg["params"],
            "label_definition": cfg.get("label_definition"), "target_rule": cfg.get("target_rule"),
            "depth": depth,
            "catboost_version": cfg.get("catboost_version")}
    json.dump(meta, open(os.path.join(HERE, name + ".json"), "w"), indent=1)


def _first_seen_bins(col):
    """Dense bins in first-seen order (the PerfectHash remap, cb-data/src/cat_hash.rs:380-471)."""
    index, bins = {}, np.empty(len(col), np.uint8)
    for i, v in enumerate(col):
        bins[i] = index.setdefault(v, len(index))
    return bins, list(index)


def one_hot_train(ref, scen):
    """catboost 1.2.10 one-hot fits (one_hot_train/{default_binary,multi}).  The model stores a
    one-hot split as the CityHash of the category label; which label that is follows from the
    model itself: the label assignment under which applying the model reproduces the
    fixture's predictions.  Splits are written as first-seen bins of that label."""
    import itertools

    fx = os.path.join(ref, "crates/cb-oracle/fixtures/one_hot_train", scen)
    cfg = json.load(open(os.path.join(fx, "config.json")))
    model = json.load(open(os.path.join(fx, "model.json")))
    X = np.load(os.path.join(fx, "X_float.npy"))
    y = np.load(os.path.join(fx, "y.npy"))
    preds = np.load(os.path.join(fx, "predictions.npy"))
    cols = json.load(open(os.path.join(fx, "cat_cols.json")))["columns"]
    cat = [_first_seen_bins(c) for c in cols]
    cat_bins = np.stack([b for b, _ in cat])
    labels = [l for _, l in cat]
    borders = [np.asarray(f["borders"], np.float64) for f in model["features_info"]["float_features"]]
    trees = model["oblivious_trees"]
    hashes = {}  # cat feature -> sorted used hash values
    for t in trees:
        for sp in t["splits"]:
            if sp["split_type"] == "OneHotFeature":
                hashes.setdefault(sp["cat_feature_index"], set()).add(sp["value"])
    feats = sorted(hashes)
    choices = [list(itertools.permutations(range(len(labels[c])), len(hashes[c]))) for c in feats]

    def apply(assign):
        out = np.zeros(X.shape[0])
        for t in trees:
            idx = np.zeros(X.shape[0], np.int64)
            for lvl, sp in enumerate(t["splits"]):
                if sp["split_type"] == "FloatFeature":
                    bit = X[:, sp["float_feature_index"]].astype(np.float32) > sp["border"]
                else:
                    c = sp["cat_feature_index"]
                    bit = cat_bins[c] == assign[c][sp["value"]]
                idx |= bit.astype(np.int64) << lvl
            out += np.asarray(t["leaf_values"])[idx]
        return out

    found = None
    for combo in itertools.product(*choices):
        assign = {c: dict(zip(sorted(hashes[c]), perm)) for c, perm in zip(feats, combo)}
        if np.max(np.abs(apply(assign) - preds)) < 1e-9:
            assert found is None, "label assignment is ambiguous"
            found = assign
    assert found is not None, "no label assignment reproduces the predictions"
    depth = len(trees[0]["splits"])
    kind = np.array([[sp["split_type"] == "OneHotFeature" for sp in t["splits"]] for t in trees])
    feat = np.array([[sp.get("float_feature_index", sp.get("cat_feature_index")) for sp in t["splits"]]
                     for t in trees], np.int64)
    border = np.array([[sp.get("border", np.nan) for sp in t["splits"]] for t in trees], np.float64)
    value_bin = np.array([[found[sp["cat_feature_index"]][sp["value"]] if sp["split_type"] == "OneHotFeature"
                           else -1 for sp in t["splits"]] for t in trees], np.int64)
    name = "upstream_one_hot_" + scen
    np.savez_compressed(os.path.join(HERE, name + ".npz"), X=X, y=y, cat_bins=cat_bins,
                        borders=np.concatenate(borders) if borders else np.zeros(0),
                        n_borders=np.array([len(b) for b in borders], np.int64),
                        split_one_hot=kind, split_feature=feat, split_border=border,
                        split_value_bin=value_bin,
                        leaf_values=np.array([t["leaf_values"] for t in trees], np.float64),
                        predictions=preds)
    meta = {"scenario": "one_hot_train/" + scen, "params": cfg["params"], "depth": depth,
            "cat_labels_first_seen": labels, "catboost_version": cfg.get("catboost_version")}
    json.dump(meta, open(os.path.join(HERE, name + ".json"), "w"), indent=1)


def ranking(ref):
    """catboost 1.2.10 PairLogit / PairLogitPairwise fits over the 12-document ranking
    corpus (ranking_corpus/inputs + per-loss model.json, staged.npy, predictions.npy)."""
    fx = os.path.join(ref, "crates/cb-oracle/fixtures/ranking_corpus")
    arrays = {k: np.load(os.path.join(fx, "inputs", k + ".npy"))
              for k in ("X", "y", "group_id", "pairs")}
    for loss in ("PairLogit", "PairLogitPairwise"):
        model = json.load(open(os.path.join(fx, loss, "model.json")))
        cfg = json.load(open(os.path.join(fx, loss, "config.json")))
        feats = model["features_info"]["float_features"]
        borders = [np.asarray(f["borders"], np.float64) for f in feats]
        trees = model["oblivious_trees"]
        arrays[loss + "_borders"] = np.concatenate(borders)
        arrays[loss + "_n_borders"] = np.array([len(b) for b in borders], np.int64)
        arrays[loss + "_split_feature"] = np.array(
            [[sp["float_feature_index"] for sp in t["splits"]] for t in trees], np.int64)
        arrays[loss + "_split_border"] = np.array([[sp["border"] for sp in t["splits"]] for t in trees])
        arrays[loss + "_leaf_values"] = np.array([t["leaf_values"] for t in trees])
        arrays[loss + "_staged"] = np.load(os.path.join(fx, loss, "staged.npy"))
        arrays[loss + "_predictions"] = np.load(os.path.join(fx, loss, "predictions.npy"))
        arrays[loss + "_config"] = np.frombuffer(json.dumps(cfg).encode(), np.uint8)
    np.savez_compressed(os.path.join(HERE, "upstream_ranking.npz"), **arrays)


def borders(ref):
    """Greedy border cells of border_types/ and borders_quant/ plus their input matrices."""
    fx = os.path.join(ref, "crates/cb-oracle/fixtures")
    inputs = {"borders_dense": "inputs/borders_dense", "borders_runs": "inputs/borders_runs",
              "numeric_nan": "inputs/numeric_nan", "numeric_tiny": "inputs/numeric_tiny",
              "float_only_byte_identity": "float_only_byte_identity/inputs"}
    arrays = {"X_" + d: np.load(os.path.join(fx, rel, "X.npy")) for d, rel in inputs.items()}
    cells = []
    cfg = json.load(open(os.path.join(fx, "border_types", "config.json")))
    for stem, sc in sorted(cfg["scenarios"].items()):
        if sc["feature_border_type"] not in ("GreedyLogSum", "GreedyMinEntropy"):
            continue
        b = np.load(os.path.join(fx, "border_types", stem + ".borders.npy"))
        per = np.load(os.path.join(fx, "border_types", stem + ".borders_per_feature.npy"))
        arrays[stem + ".borders"] = b
        arrays[stem + ".per_feature"] = per.astype(np.int64)
        cells.append({"stem": stem, "dataset": sc["dataset"], "border_count": sc["border_count"],
                      "border_type": sc["feature_border_type"], "nan_mode": sc["nan_mode"]})
    qcfg = json.load(open(os.path.join(fx, "borders_quant", "config.json")))
    for d, sc in sorted(qcfg["scenarios"].items()):
        stem = "borders_quant." + d
        arrays[stem + ".borders"] = np.load(os.path.join(fx, "borders_quant", d + ".borders.npy"))
        arrays[stem + ".per_feature"] = np.load(
            os.path.join(fx, "borders_quant", d + ".borders_per_feature.npy")).astype(np.int64)
        cells.append({"stem": stem, "dataset": sc["input_dataset"], "border_count": sc["border_count"],
                      "border_type": sc["border_selection_type"], "nan_mode": sc["nan_mode"]})
    np.savez_compressed(os.path.join(HERE, "borders.npz"), **arrays)
    json.dump({"catboost_version": cfg.get("catboost_version"), "cells": cells},
              open(os.path.join(HERE, "borders.json"), "w"), indent=1)


def categorical(ref):
    """Permutations, online CTR anchors and first-seen bins (data only)."""
    fx = os.path.join(ref, "crates/cb-oracle/fixtures")
    arrays = {}
    for scen in ("plain_ctr", "ordered_ctr", "tensor_ctr", "one_hot_cat"):
        for f in sorted(os.listdir(os.path.join(fx, scen))):
            if f.startswith(("permutation_fold", "ctr_good_count", "ctr_total_count", "ctr_value")):
                arrays[scen + "." + f[:-4]] = np.load(os.path.join(fx, scen, f))
        cfg = json.load(open(os.path.join(fx, scen, "config.json")))
        arrays[scen + ".seed"] = np.array(cfg["seed"], np.int64)
        arrays[scen + ".prior"] = np.array(float(cfg["params"]["simple_ctr"][0].split("=")[1]))
    arrays["cat_hash.hashes"] = np.load(os.path.join(fx, "cat_hash", "cat_hashes.npy")).astype(np.uint32)
    arrays["cat_hash.bins"] = np.load(os.path.join(fx, "cat_hash", "perfect_hash_bins.npy")).astype(np.uint32)
    np.savez_compressed(os.path.join(HERE, "categorical.npz"), **arrays)


def ctr_fits(ref):
    """Small CTR fits of catboost 1.2.10 (data only)."""
    fx = os.path.join(ref, "crates/cb-oracle/fixtures")
    arrays = {}
    for name in ("counter", "btmv", "mixed", "buckets"):
        d = os.path.join(fx, "ctr_device_" + name)
        m = json.load(open(os.path.join(d, "model.json")))
        cfg = json.load(open(os.path.join(d, "config.json")))
        for k in ("X", "X_cat", "y", "borders"):
            arrays[name + "." + k] = np.load(os.path.join(d, k + ".npy"))
        kind, idx, border = [], [], []
        for t in m["oblivious_trees"]:
            for sp in t["splits"]:
                ctr = sp["split_type"] != "FloatFeature"
                kind.append(int(ctr))
                idx.append(sp.get("ctr_target_border_idx", 0) if ctr else sp["float_feature_index"])
                border.append(sp["border"])
        arrays[name + ".split_is_ctr"] = np.array(kind, np.int64)
        arrays[name + ".split_index"] = np.array(idx, np.int64)
        arrays[name + ".split_border"] = np.array(border)
        arrays[name + ".leaf_values"] = np.array([t["leaf_values"] for t in m["oblivious_trees"]])
        arrays[name + ".params"] = np.frombuffer(json.dumps(cfg["params"]).encode(), np.uint8)
    np.savez_compressed(os.path.join(HERE, "upstream_ctr_fits.npz"), **arrays)


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    rng_kat(ref)
    fast_logf(ref)
    depth6(ref)
    for s in UPSTREAM:
        upstream(ref, s)
    for s in ("default_binary", "multi"):
        one_hot_train(ref, s)
    ranking(ref)
    borders(ref)
    categorical(ref)
    ctr_fits(ref)


if __name__ == "__main__":
    main()
