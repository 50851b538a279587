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


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    rng_kat(ref)
    fast_logf(ref)
    depth6(ref)
    for s in UPSTREAM:
        upstream(ref, s)


if __name__ == "__main__":
    main()
