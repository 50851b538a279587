"""Loaders for the committed golden fixtures in tests/golden (data extracted from the
reference's own test fixtures by tests/golden/make_golden.py)."""
from __future__ import annotations

import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def upstream(name: str):
    """One catboost 1.2.10 fit: inputs, used borders, expected trees and approximants."""
    z = np.load(os.path.join(GOLDEN, f"upstream_{name}.npz"))
    meta = json.load(open(os.path.join(GOLDEN, f"upstream_{name}.json")))
    X, y = z["X"], z["y"].astype(np.float64)
    nb = z["n_borders"]
    offs = np.concatenate([[0], np.cumsum(nb)])
    borders = [z["borders"][offs[i]:offs[i + 1]] for i in range(len(nb))]
    if meta.get("label_definition"):  # "y_binary = (numeric_tiny.y > median(numeric_tiny.y))"
        y = (y > np.median(y)).astype(np.float64)
    if meta.get("target_rule"):  # "digitize(y, quantile(y,[1/3,2/3])) -> {0,1,2}"
        y = np.digitize(y, np.quantile(y, [1 / 3, 2 / 3])).astype(np.float64)
    return dict(X=X, y=y, borders=borders, n_borders=nb.astype(np.uint32),
                split_feature=z["split_feature"], split_border=z["split_border"],
                leaf_values=z["leaf_values"], staged=z["staged"], predictions=z["predictions"],
                bias=z["bias"], meta=meta, params=meta["params"])


def depth6():
    cindex = np.load(os.path.join(GOLDEN, "depth6.npz"))["cindex"]
    tree = json.load(open(os.path.join(GOLDEN, "depth6.json")))
    return cindex, tree


def rng_kat():
    return json.load(open(os.path.join(GOLDEN, "rng_kat.json")))


def fast_logf_rows():
    rows = []
    for line in open(os.path.join(GOLDEN, "fast_logf.txt")):
        _, a, b = line.split()
        rows.append((int(a, 16), int(b, 16)))
    return rows


def upstream_one_hot(name: str):
    """One catboost 1.2.10 one-hot fit: float columns (to be quantized with the model's used
    borders) and categorical first-seen bins, laid out float | one-hot as on the reference's
    device feature axis."""
    z = np.load(os.path.join(GOLDEN, f"upstream_one_hot_{name}.npz"))
    meta = json.load(open(os.path.join(GOLDEN, f"upstream_one_hot_{name}.json")))
    nb = z["n_borders"]
    offs = np.concatenate([[0], np.cumsum(nb)])
    borders = [z["borders"][offs[i]:offs[i + 1]] for i in range(len(nb))]
    cat = z["cat_bins"]
    card = [int(c.max()) + 1 for c in cat]
    n_float = z["X"].shape[1]
    return dict(X=z["X"], y=z["y"].astype(np.float64), borders=borders, cat_bins=cat,
                n_float=n_float,
                # oracle convention: n_borders[f] + 1 = bins of f (cardinality for one-hot)
                n_borders=np.array(list(nb) + [c - 1 for c in card], np.uint32),
                one_hot=np.array([0] * n_float + [1] * len(card), np.uint8),
                # device convention (real_folds, boosting.rs:4334-4372)
                real_folds=np.array([len(b) + 1 for b in borders] + card, np.uint32),
                split_one_hot=z["split_one_hot"], split_feature=z["split_feature"],
                split_border=z["split_border"], split_value_bin=z["split_value_bin"],
                leaf_values=z["leaf_values"], predictions=z["predictions"], meta=meta,
                params=meta["params"])


def ranking(loss: str):
    """catboost 1.2.10 fit of ``loss`` (PairLogit / PairLogitPairwise) over the ranking corpus."""
    z = np.load(os.path.join(GOLDEN, "upstream_ranking.npz"))
    nb = z[loss + "_n_borders"]
    offs = np.concatenate([[0], np.cumsum(nb)])
    borders = [z[loss + "_borders"][offs[i]:offs[i + 1]] for i in range(len(nb))]
    cfg = json.loads(bytes(z[loss + "_config"]).decode())
    return dict(X=z["X"], y=z["y"].astype(np.float64), pairs=z["pairs"].astype(np.uint32),
                group_id=z["group_id"], borders=borders, n_borders=nb.astype(np.uint32),
                split_feature=z[loss + "_split_feature"], split_border=z[loss + "_split_border"],
                leaf_values=z[loss + "_leaf_values"], staged=z[loss + "_staged"],
                predictions=z[loss + "_predictions"], config=cfg)


def borders():
    """catboost 1.2.10 standalone greedy border sets: (cells, matrices) where each cell is a
    dict(stem, dataset, border_count, border_type, nan_mode, borders=[per-feature arrays])
    and matrices maps a dataset name to its f64 input matrix [n][F]."""
    z = np.load(os.path.join(GOLDEN, "borders.npz"))
    meta = json.load(open(os.path.join(GOLDEN, "borders.json")))
    mats = {k[2:]: z[k] for k in z.files if k.startswith("X_")}
    cells = []
    for c in meta["cells"]:
        per = z[c["stem"] + ".per_feature"]
        offs = np.concatenate([[0], np.cumsum(per)])
        flat = z[c["stem"] + ".borders"]
        cells.append(dict(c, borders=[flat[offs[i]:offs[i + 1]] for i in range(len(per))]))
    return cells, mats


def categorical():
    """catboost 1.2.10 learn permutations, online CTR anchors and first-seen bins (a dict of
    arrays keyed '<scenario>.<name>')."""
    z = np.load(os.path.join(GOLDEN, "categorical.npz"))
    return {k: z[k] for k in z.files}


CTR_SPECS = {"counter": [("Counter", 0.5, 0)], "btmv": [("BinarizedTargetMeanValue", 0.5, 0)],
             "mixed": [("Borders", 0.5, 0)], "buckets": [("Buckets", 0.5, 0), ("Buckets", 0.5, 1)]}


def ctr_fit(name: str):
    """catboost 1.2.10 CTR fit ``name`` (counter / btmv / mixed / buckets): inputs, params, and
    per-tree expected splits [(is_ctr, float feature or CTR target border index, border)] and
    leaf values."""
    z = np.load(os.path.join(GOLDEN, "upstream_ctr_fits.npz"))
    g = {k.split(".", 1)[1]: z[k] for k in z.files if k.startswith(name + ".")}
    params = json.loads(bytes(g.pop("params")).decode())
    depth = params["depth"]
    splits = list(zip(g["split_is_ctr"].tolist(), g["split_index"].tolist(), g["split_border"].tolist()))
    trees = [splits[i:i + depth] for i in range(0, len(splits), depth)]
    return dict(X=g["X"].astype(np.float32), X_cat=g["X_cat"], y=g["y"].astype(np.float64),
                borders=g["borders"], trees=trees, leaf_values=g["leaf_values"], params=params,
                specs=CTR_SPECS[name])
