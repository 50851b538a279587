"""Seeded synthetic workloads of the benchmark configs 1-5 (no dataset downloads).

Each generator returns feature-major u8 bins ``bins_fm[F][n]``, the border count per
feature, the target and the training parameters of the config.  Borders are per-feature
quantiles of a fixed-seed 200k-row sample (the reference subsamples 200k rows for border
selection too, crates/cb-data/src/borders.rs:504); duplicate quantiles are dropped, so a
feature with heavy ties gets fewer borders.  A value's bin is the number of borders
strictly below it (crates/cb-compute/src/histogram.rs:563 ``bin_of``).  Columns are
generated from independent per-column streams, so the result does not depend on the
thread count.
"""
from __future__ import annotations

import concurrent.futures as cf
import os

import numpy as np

SAMPLE_ROWS = 200_000


def _borders(col: np.ndarray, n_borders: int, seed: int) -> np.ndarray:
    n = col.shape[0]
    if n > SAMPLE_ROWS:
        sel = np.random.default_rng(seed).choice(n, SAMPLE_ROWS, replace=False)
        sample = col[sel]
    else:
        sample = col
    qs = np.linspace(0.0, 1.0, n_borders + 2)[1:-1]
    b = np.quantile(sample.astype(np.float64), qs).astype(np.float32)
    b = np.unique(b)
    # a border at or above the column maximum separates nothing
    b = b[b < sample.max()] if b.size else b
    return b.astype(np.float64)


def _quantize(col: np.ndarray, borders: np.ndarray) -> np.ndarray:
    # count of borders strictly below the value == searchsorted(..., side="left"); borders
    # are f32 values, so comparing f32 columns against f32 borders is exact
    if col.dtype == np.float32:
        return np.searchsorted(borders.astype(np.float32), col, side="left").astype(np.uint8)
    return np.searchsorted(borders, col.astype(np.float64), side="left").astype(np.uint8)


def _columns(n, F, make_col, n_borders, seed, threads=None, keep_cols=None):
    """Quantize F generated columns; only the columns listed in keep_cols stay in memory."""
    keep_cols = set(range(F)) if keep_cols is None else set(keep_cols)
    bins = np.empty((F, n), np.uint8)
    nb = np.empty(F, np.uint32)
    keep = {}
    borders = [None] * F

    def work(f):
        col = make_col(f)
        b = _borders(col, n_borders, seed * 7919 + f)
        bins[f] = _quantize(col, b)
        nb[f] = b.size
        borders[f] = b
        return f, (col if f in keep_cols else None)

    threads = threads or min(16, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(threads) as ex:
        for f, col in ex.map(work, range(F)):
            if col is not None:
                keep[f] = col
    keep["borders"] = borders
    return bins, nb, keep


def config1(scale=1.0, seed=0):
    """RMSE regression: n x 50 N(0,1), y = X.w + 0.1 N(0,1), w ~ U(-1,1); 128 borders;
    depth 6, 100 iterations, lr 0.1, no bootstrap."""
    n, F = int(100_000 * scale), 50
    g = np.random.default_rng(seed)
    X = g.standard_normal((n, F)).astype(np.float32)
    w = g.uniform(-1, 1, F)
    y = X.astype(np.float64) @ w + 0.1 * g.standard_normal(n)
    bins, nb, kept = _columns(n, F, lambda f: np.ascontiguousarray(X[:, f]), 128, seed, keep_cols=())
    return dict(name="config1", bins=bins, n_borders=nb, target=y, features=X, borders=kept["borders"],
                params=dict(loss="RMSE", depth=6, iterations=100, learning_rate=0.1,
                            l2_leaf_reg=3.0, score="Cosine", leaf_method="Gradient",
                            bootstrap_type="No", boost_from_average=True))


def config2_floats(n_rows=10_000_000, n_features=200, seed=1, threads=None):
    """The float columns of config 2 before quantization, feature-major f32 [F][n]: half
    N(0,1), half lognormal(0,1) (the same generator streams as config2)."""
    n, F, half = int(n_rows), n_features, n_features // 2
    X = np.empty((F, n), np.float32)

    def work(f):
        g = np.random.default_rng([seed, f])
        X[f] = g.standard_normal(n, dtype=np.float32)
        if f >= half:
            np.exp(X[f], out=X[f])

    with cf.ThreadPoolExecutor(threads or min(16, os.cpu_count() or 4)) as ex:
        list(ex.map(work, range(F)))
    return X


def config2_raw(n_rows=10_000_000, n_features=200, seed=1, threads=None):
    """Config 2 before quantization: the f32 columns of ``config2_floats`` and config 2's
    labels (the same streams: Bernoulli(sigmoid(X[:, :20].w))), for a caller that selects
    the borders itself (GreedyLogSum, 254) and quantizes on the device."""
    X = config2_floats(n_rows, n_features, seed, threads)
    n = X.shape[1]
    g = np.random.default_rng([seed, 10_000])
    w = g.uniform(-1, 1, 20)
    logit = np.zeros(n)
    for f in range(min(20, n_features)):
        logit += X[f].astype(np.float64) * w[f]
    p = 1.0 / (1.0 + np.exp(-logit))
    y = (g.random(n) < p).astype(np.float64)
    return dict(name="config2", floats=X, target=y,
                params=dict(loss="Logloss", depth=6, iterations=200, learning_rate=0.03, l2_leaf_reg=3.0,
                            score="Cosine", leaf_method="Gradient", bootstrap_type="Bayesian",
                            bagging_temperature=1.0, boost_from_average=False, random_seed=0,
                            border_count=254, border_type="GreedyLogSum"))


def quantize_columns(X, borders, threads=None):
    """Host bins [F][n] u8 of f32 columns: bin_of, the count of borders strictly below each
    value (NaN-free columns)."""
    F, n = X.shape
    bins = np.empty((F, n), np.uint8)

    def work(f):
        bins[f] = _quantize(X[f], np.asarray(borders[f], np.float64))

    with cf.ThreadPoolExecutor(threads or min(16, os.cpu_count() or 4)) as ex:
        list(ex.map(work, range(F)))
    return bins


def config2(scale=1.0, seed=1, n_rows=None, n_features=200):
    """Logloss: n x 200 (half N(0,1), half lognormal(0,1)); 254 borders; labels
    Bernoulli(sigmoid(X[:, :20].w)); depth 6, 200 iterations, Bayesian bootstrap T=1."""
    n = int(n_rows if n_rows is not None else 10_000_000 * scale)
    F = n_features
    half = F // 2

    def make_col(f):
        g = np.random.default_rng([seed, f])
        c = g.standard_normal(n, dtype=np.float32)
        if f >= half:
            np.exp(c, out=c)
        return c

    bins, nb, cols = _columns(n, F, make_col, 254, seed, keep_cols=range(20))
    g = np.random.default_rng([seed, 10_000])
    w = g.uniform(-1, 1, 20)
    logit = np.zeros(n)
    for f in range(min(20, F)):
        logit += cols[f].astype(np.float64) * w[f]
    p = 1.0 / (1.0 + np.exp(-logit))
    y = (g.random(n) < p).astype(np.float64)
    del cols
    return dict(name="config2", bins=bins, n_borders=nb, target=y,
                params=dict(loss="Logloss", depth=6, iterations=200, learning_rate=0.03,
                            l2_leaf_reg=3.0, score="Cosine", leaf_method="Gradient",
                            bootstrap_type="Bayesian", bagging_temperature=1.0,
                            boost_from_average=False, random_seed=0))


def config3(scale=1.0, seed=3, n_rows=None, n_features=100, group_size=20, pairs_per_group=10,
            loss="PairLogit"):
    """Pairwise ranking: n docs in query groups of 20, n x 100 N(0,1); 254 borders; relevance
    0..4 from a quantized noisy linear score of the first 10 features; about 10 random
    winner > loser pairs per group (pairs whose relevance differs); depth 6, 100 iterations."""
    n = int(n_rows if n_rows is not None else 1_000_000 * scale) // group_size * group_size
    F = n_features

    def make_col(f):
        return np.random.default_rng([seed, f]).standard_normal(n, dtype=np.float32)

    bins, nb, cols = _columns(n, F, make_col, 254, seed, keep_cols=range(min(10, F)))
    g = np.random.default_rng([seed, 77_777])
    w = g.uniform(-1, 1, min(10, F))
    score = np.zeros(n)
    for f in range(min(10, F)):
        score += cols[f].astype(np.float64) * w[f]
    score += 0.5 * g.standard_normal(n)
    rel = np.digitize(score, np.quantile(score, [0.2, 0.4, 0.6, 0.8])).astype(np.float64)
    del cols
    G = n // group_size
    # candidate pairs: 4x the target count per group, keep those with rel_i > rel_j (or the
    # swapped pair when rel_j > rel_i), first pairs_per_group of them
    c = 4 * pairs_per_group
    i = g.integers(0, group_size, size=(G, c))
    j = g.integers(0, group_size, size=(G, c))
    base = (np.arange(G) * group_size)[:, None]
    ri, rj = rel[base + i], rel[base + j]
    win = np.where(ri > rj, i, j)
    los = np.where(ri > rj, j, i)
    ok = ri != rj
    rank = np.cumsum(ok, axis=1)
    keep = ok & (rank <= pairs_per_group)
    winner = (base + win)[keep].astype(np.uint32)
    loser = (base + los)[keep].astype(np.uint32)
    group_offsets = np.arange(0, n + 1, group_size, dtype=np.uint32)
    return dict(name="config3", bins=bins, n_borders=nb, target=rel, pairs=(winner, loser),
                group_offsets=group_offsets,
                params=dict(loss=loss, depth=6, iterations=100, learning_rate=0.03,
                            l2_leaf_reg=3.0, score="Cosine",
                            leaf_method="Newton" if loss == "PairLogit" else "Gradient",
                            bootstrap_type="No", boost_from_average=False))


def config4(n_rows=2_000_000, n_float=30, n_cat=20, seed=4):
    """RMSE with categorical columns: n x 30 N(0,1) floats (254 borders) and 20 categorical
    columns, cardinality log-uniform in [2, 10000], values Zipf(1.1)-distributed over the
    categories; y = X.w + per-category effects + 0.1 N(0,1); depth 6, 200 iterations,
    Bernoulli 0.66.  Returns the float bins, every categorical column as first-seen keys
    (category codes; the caller turns them into bins on the device), the CTR target class
    (y > 0.5, the reference's binclf binarization) and the parameters.  The CTR columns
    themselves depend on the learn permutation and are built by the caller.  CTR candidates
    are single-feature projections only, i.e. max_ctr_complexity=1: the reference's default
    of 4 (crates/cb-train/src/boosting.rs:1010-1017) also scores feature-combination CTRs,
    which this build does not construct."""
    n = int(n_rows)
    g = np.random.default_rng(seed)
    X = g.standard_normal((n, n_float)).astype(np.float32)
    w = g.uniform(-1, 1, n_float)
    y = X.astype(np.float64) @ w
    bins, nb, _ = _columns(n, n_float, lambda f: np.ascontiguousarray(X[:, f]), 254, seed, keep_cols=())
    del X
    card = np.round(np.exp(g.uniform(np.log(2), np.log(10_000), n_cat))).astype(np.int64)
    cats = np.empty((n_cat, n), np.uint32)
    for j in range(n_cat):
        p = 1.0 / np.arange(1, card[j] + 1) ** 1.1
        cdf = np.cumsum(p / p.sum())
        cats[j] = np.minimum(np.searchsorted(cdf, g.random(n)), card[j] - 1)
        y += g.normal(0, 0.5, card[j])[cats[j]]
    y += 0.1 * g.standard_normal(n)
    return dict(name="config4", bins=bins, n_borders=nb, target=y, cat_keys=cats, cardinality=card,
                target_class=(y > 0.5).astype(np.uint8),
                params=dict(loss="RMSE", depth=6, iterations=200, learning_rate=0.1, l2_leaf_reg=3.0,
                            score="Cosine", leaf_method="Gradient", bootstrap_type="Bernoulli",
                            subsample=0.66, boost_from_average=True, random_seed=0,
                            ctr=("Borders", 0.5), ctr_border_count=15))


def config5(scale=1.0, seed=5, n_rows=None, n_features=4096, n_classes=10, zero_frac=0.7):
    """MultiClass K=10: n x 4096 sparse-ish (70% exact zeros, else N(0,1)); 64 borders;
    depth 8, 50 iterations, Newton leaves, no bootstrap.  Labels: argmax of 10 noisy
    linear scores of the first 32 features.  (zero_frac: the share of exact zeros, for tests.)"""
    n = int(n_rows if n_rows is not None else 1_000_000 * scale)
    F = n_features

    def make_col(f):
        g = np.random.default_rng([seed, f])
        c = g.standard_normal(n, dtype=np.float32)
        c[g.random(n) < zero_frac] = 0.0
        return c

    bins, nb, cols = _columns(n, F, make_col, 64, seed, keep_cols=range(32))
    g = np.random.default_rng([seed, 99_999])
    Wc = g.standard_normal((min(32, F), n_classes))
    s = np.zeros((n, n_classes))
    for f in range(min(32, F)):
        s += np.outer(cols[f].astype(np.float64), Wc[f])
    s += g.standard_normal((n, n_classes))
    y = np.argmax(s, axis=1).astype(np.float64)
    del cols
    return dict(name="config5", bins=bins, n_borders=nb, target=y,
                params=dict(loss="MultiClass", depth=8, iterations=50, learning_rate=0.1,
                            l2_leaf_reg=3.0, score="Cosine", leaf_method="Newton",
                            bootstrap_type="No", approx_dim=n_classes, boost_from_average=False))


def random_case(seed, n, F, max_borders=16, K=1, zero_weight_frac=0.0):
    """Small randomized case for parity tests: varying border counts per feature."""
    g = np.random.default_rng(seed)
    nb = g.integers(1, max_borders + 1, size=F).astype(np.uint32)
    nb[g.random(F) < 0.1] = 0  # border-less features are listed but never scored
    bins = np.stack([g.integers(0, int(nb[f]) + 1, size=n) for f in range(F)]).astype(np.uint8)
    if K == 1:
        y = g.standard_normal(n)
    else:
        y = g.integers(0, K, size=n).astype(np.float64)
    w = g.uniform(0.5, 2.0, size=n)
    if zero_weight_frac:
        w[g.random(n) < zero_weight_frac] = 0.0
    return bins, nb, y, w


def reference_speed_cell(n_rows, n_features=50, classification=False, seed=42):
    """A cell of the reference's published GPU speed grid (bench/full_param_gpu_speed/
    bench.py:51-62,460-470 over bench/generator.py:106-138): row-major f32 X (n_rows,
    n_features) of standard normals, the regression target X @ w + 0.1 N(0, 1), or for
    classification {0, 1} drawn through a logistic link of X @ w' (w, w' standard normal).
    The recipe is the reference's; the values come from numpy's seeded Generator, not its
    RandomState stream (a speed workload, not a fixture)."""
    g = np.random.default_rng(seed)
    X = g.standard_normal((n_rows, n_features), dtype=np.float32)
    if classification:
        w = g.standard_normal(n_features)
        p = 1.0 / (1.0 + np.exp(-(X.astype(np.float64) @ w)))
        y = (g.random(n_rows) < p).astype(np.float64)
    else:
        w = g.standard_normal(n_features).astype(np.float32)
        y = (X @ w + 0.1 * g.standard_normal(n_rows, dtype=np.float32)).astype(np.float64)
    return X, y
