"""ctypes front-end of the CPU restatement in ``oracle/cb_oracle.c``.

TEST INFRASTRUCTURE ONLY: the parity checker and the CPU baseline.  Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
import this module; the product package never does.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libcb_oracle.so")
_lib = None

# CrossEntropy (soft targets in [0, 1]) runs the Logloss arm: its ders are the Logloss ders by
# definition (cross_entropy_der1/2, loss.rs:80-97)
LOSS = {"RMSE": 0, "Logloss": 1, "MultiClass": 2, "PairLogit": 3, "PairLogitPairwise": 4, "CrossEntropy": 1}
SCORE = {"Cosine": 0, "L2": 1, "SolarL2": 2, "LOOL2": 3, "SatL2": 4}
BOOT = {"No": 0, "Bayesian": 1, "Bernoulli": 2}
LEAF = {"Gradient": 0, "Newton": 1}


class Rng(C.Structure):
    _fields_ = [("x1", C.c_uint64), ("c1", C.c_uint64), ("x2", C.c_uint64),
                ("c2", C.c_uint64), ("calls", C.c_uint64)]


class Params(C.Structure):
    _fields_ = [("loss", C.c_int32), ("score_function", C.c_int32),
                ("bootstrap_type", C.c_int32), ("leaf_method", C.c_int32),
                ("depth", C.c_int32), ("iterations", C.c_int32),
                ("boost_from_average", C.c_int32), ("n_threads", C.c_int32),
                ("approx_dim", C.c_int32), ("pad_", C.c_int32),
                ("learning_rate", C.c_double), ("l2_leaf_reg", C.c_double),
                ("subsample", C.c_double), ("bagging_temperature", C.c_float),
                ("pad2_", C.c_float), ("random_seed", C.c_uint64),
                ("one_hot_flags", C.c_void_p),
                ("pair_winner", C.c_void_p), ("pair_loser", C.c_void_p), ("pair_weight", C.c_void_p),
                ("n_pairs", C.c_uint64), ("pairwise_non_diag_reg", C.c_double),
                ("n_ctr", C.c_uint32), ("ctr_avg_bins", C.c_void_p), ("ctr_bucket_count", C.c_void_p),
                ("ctr_group", C.c_void_p), ("n_cat", C.c_uint32), ("cat_buckets", C.c_void_p),
                ("model_size_reg", C.c_double)]


ONE_HOT_SPLIT = 0x40000000  # flag bit on the feature entry of an equality split


def build(force: bool = False) -> str:
    """Compile the restatement with its Makefile (gcc, OpenMP)."""
    args = ["make", "-C", _HERE] + (["-B"] if force else [])
    subprocess.run(args, check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        P = C.c_void_p
        L.orc_rng_new.argtypes = [C.POINTER(Rng), C.c_uint64, C.c_uint32, C.c_uint64, C.c_uint32]
        L.orc_rng_from_seed.argtypes = [C.POINTER(Rng), C.c_uint64]
        L.orc_rng_gen.argtypes = [C.POINTER(Rng)]
        L.orc_rng_gen.restype = C.c_uint64
        L.orc_rng_advance.argtypes = [C.POINTER(Rng), C.c_uint64]
        L.orc_rng_real1.argtypes = [C.POINTER(Rng)]
        L.orc_rng_real1.restype = C.c_double
        L.orc_rng_uniform.argtypes = [C.POINTER(Rng), C.c_uint64]
        L.orc_rng_uniform.restype = C.c_uint64
        L.orc_std_normal.argtypes = [C.POINTER(Rng)]
        L.orc_leaf_score_term.argtypes = [C.c_int32, C.c_double, C.c_double]
        L.orc_leaf_score_term.restype = C.c_double
        L.orc_std_normal.restype = C.c_double
        L.orc_fast_logf.argtypes = [C.c_float]
        L.orc_fast_logf.restype = C.c_float
        L.orc_bootstrap.argtypes = [C.c_int32, C.c_uint64, C.c_double, C.c_float, C.POINTER(Rng), P, P]
        L.orc_bootstrap.restype = C.c_int
        L.orc_quantize.argtypes = [P, C.c_uint64, P, C.c_uint32, P]
        L.orc_ders.argtypes = [C.c_int32, P, P, C.c_uint64, P, P]
        L.orc_grow_tree.argtypes = [P, P, C.c_uint64, C.c_uint32, P, P, C.c_int32, C.c_int32,
                                    C.c_int32, C.c_double, C.POINTER(Rng), C.c_int32, P, P, P, P, P]
        L.orc_grow_tree.restype = C.c_int
        L.orc_leaf_sums.argtypes = [P, C.c_uint64, C.c_uint32, P, P, P, P]
        L.orc_train.argtypes = [C.POINTER(Params), P, P, C.c_uint64, C.c_uint32, P, P, P, P, P, P, P]
        L.orc_train.restype = C.c_int
        L.orc_pairs_order.argtypes = [P, C.c_uint64, C.c_uint64, P]
        L.orc_pairlogit_ders.argtypes = [P, C.c_uint64, P, P, P, C.c_uint64, P, P]
        L.orc_pairwise_weights.argtypes = [C.c_uint64, P, P, P, C.c_uint64, P]
        L.orc_grow_tree_pairwise.argtypes = [P, P, C.c_uint64, C.c_uint32, P, P, P, P, C.c_uint64,
                                             C.c_int32, C.c_double, C.c_double, C.c_int32, P, P, P]
        L.orc_grow_tree_pairwise.restype = C.c_int
        L.orc_sample_indices_for_borders.argtypes = [C.c_uint64, C.c_uint64, P]
        L.orc_select_borders_greedy.argtypes = [P, C.c_uint64, C.c_uint32, C.c_int32, C.c_int32, P]
        L.orc_select_borders_greedy.restype = C.c_uint32
        L.orc_shuffled_indices.argtypes = [C.c_uint64, C.c_uint64, P]
        L.orc_permutations.argtypes = [C.c_uint64, C.c_uint32, C.c_uint64, P]
        L.orc_perfect_hash.argtypes = [P, C.c_uint64, P]
        L.orc_perfect_hash.restype = C.c_uint32
        L.orc_ctr_column.argtypes = [C.c_int32, C.c_uint32, C.c_double, C.c_double, C.c_uint32, P,
                                     C.c_uint32, C.c_uint64, P, P, P, P, P, P]
        L.orc_ctr_column.restype = C.c_int
        L.orc_apply_oblivious.argtypes = [P, C.c_uint64, C.c_uint32, P, P, P, P, P, C.c_uint32,
                                          C.c_uint32, P, P, P]
        L.orc_apply_oblivious.restype = C.c_int
        L.orc_pairwise_feature_scores.argtypes = [P, P, P, C.c_uint64, P, P, P, C.c_uint64, C.c_int32,
                                                  C.c_int32, C.c_double, C.c_double, P]
        L.orc_pairwise_leaf_deltas.argtypes = [P, C.c_uint64, P, P, P, P, C.c_uint64, C.c_uint32,
                                               C.c_double, C.c_double, P]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def rng_from_seed(seed: int) -> Rng:
    r = Rng()
    lib().orc_rng_from_seed(C.byref(r), C.c_uint64(seed & (2**64 - 1)))
    return r


def rng_new(seed1, seq1, seed2, seq2) -> Rng:
    r = Rng()
    lib().orc_rng_new(C.byref(r), seed1, seq1, seed2, seq2)
    return r


def fast_logf(v: float) -> float:
    return lib().orc_fast_logf(v)


def bootstrap(kind: str, n: int, subsample: float, temperature: float, rng: Rng):
    sw = np.empty(n, np.float64)
    ctrl = np.empty(n, np.uint8)
    rc = lib().orc_bootstrap(BOOT[kind], n, subsample, temperature, C.byref(rng), _p(sw), _p(ctrl))
    assert rc == 0
    return sw, ctrl.astype(bool)


def quantize(values: np.ndarray, borders: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(values, np.float32)
    b = np.ascontiguousarray(borders, np.float64)
    out = np.empty(v.shape[0], np.uint8)
    lib().orc_quantize(_p(v), v.shape[0], _p(b), b.shape[0], _p(out))
    return out


def ders(loss: str, approx: np.ndarray, target: np.ndarray):
    a = np.ascontiguousarray(approx, np.float64)
    t = np.ascontiguousarray(target, np.float64)
    d1 = np.empty_like(a)
    d2 = np.empty_like(a)
    lib().orc_ders(LOSS[loss], _p(a), _p(t), a.shape[0], _p(d1), _p(d2))
    return d1, d2


def _split_flags(splits):
    """Strip the one-hot flag bit from the feature entries; return (splits, one_hot)."""
    one_hot = (splits[..., 0] & ONE_HOT_SPLIT) != 0
    splits = splits.copy()
    splits[..., 0] &= ~ONE_HOT_SPLIT
    return splits, one_hot


def leaf_score_term(score, s, w):
    """One leaf's additive term of the SolarL2 / LOOL2 / SatL2 calcers (der sum s, weight w)."""
    return lib().orc_leaf_score_term(SCORE[score], float(s), float(w))


def grow_tree(bins_fm, n_borders, score_der, score_w, depth, score="Cosine", scaled_l2=3.0,
              rng: Rng | None = None, want_hists=False, n_threads=0, one_hot=None):
    """One oblivious tree.  ``bins_fm`` is u8 [F, n]; ``score_der`` is [K, n] or [n].
    ``one_hot`` (optional, [F]) flags one-hot columns; for them ``n_borders[f] + 1`` is the
    column's cardinality."""
    bins_fm = np.ascontiguousarray(bins_fm, np.uint8)
    F, n = bins_fm.shape
    nb = np.ascontiguousarray(n_borders, np.uint32)
    sd = np.ascontiguousarray(score_der, np.float64)
    K = 1 if sd.ndim == 1 else sd.shape[0]
    sw = np.ascontiguousarray(score_w, np.float64)
    splits = np.zeros((depth, 2), np.int32)
    scores = np.zeros(depth, np.float64)
    leaf_of = np.zeros(n, np.uint32)
    n_bins = int(nb.max()) + 1 if F else 1
    hists = None
    if want_hists:
        total = sum((1 << l) * F * n_bins * (K + 1) for l in range(depth))
        hists = np.zeros(total, np.float64)
    oh = None if one_hot is None else np.ascontiguousarray(one_hot, np.uint8)
    rc = lib().orc_grow_tree(_p(bins_fm), _p(nb), n, F, _p(sd), _p(sw), K, depth, SCORE[score],
                             scaled_l2, C.byref(rng) if rng is not None else None, n_threads,
                             _p(splits), _p(scores), _p(leaf_of), _p(hists), _p(oh))
    if rc != 0:
        raise RuntimeError(f"orc_grow_tree failed rc={rc}")
    splits, is_oh = _split_flags(splits)
    out = {"splits": splits, "one_hot": is_oh, "scores": scores, "leaf_of": leaf_of, "n_bins": n_bins}
    if want_hists:
        levels = []
        off = 0
        for l in range(depth):
            sz = (1 << l) * F * n_bins * (K + 1)
            levels.append(hists[off:off + sz].reshape(1 << l, F, n_bins, K + 1))
            off += sz
        out["hists"] = levels
    return out


def pairs_in_competitor_order(winner, loser, weight=None, n=None):
    """Pairs stably ordered by winner: the reference's competitor order (group ascending,
    winner ascending, input order per winner)."""
    w = np.ascontiguousarray(winner, np.uint32)
    l = np.ascontiguousarray(loser, np.uint32)
    n = int(max(w.max(), l.max()) + 1) if n is None else n
    perm = np.empty(w.shape[0], np.uint64)
    lib().orc_pairs_order(_p(w), w.shape[0], n, _p(perm))
    perm = perm.astype(np.int64)
    wt = np.ones(w.shape[0]) if weight is None else np.asarray(weight, np.float64)
    return w[perm].copy(), l[perm].copy(), np.ascontiguousarray(wt[perm])


def pairlogit_ders(approx, winner, loser, weight):
    """PairLogit der1/der2 (pairs in competitor order)."""
    a = np.ascontiguousarray(approx, np.float64)
    w, l, wt = (np.ascontiguousarray(x) for x in (winner, loser, weight))
    d1 = np.empty_like(a)
    d2 = np.empty_like(a)
    lib().orc_pairlogit_ders(_p(a), a.shape[0], _p(w), _p(l), _p(wt), w.shape[0], _p(d1), _p(d2))
    return d1, d2


def pairwise_weights(n, winner, loser, weight):
    w, l, wt = (np.ascontiguousarray(x) for x in (winner, loser, weight))
    pw = np.empty(n)
    lib().orc_pairwise_weights(n, _p(w), _p(l), _p(wt), w.shape[0], _p(pw))
    return pw


def grow_tree_pairwise(bins_fm, n_borders, der, winner, loser, weight, depth, l2, prior=0.1,
                       n_threads=0):
    """One PairLogitPairwise tree (pairs in competitor order)."""
    bins_fm = np.ascontiguousarray(bins_fm, np.uint8)
    F, n = bins_fm.shape
    nb = np.ascontiguousarray(n_borders, np.uint32)
    d = np.ascontiguousarray(der, np.float64)
    w, l, wt = (np.ascontiguousarray(x) for x in (winner, loser, weight))
    splits = np.zeros((depth, 2), np.int32)
    scores = np.zeros(depth)
    leaf_of = np.zeros(n, np.uint32)
    rc = lib().orc_grow_tree_pairwise(_p(bins_fm), _p(nb), n, F, _p(d), _p(w), _p(l), _p(wt),
                                      w.shape[0], depth, l2, prior, n_threads, _p(splits),
                                      _p(scores), _p(leaf_of))
    if rc != 0:
        raise RuntimeError(f"orc_grow_tree_pairwise failed rc={rc}")
    return {"splits": splits, "scores": scores, "leaf_of": leaf_of}


def pairwise_feature_scores(col, leaf_of, der, winner, loser, weight, P, B, l2, prior=0.1):
    """Pairwise score of every border (B-1 values) of one feature with P parent leaves."""
    c = np.ascontiguousarray(col, np.uint8)
    lo = np.ascontiguousarray(leaf_of, np.uint32)
    d = np.ascontiguousarray(der, np.float64)
    w, l, wt = (np.ascontiguousarray(x) for x in (winner, loser, weight))
    out = np.zeros(B - 1)
    lib().orc_pairwise_feature_scores(_p(c), _p(lo), _p(d), c.shape[0], _p(w), _p(l), _p(wt),
                                      w.shape[0], P, B, l2, prior, _p(out))
    return out


def pairwise_leaf_deltas(leaf_of, der, winner, loser, weight, n_leaves, l2, prior=0.1):
    lo = np.ascontiguousarray(leaf_of, np.uint32)
    d = np.ascontiguousarray(der, np.float64)
    w, l, wt = (np.ascontiguousarray(x) for x in (winner, loser, weight))
    out = np.zeros(n_leaves)
    lib().orc_pairwise_leaf_deltas(_p(lo), lo.shape[0], _p(d), _p(w), _p(l), _p(wt), w.shape[0],
                                   n_leaves, l2, prior, _p(out))
    return out


PENALTY = {"GreedyLogSum": 0, "GreedyMinEntropy": 1}


def select_borders(column, border_count, nan_sentinel=False, kind="GreedyLogSum"):
    """Greedy border set of one f32 column (NaNs allowed; sampled above 200000 rows)."""
    c = np.ascontiguousarray(column, np.float32)
    out = np.zeros(border_count + 1)
    k = lib().orc_select_borders_greedy(_p(c), c.shape[0], border_count, int(nan_sentinel),
                                        PENALTY[kind], _p(out))
    return out[:k].copy()


def sample_indices_for_borders(n, sample_size=200_000):
    out = np.zeros(min(n, sample_size), np.uint32)
    lib().orc_sample_indices_for_borders(n, sample_size, _p(out))
    return out


CTR = {"Borders": 0, "Buckets": 1, "BinarizedTargetMeanValue": 2, "Counter": 4}


def shuffled_indices(n, seed):
    out = np.zeros(n, np.uint32)
    lib().orc_shuffled_indices(n, seed, _p(out))
    return out


def permutations(n, count, seed):
    out = np.zeros((count, n), np.uint32)
    lib().orc_permutations(n, count, seed, _p(out))
    return out


def perfect_hash(keys):
    """First-seen dense bins of u32 keys and the number of distinct keys."""
    k = np.ascontiguousarray(keys, np.uint32)
    out = np.zeros(k.shape[0], np.uint32)
    d = lib().orc_perfect_hash(_p(k), k.shape[0], _p(out))
    return out, int(d)


def ctr_column(ctr_type, bucket, permutation, target_class, prior=0.5, target_border_idx=0,
               border_count=15, n_buckets=None, prior_denom=1.0):
    """One online CTR column: dict(good, total, value, bin) in object order."""
    b = np.ascontiguousarray(bucket, np.uint32)
    pm = np.ascontiguousarray(permutation, np.uint32)
    tc = np.ascontiguousarray(target_class, np.uint8)
    n = b.shape[0]
    nb = int(b.max()) + 1 if n_buckets is None and n else (n_buckets or 0)
    good, total = np.zeros(n), np.zeros(n, np.int64)
    value, bins = np.zeros(n), np.zeros(n, np.uint8)
    rc = lib().orc_ctr_column(CTR[ctr_type], target_border_idx, prior, prior_denom, border_count,
                              _p(b), nb, n, _p(pm), _p(tc), _p(good), _p(total), _p(value), _p(bins))
    if rc != 0:
        raise ValueError(f"orc_ctr_column rc={rc}")
    return dict(good=good, total=total, value=value, bin=bins)


def model_arrays(split_features, split_borders, leaf_values, K=1):
    """Flat CSR model arrays of an oblivious ensemble: split_features / split_borders are
    per-tree lists, leaf_values per-tree arrays of 2^depth * K (leaf-major)."""
    sf = np.ascontiguousarray(np.concatenate([np.asarray(t, np.uint32) for t in split_features]), np.uint32)
    sb = np.ascontiguousarray(np.concatenate([np.asarray(t, np.float64) for t in split_borders]), np.float64)
    so = np.concatenate([[0], np.cumsum([len(t) for t in split_features])]).astype(np.uint32)
    lv = np.ascontiguousarray(np.concatenate([np.asarray(t, np.float64).ravel() for t in leaf_values]))
    lo = np.concatenate([[0], np.cumsum([np.asarray(t).size // K for t in leaf_values])]).astype(np.uint32)
    return sf, sb, so, lv, lo


def apply_oblivious(x_fm, split_features, split_borders, tree_split_offsets, leaf_values,
                    tree_leaf_offsets, K=1, bias=None, nan_as_true=None):
    """Raw predictions [K][n] of float features x_fm [F][n] (f32)."""
    x = np.ascontiguousarray(x_fm, np.float32)
    F, n = x.shape
    b = None if bias is None else np.ascontiguousarray(np.broadcast_to(bias, (K,)), np.float64)
    na = None if nan_as_true is None else np.ascontiguousarray(nan_as_true, np.uint8)
    out = np.zeros((K, n))
    arrs = [np.ascontiguousarray(a) for a in (split_features, split_borders, tree_split_offsets,
                                               leaf_values, tree_leaf_offsets)]
    lib().orc_apply_oblivious(_p(x), n, F, _p(arrs[0]), _p(arrs[1]), _p(arrs[2]), _p(arrs[3]),
                              _p(arrs[4]), arrs[2].shape[0] - 1, K, _p(b), _p(na), _p(out))
    return out


def leaf_sums(leaf_of, n_leaves, der, weight=None):
    lo = np.ascontiguousarray(leaf_of, np.uint32)
    d = np.ascontiguousarray(der, np.float64)
    w = None if weight is None else np.ascontiguousarray(weight, np.float64)
    sd = np.zeros(n_leaves)
    sw = np.zeros(n_leaves)
    lib().orc_leaf_sums(_p(lo), lo.shape[0], n_leaves, _p(d), _p(w), _p(sd), _p(sw))
    return sd, sw


def train(bins_fm, n_borders, target, *, loss="RMSE", depth=6, iterations=10, learning_rate=0.1,
          l2_leaf_reg=3.0, score="Cosine", bootstrap_type="No", subsample=0.66,
          bagging_temperature=1.0, leaf_method="Gradient", boost_from_average=False,
          random_seed=0, weight=None, approx_dim=1, n_threads=0, staged=False, one_hot=None,
          pairs=None, pairwise_non_diag_reg=0.1, ctr=None):
    """CPU boosting loop.  ``one_hot`` (optional, [F]) flags one-hot columns (for them
    ``n_borders[f] + 1`` is the cardinality); one-hot with bootstrap raises (-4), as the
    reference refuses it.  ``pairs`` = (winner, loser[, weight]) for PairLogit /
    PairLogitPairwise, in any order.  ``ctr`` = dict(avg_bins [n_ctr][n], bucket_count,
    group, cat_buckets [n_cat][n], model_size_reg) for fits whose last n_ctr columns are CTR
    columns under the structure permutation."""
    bins_fm = np.ascontiguousarray(bins_fm, np.uint8)
    F, n = bins_fm.shape
    nb = np.ascontiguousarray(n_borders, np.uint32)
    t = np.ascontiguousarray(target, np.float64)
    w = None if weight is None else np.ascontiguousarray(weight, np.float64)
    K = approx_dim if loss == "MultiClass" else 1
    p = Params(loss=LOSS[loss], score_function=SCORE[score], bootstrap_type=BOOT[bootstrap_type],
               leaf_method=LEAF[leaf_method], depth=depth, iterations=iterations,
               boost_from_average=int(boost_from_average), n_threads=n_threads, approx_dim=K,
               learning_rate=learning_rate, l2_leaf_reg=l2_leaf_reg, subsample=subsample,
               bagging_temperature=bagging_temperature, random_seed=random_seed)
    oh = None if one_hot is None else np.ascontiguousarray(one_hot, np.uint8)
    p.one_hot_flags = None if oh is None else oh.ctypes.data
    keep = []
    if pairs is not None:
        pw_ = np.ascontiguousarray(pairs[0], np.uint32)
        pl_ = np.ascontiguousarray(pairs[1], np.uint32)
        pwt = None if len(pairs) < 3 or pairs[2] is None else np.ascontiguousarray(pairs[2], np.float64)
        keep += [pw_, pl_, pwt]
        p.pair_winner, p.pair_loser = pw_.ctypes.data, pl_.ctypes.data
        p.pair_weight = None if pwt is None else pwt.ctypes.data
        p.n_pairs = pw_.shape[0]
    p.pairwise_non_diag_reg = pairwise_non_diag_reg
    if ctr is not None:
        # the last ctr["avg_bins"].shape[0] features are CTR columns (structure permutation)
        avg = np.ascontiguousarray(ctr["avg_bins"], np.uint8)
        bc = np.ascontiguousarray(ctr["bucket_count"], np.uint32)
        grp = np.ascontiguousarray(ctr.get("group", np.arange(avg.shape[0])), np.uint32)
        cat = np.ascontiguousarray(ctr.get("cat_buckets", np.zeros((0, n))), np.uint32)
        keep += [avg, bc, grp, cat]
        p.n_ctr, p.ctr_avg_bins, p.ctr_bucket_count = avg.shape[0], avg.ctypes.data, bc.ctypes.data
        p.ctr_group, p.n_cat, p.cat_buckets = grp.ctypes.data, cat.shape[0], cat.ctypes.data
        p.model_size_reg = ctr.get("model_size_reg", 0.5)
    splits = np.zeros((iterations, depth, 2), np.int32)
    leaves = np.zeros((iterations, K, 1 << depth), np.float64)
    approx = np.zeros((K, n), np.float64)
    st = np.zeros((iterations, K, n), np.float64) if staged else None
    bias = np.zeros(1, np.float64)
    rc = lib().orc_train(C.byref(p), _p(bins_fm), _p(nb), n, F, _p(t), _p(w), _p(splits),
                         _p(leaves), _p(approx), _p(st), _p(bias))
    if rc != 0:
        raise RuntimeError(f"orc_train failed rc={rc}")
    splits, is_oh = _split_flags(splits)
    out = {"splits": splits, "one_hot": is_oh, "leaf_values": leaves, "approx": approx,
           "bias": float(bias[0])}
    if staged:
        out["staged"] = st
    return out
