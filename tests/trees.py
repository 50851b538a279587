"""Tree helpers shared by the oracle and GPU one-hot tests: per-row leaf indices,
partition equivalence, and the fixtures' bins / splits on the device feature axis."""
from __future__ import annotations

import numpy as np


def one_hot_bins(u, quantize):
    """Fixture bins [F][n]: float columns through ``quantize(values_f32, borders)``, then the
    categorical first-seen bins."""
    fb = [quantize(u["X"][:, j].astype(np.float32), u["borders"][j]) for j in range(u["n_float"])]
    return np.stack(fb + list(u["cat_bins"])).astype(np.uint8)


def tree_rows(bins, splits, one_hot):
    """Per-row leaf index of one oblivious tree (bit l = pass of the level-l split)."""
    idx = np.zeros(bins.shape[1], np.int64)
    for lvl, ((f, b), oh) in enumerate(zip(splits, one_hot)):
        col = bins[int(f)]
        idx |= ((col == b) if oh else (col > b)).astype(np.int64) << lvl
    return idx


def same_partition(bins, splits_a, oh_a, splits_b, oh_b):
    """Two trees induce the same leaf partition, up to the bit flips of a binary one-hot
    column tested on its other value (complementary equality splits are exactly tied)."""
    ia = tree_rows(bins, splits_a, oh_a)
    ib = tree_rows(bins, splits_b, oh_b)
    flip = 0
    for lvl in range(len(splits_a)):
        (fa, ba), (fb, bb) = splits_a[lvl], splits_b[lvl]
        if (int(fa), int(ba), bool(oh_a[lvl])) == (int(fb), int(bb), bool(oh_b[lvl])):
            continue
        col = bins[int(fa)]
        binary = oh_a[lvl] and oh_b[lvl] and fa == fb and int(col.max()) == 1
        if not binary:
            return False, None
        flip |= 1 << lvl
    return bool(np.array_equal(ia ^ flip, ib)), flip


def upstream_one_hot_splits(u, t):
    """Upstream tree t as (feature on the device axis, bin id) + one-hot flags."""
    sp, oh = [], []
    for lvl in range(u["split_feature"].shape[1]):
        if u["split_one_hot"][t, lvl]:
            sp.append((u["n_float"] + int(u["split_feature"][t, lvl]), int(u["split_value_bin"][t, lvl])))
            oh.append(True)
        else:
            f = int(u["split_feature"][t, lvl])
            b = int(np.searchsorted(u["borders"][f], u["split_border"][t, lvl]))
            assert u["borders"][f][b] == u["split_border"][t, lvl]
            sp.append((f, b))
            oh.append(False)
    return sp, oh


def ctr_fit_inputs(u, O, seed=0):
    """Inputs of a CTR fit from a ``golden_data.ctr_fit`` record, built with the oracle ``O``:
    float bins over the full border set, first-seen buckets of the categorical codes, the
    learn permutation S and the averaging permutation Q = S[P_avg] (permutations(n, 2, seed):
    one learning fold, boosting.rs:5470-5520), the CTR columns of every spec under both."""
    import numpy as np
    X, y, B = u["X"], u["y"], u["borders"]
    n, F0 = X.shape
    fb = np.stack([O.quantize(X[:, j], B[j]) for j in range(F0)])
    bucket, nb = O.perfect_hash(np.asarray(u["X_cat"]).reshape(n, -1)[:, 0].astype(np.uint32))
    st = O.permutations(n, 2, seed)
    S, Q = st[0], st[0][st[1]]
    cls = (y > 0.5).astype(np.uint8)
    col = lambda perm: np.stack([O.ctr_column(t, bucket, perm, cls, prior=pr, target_border_idx=tb)["bin"]
                                 for t, pr, tb in u["specs"]])
    sc, av = col(S), col(Q)
    groups = {}
    group = np.array([groups.setdefault(t, len(groups)) for t, _, _ in u["specs"]], np.uint32)
    return dict(bins=np.concatenate([fb, sc]), n_borders=np.full(F0 + sc.shape[0], 15, np.uint32),
                n_float=F0, ctr=dict(avg_bins=av, bucket_count=np.full(sc.shape[0], nb, np.uint32), group=group,
                                     cat_buckets=bucket[None, :], cat_bucket_count=np.array([nb], np.uint32),
                                     model_size_reg=0.5))


def ctr_tree_matches(u, fit, splits, leaves, t, bins_avg_float):
    """Tree t of a CTR fit against catboost's: the same splits (CTR borders in catboost's value
    space (b + 1) - 2^-20, computed in f32) and leaf values to 1e-9 relative."""
    import numpy as np
    F0 = fit["n_float"]
    got = []
    for f, b in splits:
        if f < F0:
            got.append((0, int(f), float(np.float32(u["borders"][f][b]))))
        else:
            tb = u["specs"][f - F0][2]
            got.append((1, tb, float(np.float32(np.float32(b) + np.float32(1)) - np.float32(2.0 ** -20))))
    exp = [(k, i, float(np.float32(b))) for k, i, b in u["trees"][t]]
    return got == exp and np.allclose(leaves, u["leaf_values"][t], rtol=1e-9, atol=1e-15)


def level_tie_levels(bins, splits_a, splits_b):
    """Levels where two oblivious trees choose different float splits that are tied in exact
    arithmetic whatever the row statistics: before the level both trees hold the same leaf
    partition (as sets of rows), and in every leaf the two candidates send the same rows to
    one side -- TRUE of one is TRUE or FALSE of the other.  The score (Cosine or L2) is a sum
    over (leaf, side) of terms that depend on that side's rows only, so such candidates fold
    the same terms in another order and their exact scores are equal.  Returns the tied
    levels; raises AssertionError when a differing level is not such a tie."""
    n = bins.shape[1]
    ia = np.zeros(n, np.int64)
    ib = np.zeros(n, np.int64)
    tied = []
    for lvl, ((fa, ba), (fb, bb)) in enumerate(zip(splits_a, splits_b)):
        pa = bins[int(fa)] > ba
        pb = bins[int(fb)] > bb
        pairs = np.unique(np.stack([ia, ib]), axis=1)
        assert pairs.shape[1] == np.unique(ia).size == np.unique(ib).size, \
            f"level {lvl}: the leaf partitions before the level differ"
        if (int(fa), int(ba)) != (int(fb), int(bb)):
            for leaf in np.unique(ia):
                rows = ia == leaf
                same = np.array_equal(pa[rows], pb[rows])
                swapped = np.array_equal(pa[rows], ~pb[rows])
                assert same or swapped, f"level {lvl}: candidates ({fa},{ba}) and ({fb},{bb}) split a leaf differently"
            tied.append(lvl)
        ia |= pa.astype(np.int64) << lvl
        ib |= pb.astype(np.int64) << lvl
    return tied


def exact_cosine_terms(bins, prior_splits, cand, der, w, lam):
    """Numerator and denominator of the Cosine score of candidate ``cand`` = (feature, bin)
    after the levels ``prior_splits``, in exact rational arithmetic over the f64 inputs:
    sum over (leaf, side) of avg * s and avg^2 * W, s = sum w der, W = sum w,
    avg = s / (W + lam) when W > 0 (score.rs:93-147, leaf.rs:161)."""
    from fractions import Fraction as Fr
    leaf = np.zeros(bins.shape[1], np.int64)
    for lvl, (f, b) in enumerate(prior_splits):
        leaf |= (bins[int(f)] > b).astype(np.int64) << lvl
    side = bins[int(cand[0])] > cand[1]
    lam = Fr(float(lam))
    num, den = Fr(0), Fr(0)
    for key in np.unique(leaf * 2 + side):
        rows = np.nonzero(leaf * 2 + side == key)[0]
        s = sum((Fr(float(w[i])) * Fr(float(der[i])) for i in rows), Fr(0))
        W = sum((Fr(float(w[i])) for i in rows), Fr(0))
        if W > 0:
            avg = s / (W + lam)
            num += avg * s
            den += avg * avg * W
    return num, den
