"""Pins the CPU restatement (oracle/) before anything is checked against it.

Each check compares the oracle with something it was not derived from: the reference's
known-answer vectors, its golden depth-6 tree, upstream catboost 1.2.10 fits, or a
brute-force recomputation of the split score from per-leaf partitions.
"""
import ctypes as C
import struct

import numpy as np
import pytest

from oracle import oracle as O
from tests import golden_data as G
from tests.trees import one_hot_bins, same_partition, upstream_one_hot_splits


def test_rng_known_answers():
    kat = G.rng_kat()
    r = O.rng_from_seed(17)
    assert O.lib().orc_rng_gen(C.byref(r)) == kat["from_seed_17_first_gen_rand"]
    r = O.rng_new(0, 1, 2, 3)
    seq = [O.lib().orc_rng_uniform(C.byref(r), 100) for _ in range(20)]
    assert seq == kat["new_0_1_2_3_uniform_100"]


def test_rng_advance_matches_stepping():
    a = O.rng_new(0, 1, 2, 3)
    b = O.rng_new(0, 1, 2, 3)
    for _ in range(100):
        O.lib().orc_rng_gen(C.byref(a))
    O.lib().orc_rng_advance(C.byref(b), 100)
    assert O.lib().orc_rng_gen(C.byref(a)) == O.lib().orc_rng_gen(C.byref(b))
    c = O.rng_from_seed(5)
    d = O.rng_from_seed(5)
    O.lib().orc_rng_advance(C.byref(d), 0)
    assert O.lib().orc_rng_gen(C.byref(c)) == O.lib().orc_rng_gen(C.byref(d))


def test_std_normal_known_answers():
    """orc_std_normal against the reference's known answers (cb-core/src/normal_test.rs:35-99):
    seed 17's first normal rejects one uniform pair (4 draws) and its second takes 2; seeds 0
    and 42 accept their first pair.  The draw counts are read off the generator state: after
    the normals it equals a fresh generator advanced by that many draws."""
    def state(r):
        return (r.x1, r.c1, r.x2, r.c2)

    r = O.rng_from_seed(17)
    n1 = O.lib().orc_std_normal(C.byref(r))
    a = O.rng_from_seed(17)
    O.lib().orc_rng_advance(C.byref(a), 4)
    assert state(r) == state(a)
    n2 = O.lib().orc_std_normal(C.byref(r))
    O.lib().orc_rng_advance(C.byref(a), 2)
    assert state(r) == state(a)
    assert abs(n1 - (-1.812286613368193e-1)) < 1e-15
    assert abs(n2 - 2.8332477304781295e-1) < 1e-15
    for seed, want in ((0, 6.337067335392765e-1), (42, 1.9692715540692288e-1)):
        r = O.rng_from_seed(seed)
        v = O.lib().orc_std_normal(C.byref(r))
        a = O.rng_from_seed(seed)
        O.lib().orc_rng_advance(C.byref(a), 2)
        assert state(r) == state(a) and abs(v - want) < 1e-15, seed


def test_real1_is_53bit_closed_interval():
    r = O.rng_from_seed(17)
    v = O.lib().orc_rng_real1(C.byref(r))
    assert v == (14895365814383052362 >> 11) * (1.0 / 9007199254740991.0)


def test_fast_logf_bit_vectors():
    rows = G.fast_logf_rows()
    assert len(rows) == 1206
    bad = 0
    for a, b in rows:
        x = struct.unpack("<f", struct.pack("<I", a))[0]
        y = struct.unpack("<I", struct.pack("<f", O.fast_logf(x)))[0]
        bad += y != b
    assert bad == 0


def test_bayesian_weights_are_per_block_streams():
    """Bayesian weights of block b depend only on (seed + b): dropping the first block and
    re-seeding must reproduce the second block (closed-form property of the sampler)."""
    r = O.rng_from_seed(3)
    sw, ctrl = O.bootstrap("Bayesian", 2500, 1.0, 1.0, r)
    assert ctrl.all() and (sw > 0).all()
    # temperature 1 => powf(x, 1) == x, weights are -FastLogf(u), mean ~ 1
    assert abs(sw.mean() - 1.0) < 0.1


def test_bernoulli_consumes_n_draws():
    r1 = O.rng_from_seed(9)
    O.bootstrap("Bernoulli", 777, 0.5, 1.0, r1)
    r2 = O.rng_from_seed(9)
    O.lib().orc_rng_advance(C.byref(r2), 777)
    assert O.lib().orc_rng_gen(C.byref(r1)) == O.lib().orc_rng_gen(C.byref(r2))


@pytest.mark.parametrize("loss", ["rmse", "logloss"])
def test_depth6_golden_tree(loss):
    cindex, fx = G.depth6()
    r = fx[loss]
    der, w = np.array(r["der1"]), np.array(r["weight"])
    out = O.grow_tree(cindex.T, np.full(cindex.shape[1], 32, np.uint32), der, w, 6, "Cosine",
                      r["scaled_l2"])
    assert [tuple(s) for s in out["splits"].tolist()] == [(s["feature"], s["bin"]) for s in r["splits"]]
    np.testing.assert_allclose(out["scores"], [s["score"] for s in r["splits"]], rtol=1e-12)
    assert np.array_equal(out["leaf_of"], np.array(r["leaf_of"]))
    sd, sw = O.leaf_sums(out["leaf_of"], 64, der, w)
    np.testing.assert_allclose(sd, [x["sum_der1"] for x in r["per_leaf"]], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(sw, [x["sum_weight"] for x in r["per_leaf"]], rtol=0, atol=0)


def _fit_upstream(name, **over):
    u = G.upstream(name)
    P = u["params"]
    bins = np.stack([O.quantize(u["X"][:, f].astype(np.float32), u["borders"][f])
                     for f in range(u["X"].shape[1])])
    K = 1
    loss = u["meta"]["loss_function"]
    if loss == "MultiClass":
        K = int(u["y"].max()) + 1
    out = O.train(bins, u["n_borders"], u["y"], loss=loss, depth=P["depth"],
                  iterations=P["iterations"], learning_rate=P["learning_rate"],
                  l2_leaf_reg=P["l2_leaf_reg"], score=P["score_function"],
                  bootstrap_type=P.get("bootstrap_type", "No"), subsample=P.get("subsample", 0.66),
                  bagging_temperature=P.get("bagging_temperature", 1.0),
                  leaf_method=P["leaf_estimation_method"], boost_from_average=P["boost_from_average"],
                  random_seed=P["random_seed"], approx_dim=K, staged=True, **over)
    return u, out, K


@pytest.mark.parametrize("name", ["bootstrap_no", "bootstrap_bayesian", "bootstrap_bernoulli",
                                  "regression_skeleton", "binclf_skeleton", "multiclass_softmax"])
def test_upstream_catboost_fit(name):
    """Full boosting loop (bootstrap draws, RNG phase, leaf estimation) against catboost 1.2.10.
    Candidate borders are the model's used borders: every chosen split is among them, so the
    argmax is unchanged and the draw count (per listed feature) is unaffected."""
    u, out, K = _fit_upstream(name)
    T = u["split_feature"].shape[0]
    for t in range(T):
        got = [(int(f), np.float32(u["borders"][f][b])) for f, b in out["splits"][t]]
        exp = [(int(f), np.float32(b)) for f, b in zip(u["split_feature"][t], u["split_border"][t])]
        assert got == exp, f"tree {t}"
        # model.json leaf values are leaf-major (leaf, dim); the oracle's are [dim][leaf]
        np.testing.assert_allclose(out["leaf_values"][t].T.reshape(-1), u["leaf_values"][t],
                                   rtol=1e-5, atol=1e-7)
    n = u["X"].shape[0]
    staged = u["staged"].reshape(T, n, K) if K > 1 else u["staged"].reshape(T, n, 1)
    np.testing.assert_allclose(out["staged"].transpose(0, 2, 1), staged, rtol=1e-5, atol=1e-6)


def _brute_scores(bins_fm, n_borders, der, w, leaf_of, n_leaves, l2, cosine=True):
    """Score every candidate from scratch: per-leaf partition sums by bincount, no histogram,
    no subtraction, no prefix scan."""
    F, n = bins_fm.shape
    res = {}
    for f in range(F):
        for b in range(int(n_borders[f])):
            new_leaf = leaf_of + (bins_fm[f] > b) * n_leaves
            s = np.bincount(new_leaf, weights=der, minlength=2 * n_leaves)
            ww = np.bincount(new_leaf, weights=w, minlength=2 * n_leaves)
            avg = np.where(ww > 0, s / (ww + l2), 0.0)
            num = float(np.sum(avg * s))
            res[(f, b)] = num / np.sqrt(1e-100 + float(np.sum(avg * avg * ww))) if cosine else num
    return res


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_tree_matches_bruteforce_partition_scoring(seed):
    rng = np.random.default_rng(seed)
    n, F, depth = 300, 5, 4
    nb = rng.integers(1, 9, size=F).astype(np.uint32)
    bins = np.stack([rng.integers(0, nb[f] + 1, size=n) for f in range(F)]).astype(np.uint8)
    der = rng.normal(size=n)
    w = rng.uniform(0.2, 2.0, size=n)
    w[rng.random(n) < 0.2] = 0.0  # sampled-out rows
    der[w == 0] = 0.0
    out = O.grow_tree(bins, nb, der, w, depth, "Cosine", 1.5, want_hists=True)
    leaf_of = np.zeros(n, np.int64)
    for level in range(depth):
        sc = _brute_scores(bins, nb, der, w, leaf_of, 1 << level, 1.5)
        best = max(sc.values())
        f, b = out["splits"][level]
        assert abs(sc[(int(f), int(b))] - best) <= 1e-12 * abs(best)
        first = min(k for k, v in sc.items() if v >= best * (1 - 1e-12))
        assert (int(f), int(b)) == first
        # histogram invariant: every feature's bins sum to the same per-leaf totals
        h = out["hists"][level]
        tot_w = np.bincount(leaf_of, weights=w, minlength=1 << level)
        np.testing.assert_allclose(h[:, :, :, 1].sum(axis=2), np.repeat(tot_w[:, None], F, 1)
                                   * (nb[None, :] > 0), rtol=1e-12, atol=1e-12)
        leaf_of = leaf_of + (bins[f] > b) * (1 << level)
    assert np.array_equal(out["leaf_of"], leaf_of)


def test_crossentropy_ders_are_the_logloss_ders():
    """cross_entropy_der1/2 (loss.rs:80-97) are defined as the Logloss ders over the same
    (soft) targets; the oracle's CrossEntropy arm equals its Logloss arm, and the Logloss ders
    hold their closed form at sampled points (der1 = t - p, der2 = -p (1 - p))."""
    g = np.random.default_rng(2)
    a = g.normal(size=1000) * 4
    t = g.random(1000)
    c1, c2 = O.ders("CrossEntropy", a, t)
    l1, l2 = O.ders("Logloss", a, t)
    assert np.array_equal(c1, l1) and np.array_equal(c2, l2)
    p = 1.0 / (1.0 + np.exp(-a))
    np.testing.assert_allclose(l1, t - p, rtol=1e-12, atol=1e-15)
    np.testing.assert_allclose(l2, -p * (1.0 - p), rtol=1e-12, atol=1e-15)


# SolarL2 / LOOL2 / SatL2 per-leaf terms (score.rs:283-350; GPU-only upstream, so no fixture
# holds them): values worked out by hand from the published formulas, edges included.
CALCER_TERMS = [
    ("SolarL2", 2.0, 3.0, -(4.0 / 3.0) * (1.0 + 2.0 * 1.3862943611198906)),   # -s^2 (1 + 2 ln 4) / 3
    ("SolarL2", -1.0, 1.0, -(1.0 + 2.0 * 0.6931471805599453)),              # ln 2
    ("SolarL2", 5.0, 1e-21, 0.0),                                            # w <= 1e-20
    ("LOOL2", 2.0, 3.0, -3.0),         # (3/2)^2 * -4 / 3
    ("LOOL2", 2.0, 1.0, 0.0),          # w <= 1: adjust 0
    ("LOOL2", 3.0, 0.5, 0.0),
    ("LOOL2", -4.0, 5.0, -(25.0 / 16.0) * 16.0 / 5.0),   # (5/4)^2 * -16 / 5 = -5
    ("SatL2", 2.0, 3.0, -4.0),         # 3 (3-2) / (9-9+1) = 3;  3 * -4 / 3
    ("SatL2", 1.0, 4.0, -0.4),         # 4 * 2 / (16-12+1) = 8/5;  1.6 * -1 / 4
    ("SatL2", 2.0, 2.0, 0.0),          # w <= 2: adjust 0
    ("SatL2", 2.0, 0.0, 0.0),
]


@pytest.mark.parametrize("score,s,w,exp", CALCER_TERMS)
def test_leaf_score_terms_hand_computed(score, s, w, exp):
    got = O.leaf_score_term(score, s, w)
    assert abs(got - exp) <= 1e-15 * max(1.0, abs(exp)), (got, exp)


def _hand_term(score, s, w):
    """The per-leaf terms as worked out above, vectorized over leaves (test-side restatement
    for the partition brute force; the constants above pin the formula itself)."""
    s = np.asarray(s, np.float64)
    w = np.asarray(w, np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        if score == "SolarL2":
            t = (-s * s) * (1.0 + 2.0 * np.log(w + 1.0)) / w
            return np.where(w > 1e-20, t, 0.0)
        if score == "LOOL2":
            adj = np.where(w > 1.0, w / (w - 1.0), 0.0) ** 2
        else:
            adj = np.where(w > 2.0, w * (w - 2.0) / (w * w - 3.0 * w + 1.0), 0.0)
        return np.where(w > 0.0, adj * (-s * s) / w, 0.0)


@pytest.mark.parametrize("score", ["SolarL2", "LOOL2", "SatL2"])
@pytest.mark.parametrize("seed", [0, 1])
def test_calcer_tree_matches_bruteforce_partition_scoring(score, seed):
    """The oracle's tree under each calcer: every level's split scores highest among the sums of
    per-leaf terms over the 2P children, from per-leaf partition sums, and no candidate before it
    in (feature, border) order scores higher (beyond f64 rounding of the fold: partitions that
    coincide tie exactly).  Few rows, integer weights: leaves cross the w = 1 and w = 2 edges."""
    rng = np.random.default_rng(10 + seed)
    n, F, depth = 60, 5, 4
    nb = rng.integers(1, 9, size=F).astype(np.uint32)
    bins = np.stack([rng.integers(0, nb[f] + 1, size=n) for f in range(F)]).astype(np.uint8)
    der = rng.normal(size=n) + 0.3 * bins[0]
    w = rng.integers(0, 3, size=n).astype(np.float64)   # integer weights: leaves cross w = 1, 2
    der[w == 0] = 0.0
    out = O.grow_tree(bins, nb, der * w, w, depth, score, 1.5)
    leaf_of = np.zeros(n, np.int64)
    for level in range(depth):
        P = 1 << level
        sc = {}
        for f in range(F):
            for b in range(int(nb[f])):
                nl = leaf_of + (bins[f] > b) * P
                ss = np.bincount(nl, weights=der * w, minlength=2 * P)
                ww = np.bincount(nl, weights=w, minlength=2 * P)
                sc[(f, b)] = float(np.sum(_hand_term(score, ss, ww)))
        best = max(sc.values())
        tol = 1e-12 * max(1.0, abs(best))
        f, b = out["splits"][level]
        chosen = sc[(int(f), int(b))]
        assert chosen >= best - tol
        assert all(v <= chosen + tol for k, v in sc.items() if k < (int(f), int(b)))
        leaf_of = leaf_of + (bins[f] > b) * P
    assert np.array_equal(out["leaf_of"], leaf_of)


# ------------------------------------------------------------------------------ one-hot
def _upstream_one_hot_fit(name):
    u = G.upstream_one_hot(name)
    p = u["params"]
    bins = one_hot_bins(u, O.quantize)
    out = O.train(bins, u["n_borders"], u["y"], loss="Logloss", depth=p["depth"],
                  iterations=p["iterations"], learning_rate=p["learning_rate"],
                  l2_leaf_reg=p["l2_leaf_reg"], score=p["score_function"], leaf_method="Gradient",
                  bootstrap_type="No", boost_from_average=p["boost_from_average"],
                  one_hot=u["one_hot"], staged=True)
    return u, bins, out


@pytest.mark.parametrize("name", ["default_binary", "multi"])
def test_one_hot_upstream_fit(name):
    """One-hot equality candidates (scan_and_score_one_hot_bins_into, histogram.rs:1175-1287;
    append_one_hot_candidates, tree.rs:1305) and the f32 learning rate (boosting.rs:4958)
    against catboost 1.2.10: same partitions every tree, leaf values (after the bit flip of a
    tied binary column) and predictions to 1e-12."""
    u, bins, out = _upstream_one_hot_fit(name)
    T = u["split_feature"].shape[0]
    for t in range(T):
        sp, oh = upstream_one_hot_splits(u, t)
        ok, flip = same_partition(bins, out["splits"][t], out["one_hot"][t], sp, oh)
        assert ok, f"tree {t}: {out['splits'][t].tolist()} vs {sp}"
        mine = out["leaf_values"][t, 0]
        perm = np.arange(mine.shape[0]) ^ flip
        np.testing.assert_allclose(mine[perm], u["leaf_values"][t], rtol=0, atol=1e-12)
    assert np.abs(out["approx"][0] - u["predictions"]).max() <= 1e-12
    assert out["one_hot"].any()


def test_one_hot_with_bootstrap_is_refused():
    """boosting.rs:5744-5756: one-hot columns with active RNG draws -> Unsupported."""
    u = G.upstream_one_hot("default_binary")
    bins = one_hot_bins(u, O.quantize)
    with pytest.raises(RuntimeError, match="rc=-4"):
        O.train(bins, u["n_borders"], u["y"], loss="Logloss", depth=2, iterations=1,
                bootstrap_type="Bernoulli", one_hot=u["one_hot"])


def _brute_scores_one_hot(bins_fm, n_borders, one_hot, der, w, leaf_of, n_leaves, l2):
    """Every float and one-hot candidate scored from scratch (bincount partitions), keyed in
    enumeration order: (0, f, b) floats first, then (1, f, v) one-hot values present."""
    res = {}
    for f in range(bins_fm.shape[0]):
        cands = np.unique(bins_fm[f]) if one_hot[f] else range(int(n_borders[f]))
        for b in cands:
            passed = (bins_fm[f] == b) if one_hot[f] else (bins_fm[f] > b)
            new_leaf = leaf_of + passed * n_leaves
            s = np.bincount(new_leaf, weights=der, minlength=2 * n_leaves)
            ww = np.bincount(new_leaf, weights=w, minlength=2 * n_leaves)
            avg = np.where(ww > 0, s / (ww + l2), 0.0)
            res[(int(one_hot[f]), f, int(b))] = float(np.sum(avg * s)) / np.sqrt(
                1e-100 + float(np.sum(avg * avg * ww)))
    return res


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_one_hot_tree_matches_bruteforce(seed):
    rng = np.random.default_rng(100 + seed)
    n, depth = 400, 4
    nb = np.array([7, 5, 0, 9, 4, 2, 6], np.uint32)      # floats: borders; one-hot: card - 1
    one_hot = np.array([0, 0, 0, 1, 1, 1, 0], np.uint8)
    bins = np.stack([rng.integers(0, nb[f] + 1, size=n) for f in range(nb.shape[0])]).astype(np.uint8)
    der = rng.normal(size=n)
    w = rng.uniform(0.2, 2.0, size=n)
    out = O.grow_tree(bins, nb, der, w, depth, "Cosine", 1.5, one_hot=one_hot)
    leaf_of = np.zeros(n, np.int64)
    for level in range(depth):
        sc = _brute_scores_one_hot(bins, nb, one_hot, der, w, leaf_of, 1 << level, 1.5)
        best = max(sc.values())
        f, b = (int(x) for x in out["splits"][level])
        key = (int(out["one_hot"][level]), f, b)
        assert key[0] == one_hot[f]
        assert abs(sc[key] - best) <= 1e-12 * abs(best)
        tied = [k for k, v in sc.items() if v >= best * (1 - 1e-12)]
        # first in enumeration order, or the complementary value of a binary one-hot column
        assert key == min(tied) or (key[0] == 1 and nb[f] == 1 and min(tied)[:2] == key[:2])
        passed = (bins[f] == b) if key[0] else (bins[f] > b)
        leaf_of = leaf_of + passed * (1 << level)
    assert np.array_equal(out["leaf_of"], leaf_of)


# ------------------------------------------------------------------------------ pairwise ranking
# l2 of the reference's own oracle tests for these fixtures: PairLogit 3 (Newton leaves,
# crates/cb-train/tests/pairlogit_oracle_test.rs:84-89), PairLogitPairwise 5
# (pairlogit_pairwise_oracle_test.rs base_params).
RANKING = {"PairLogit": (3.0, "Newton"), "PairLogitPairwise": (5.0, "Gradient")}


def ranking_bins(u):
    return np.stack([O.quantize(u["X"][:, j].astype(np.float32), u["borders"][j])
                     for j in range(u["X"].shape[1])])


@pytest.mark.parametrize("loss", sorted(RANKING))
def test_ranking_upstream_fit(loss):
    """PairLogit ders (ranking_der.rs:408-445), pairwise histogram weights, doc-weighted leaf
    centering (boosting.rs:2844-2882), and for PairLogitPairwise the pairwise split scoring
    (pairwise_scoring.rs) + Cholesky leaves (pairwise_leaves.rs), against catboost 1.2.10."""
    u = G.ranking(loss)
    l2, leaf = RANKING[loss]
    cfg = u["config"]
    bins = ranking_bins(u)
    out = O.train(bins, u["n_borders"], u["y"], loss=loss, depth=cfg["depth"],
                  iterations=cfg["iterations"], learning_rate=cfg["learning_rate"], l2_leaf_reg=l2,
                  score="Cosine", leaf_method=leaf, bootstrap_type="No",
                  pairs=(u["pairs"][:, 0], u["pairs"][:, 1]), staged=True)
    T, n = cfg["iterations"], u["X"].shape[0]
    for t in range(T):
        got = [(int(f), u["borders"][f][b]) for f, b in out["splits"][t]]
        exp = list(zip(u["split_feature"][t].tolist(), u["split_border"][t].tolist()))
        assert got == exp, f"tree {t}"
        np.testing.assert_allclose(out["leaf_values"][t, 0], u["leaf_values"][t], rtol=0, atol=1e-10)
    np.testing.assert_allclose(out["staged"][:, 0, :], u["staged"].reshape(T, n), rtol=0, atol=1e-10)
    np.testing.assert_allclose(out["approx"][0], u["predictions"], rtol=0, atol=1e-10)


def _ranking_case(seed, n_groups=12, gsize=6, pairs_per_group=5, F=3, max_b=6):
    g = np.random.default_rng(seed)
    n = n_groups * gsize
    win, los = [], []
    for q in range(n_groups):
        for _ in range(pairs_per_group):
            a, b = g.choice(gsize, 2, replace=False)
            win.append(q * gsize + a)
            los.append(q * gsize + b)
    win, los = np.array(win, np.uint32), np.array(los, np.uint32)
    wt = g.uniform(0.5, 2.0, size=win.shape[0])
    nb = g.integers(1, max_b, size=F).astype(np.uint32)
    bins = np.stack([g.integers(0, nb[f] + 1, size=n) for f in range(F)]).astype(np.uint8)
    return g, n, bins, nb, win, los, wt


def test_pairlogit_ders_closed_form():
    """der1[i] = sum_{i wins} w p - sum_{i loses} w p, p = e^{a_l} / (e^{a_l} + e^{a_w});
    der2 likewise with w p (p - 1), vectorized (no scatter order)."""
    g, n, _, _, win, los, wt = _ranking_case(3)
    a = g.normal(size=n)
    w, l, x = O.pairs_in_competitor_order(win, los, wt, n)
    d1, d2 = O.pairlogit_ders(a, w, l, x)
    p = np.exp(a[l]) / (np.exp(a[l]) + np.exp(a[w]))
    e1 = np.bincount(w, x * p, n) - np.bincount(l, x * p, n)
    e2 = np.bincount(w, x * p * (p - 1), n) + np.bincount(l, x * p * (p - 1), n)
    np.testing.assert_allclose(d1, e1, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(d2, e2, rtol=1e-12, atol=1e-14)
    pw = O.pairwise_weights(n, w, l, x)
    np.testing.assert_allclose(pw, np.bincount(w, x, n) + np.bincount(l, x, n), rtol=1e-14)


def _direct_pairwise(child, der, win, los, wt, n_children, l2, prior):
    """The leaf system of a partition built from scratch: W from the pairs incident on two
    different children, der per child, (n-1)x(n-1) solve with the priors, zero-averaged;
    score = a.der - 0.5 a.W.a."""
    W = np.zeros((n_children, n_children))
    for a_, b_, x in zip(child[win], child[los], wt):
        if a_ == b_:
            continue
        W[a_, b_] -= x
        W[b_, a_] -= x
        W[a_, a_] += x
        W[b_, b_] += x
    d = np.bincount(child, der, n_children)
    m = n_children - 1
    reg = (np.full((m, m), -prior / n_children) + np.eye(m) * (prior + l2))
    res = np.append(np.linalg.solve(W[:m, :m] + reg, d[:m]), 0.0)
    res -= res.mean()
    return res, float(res @ d - 0.5 * res @ W @ res)


@pytest.mark.parametrize("seed,level", [(0, 0), (1, 1), (2, 2), (3, 3)])
def test_pairwise_scores_match_direct_partition(seed, level):
    """The incremental per-border weight matrix of calculate_pairwise_score
    (UpdateWeightSumFromTotal / FromNonDiagStats) equals the pairwise weight matrix of the
    2P-child partition built directly (child 2y = bucket <= s, 2y+1 = bucket > s)."""
    g, n, bins, nb, win, los, wt = _ranking_case(10 + seed, n_groups=20)
    P = 1 << level
    leaf_of = g.integers(0, P, size=n).astype(np.uint32)
    der = g.normal(size=n)
    w, l, x = O.pairs_in_competitor_order(win, los, wt, n)
    for f in range(bins.shape[0]):
        B = int(nb[f]) + 1
        got = O.pairwise_feature_scores(bins[f], leaf_of, der, w, l, x, P, B, 5.0, 0.1)
        for s in range(B - 1):
            child = (2 * leaf_of + (bins[f] > s)).astype(np.int64)
            _, exp = _direct_pairwise(child, der, w.astype(np.int64), l.astype(np.int64), x, 2 * P, 5.0, 0.1)
            assert abs(got[s] - exp) <= 1e-9 * max(1.0, abs(exp)), (f, s, got[s], exp)


def test_pairwise_leaf_deltas_match_direct_solve():
    g, n, _, _, win, los, wt = _ranking_case(21, n_groups=30)
    leaf_of = g.integers(0, 8, size=n).astype(np.uint32)
    der = g.normal(size=n)
    w, l, x = O.pairs_in_competitor_order(win, los, wt, n)
    got = O.pairwise_leaf_deltas(leaf_of, der, w, l, x, 8, 3.0, 0.1)
    exp, _ = _direct_pairwise(leaf_of.astype(np.int64), der, w.astype(np.int64), l.astype(np.int64), x, 8, 3.0, 0.1)
    np.testing.assert_allclose(got, exp, rtol=1e-9, atol=1e-12)


# ------------------------------------------------------------------------------ model apply
APPLY_FIXTURES = ["regression_skeleton", "binclf_skeleton", "bootstrap_no", "bootstrap_bayesian",
                  "bootstrap_bernoulli", "multiclass_softmax"]


def upstream_model(u):
    """Flat CSR model arrays of an upstream fixture (float splits, leaf-major leaf values)."""
    T, d = u["split_feature"].shape
    K = u["leaf_values"].shape[1] >> d
    arrs = O.model_arrays(list(u["split_feature"]), list(u["split_border"]), list(u["leaf_values"]), K)
    return arrs, K


@pytest.mark.parametrize("name", APPLY_FIXTURES)
def test_apply_matches_upstream_predictions(name):
    """predict_raw (cb-model/src/apply.rs) against catboost 1.2.10 RawFormulaVal predictions
    (the last staged approximant for the multiclass fixture, whose predictions are
    probabilities)."""
    u = G.upstream(name)
    arrs, K = upstream_model(u)
    out = O.apply_oblivious(u["X"].T.astype(np.float32), *arrs, K=K, bias=u["bias"])
    n = u["X"].shape[0]
    exp = u["staged"].reshape(-1, n, K)[-1].T if K > 1 else u["predictions"][None]
    np.testing.assert_allclose(out, exp, rtol=0, atol=1e-12)


def test_apply_nan_and_absent_features():
    """NaN fails every split unless its feature is flagged (nan_mode=Max), a split on a
    feature the matrix lacks is absent, a leaf index past the tree contributes 0 -- against
    a direct per-object evaluation."""
    g = np.random.default_rng(5)
    n, F, T, d, K = 300, 6, 7, 3, 2
    x = g.normal(size=(F, n)).astype(np.float32)
    x[g.random((F, n)) < 0.1] = np.nan
    sf = [g.integers(0, F + 2, size=d) for _ in range(T)]          # F, F+1 are absent
    sb = [g.normal(size=d) for _ in range(T)]
    lv = [g.normal(size=(1 << d) * K) for _ in range(T)]
    lv[3] = lv[3][: 4 * K]                                             # a short tree: leaves 4..7 add 0
    arrs = O.model_arrays(sf, sb, lv, K)
    nan_true = (np.arange(F) % 2).astype(np.uint8)
    out = O.apply_oblivious(x, *arrs, K=K, bias=[0.5, -0.25], nan_as_true=nan_true)
    exp = np.zeros((K, n))
    for i in range(n):
        for t in range(T):
            leaf = 0
            for lvl in range(d):
                f = int(sf[t][lvl])
                if f < F:
                    v = x[f, i]
                    p = bool(nan_true[f]) if np.isnan(v) else float(v) > sb[t][lvl]
                    leaf |= int(p) << lvl
            if leaf < lv[t].size // K:
                exp[:, i] += lv[t][leaf * K:(leaf + 1) * K]
    exp += np.array([0.5, -0.25])[:, None]
    np.testing.assert_allclose(out, exp, rtol=1e-14, atol=1e-14)


# --------------------------------------------------------------------------------------
# float-feature preparation: greedy borders and bin_of
# --------------------------------------------------------------------------------------
F32_MAX = float(np.finfo(np.float32).max)


def oracle_borders_of(col, border_count, nan_mode, kind):
    """Pool::quantize's per-feature border step (quantize.rs:74-110) over the oracle."""
    has_nan = bool(np.isnan(col).any())
    b = O.select_borders(col, border_count, has_nan and nan_mode == "Min", kind)
    if has_nan and nan_mode == "Max":
        b = np.append(b, F32_MAX)
    return b


def test_borders_match_upstream_fixtures():
    """Every greedy cell of border_types/ and borders_quant/ (catboost 1.2.10 standalone
    quantization) reproduced exactly, per feature."""
    cells, mats = G.borders()
    assert len(cells) == 20
    for c in cells:
        X = mats[c["dataset"]].astype(np.float32)
        for f, want in enumerate(c["borders"]):
            got = oracle_borders_of(X[:, f], c["border_count"], c["nan_mode"], c["border_type"])
            assert np.array_equal(got.astype(np.float32), want.astype(np.float32)), (c["stem"], f)


def test_borders_tiny_known_answers():
    # two distinct values -> one border, the f32 midpoint (borders_test.rs two-value case)
    assert O.select_borders(np.array([-1.0, 1.0], np.float32), 8).tolist() == [0.0]
    b = O.select_borders(np.array([1.0, 2.0], np.float32), 8)
    assert b.tolist() == [float(np.float32(0.5) * np.float32(1) + np.float32(0.5) * np.float32(2))]
    # constant, empty and all-NaN columns have no border; the Min sentinel still leads
    assert O.select_borders(np.full(10, 3.0, np.float32), 8).size == 0
    assert O.select_borders(np.zeros(0, np.float32), 8).size == 0
    assert O.select_borders(np.full(4, np.nan, np.float32), 8, True).tolist() == [
        float(np.finfo(np.float32).min)]
    # -0/+0 midpoint normalizes to +0
    z = O.select_borders(np.array([-0.0, -0.0, 0.0, 1.0], np.float32), 8)
    assert all(np.copysign(1.0, v) > 0 for v in z if v == 0.0)


def test_borders_are_order_free_and_budgeted():
    """A pure function of the value multiset; never over budget; ascending; inside range."""
    rng = np.random.default_rng(3)
    col = np.round(rng.normal(size=3000) * 4).astype(np.float32) / 4
    for k in (1, 2, 7, 31, 128, 254):
        a = O.select_borders(col, k)
        assert a.size <= k and np.all(np.diff(a) > 0)
        assert a[0] > col.min() and a[-1] < col.max()
        assert np.array_equal(a, O.select_borders(col[::-1].copy(), k))
        assert np.array_equal(a, O.select_borders(rng.permutation(col), k))
    # budget reached on a column with enough distinct values; one slot goes to the sentinel
    u = np.arange(1000, dtype=np.float32)
    assert O.select_borders(u, 31).size == 31
    assert O.select_borders(np.append(u, np.nan).astype(np.float32), 31, True).size == 31


def test_border_sample_is_a_fixed_seed_fisher_yates():
    """sample_indices_for_build_borders (borders.rs:504-516): partial Fisher-Yates over
    TFastRng64.from_seed(0) (uniform() pinned by the rng known answers), sorted."""
    n, k = 200_000 + 7_345, 200_000
    idx = np.arange(n, dtype=np.int64)
    r = O.rng_from_seed(0)
    for i in range(k):
        off = O.lib().orc_rng_uniform(C.byref(r), n - i)
        idx[i], idx[i + off] = idx[i + off], idx[i]
    want = np.sort(idx[:k])
    got = O.sample_indices_for_borders(n)
    assert np.array_equal(got.astype(np.int64), want)
    assert np.array_equal(O.sample_indices_for_borders(1000), np.arange(1000))


def test_oversized_column_is_subsampled_before_nan_drop():
    """Above 200000 rows the borders come from the sampled objects, NaN dropped after the
    draw (borders_test.rs presampled case) -- and the smooth-column quality bound of
    borders_test.rs (g): 31 borders, each within 0.01 of the uniform quantile."""
    n = 200_000 * 2 + 12_345
    i = np.arange(n, dtype=np.uint64)
    h = i * np.uint64(0x9E3779B97F4A7C15)
    h = (h << np.uint64(31)) | (h >> np.uint64(33))
    col = ((h >> np.uint64(40)).astype(np.float32) / np.float32(1 << 24)) * np.float32(2e3) - np.float32(1e3)
    col[(h % np.uint64(7)) == 0] = 42.5
    col[(h % np.uint64(100)) == 0] = np.nan
    s = O.sample_indices_for_borders(n)
    assert np.array_equal(O.select_borders(col, 31), O.select_borders(col[s], 31))
    n3 = 600_000
    j = np.arange(n3, dtype=np.uint64)
    g = j * np.uint64(0x9E3779B97F4A7C15)
    g = (g << np.uint64(31)) | (g >> np.uint64(33))
    smooth = (g >> np.uint64(40)).astype(np.float32) / np.float32(1 << 24)
    a = O.select_borders(smooth, 31)
    assert a.size == 31
    assert np.all(np.abs(a - (np.arange(31) + 1) / 32.0) < 0.01)


def test_quantize_is_bin_of():
    """bin_of (histogram.rs:563-569) by brute force: count of borders strictly below the
    value; NaN to the top bin behind an f32::MAX last border, else bin 0."""
    rng = np.random.default_rng(5)
    b = np.unique(rng.normal(size=40).astype(np.float32)).astype(np.float64)
    v = np.concatenate([rng.normal(size=500).astype(np.float32), b.astype(np.float32),
                        np.array([np.nan, np.inf, -np.inf, 0.0, -0.0], np.float32)])
    brute = np.array([0 if np.isnan(x) else int(np.sum(b < float(x))) for x in v])
    assert np.array_equal(O.quantize(v, b), brute)
    bm = np.append(b, F32_MAX)
    brute_m = np.array([len(bm) if np.isnan(x) else int(np.sum(bm < float(x))) for x in v])
    assert np.array_equal(O.quantize(v, bm), brute_m)
    assert O.quantize(v, np.zeros(0)).max() == 0


# --------------------------------------------------------------------------------------
# categorical inputs: learn permutations, first-seen bins, online CTR columns
# --------------------------------------------------------------------------------------
CTR_SCENARIOS = ("plain_ctr", "ordered_ctr", "tensor_ctr", "one_hot_cat")


def test_permutations_match_upstream():
    """create_shuffled_indices / permutations (permutation.rs) against catboost 1.2.10's fold
    permutations; fold 1 continues the same stream."""
    g = G.categorical()
    for scen in CTR_SCENARIOS:
        want = g[scen + ".permutation_fold0"]
        assert np.array_equal(O.shuffled_indices(want.size, int(g[scen + ".seed"])), want), scen
    two = O.permutations(30, 2, 0)
    assert np.array_equal(two[0], g["ordered_ctr.permutation_fold0"])
    assert np.array_equal(two[1], g["ordered_ctr.permutation_fold1"])


def test_ctr_value_formula_matches_upstream_anchors():
    """calc_ctr_online (num + prior) / (total + 1) reproduces catboost's per-object CTR values
    from its own integer anchors, in all four scenarios (catboost keeps them in f32: equal
    after rounding to f32)."""
    g = G.categorical()
    for scen in CTR_SCENARIOS:
        good, total = g[scen + ".ctr_good_count"].astype(float), g[scen + ".ctr_total_count"]
        calc = (good + float(g[scen + ".prior"])) / (total + 1.0)
        assert np.array_equal(calc.astype(np.float32), g[scen + ".ctr_value"].astype(np.float32)), scen
        assert np.all((good >= 0) & (good <= total))


def test_perfect_hash_matches_upstream_bins():
    g = G.categorical()
    h, b = g["cat_hash.hashes"], g["cat_hash.bins"]
    n = h.size // 2
    for c in range(2):
        bins, d = O.perfect_hash(h[c * n:(c + 1) * n])
        assert np.array_equal(bins, b[c * n:(c + 1) * n]) and d == int(b[c * n:(c + 1) * n].max()) + 1


def test_perfect_hash_is_first_seen_order():
    rng = np.random.default_rng(1)
    keys = rng.integers(0, 2**32, 50, dtype=np.uint64).astype(np.uint32)[rng.integers(0, 50, 3000)]
    bins, d = O.perfect_hash(keys)
    seen = {}
    want = np.array([seen.setdefault(int(k), len(seen)) for k in keys], np.uint32)
    assert np.array_equal(bins, want) and d == len(seen)


def _bruteforce_ctr(kind, bucket, perm, cls, prior, tbi, bc):
    """Independent recount: per bucket, the classes of its objects in permutation order."""
    n = bucket.size
    pos = np.empty(n, np.int64)
    pos[perm] = np.arange(n)
    n0 = np.zeros(n, np.int64)
    n1 = np.zeros(n, np.int64)
    size = np.bincount(bucket, minlength=int(bucket.max()) + 1)
    for b in np.unique(bucket):
        objs = np.nonzero(bucket == b)[0]
        objs = objs[np.argsort(pos[objs])]
        c = cls[objs].astype(np.int64)
        n1[objs] = np.cumsum(c) - c
        n0[objs] = np.arange(objs.size) - n1[objs]
    total = n0 + n1
    if kind == "Counter":
        num, total = size[bucket].astype(float), np.full(n, size.max())
    elif kind == "Buckets":
        num = (n0 if tbi == 0 else n1 if tbi == 1 else 0 * n0).astype(float)
    elif kind == "Borders":
        num = (n1 if tbi == 0 else 0 * n1).astype(float)
    else:  # BinarizedTargetMeanValue: f32 running sum of ones
        num = np.minimum(n1, 2**24).astype(np.float32).astype(float)
    value = (num + prior) / (total + 1.0)
    shift, norm = -min(0.0, prior), max(1.0, prior) - min(0.0, prior)
    if kind == "BinarizedTargetMeanValue":
        c32 = (num.astype(np.float32) + np.float32(prior)) / (total.astype(np.float32) + np.float32(1))
        bf = (((c32 + np.float32(shift)) / np.float32(norm)) * np.float32(bc)).astype(float)
    else:
        bf = (value + shift) / norm * bc
    return dict(good=num, total=total, value=value, bin=np.clip(np.trunc(bf), 0, bc).astype(np.uint8))


@pytest.mark.parametrize("kind,tbi", [("Borders", 0), ("Borders", 1), ("Buckets", 0), ("Buckets", 1),
                                      ("BinarizedTargetMeanValue", 0), ("Counter", 0)])
@pytest.mark.parametrize("prior", [0.0, 0.5, 1.0, 2.0, -0.5])
def test_ctr_column_matches_bruteforce(kind, tbi, prior):
    rng = np.random.default_rng(7)
    n = 4000
    bucket = np.minimum(rng.zipf(1.3, n) - 1, 300).astype(np.uint32)
    bucket = O.perfect_hash(bucket)[0]
    perm = O.shuffled_indices(n, 3)
    cls = (rng.random(n) < 0.4).astype(np.uint8)
    got = O.ctr_column(kind, bucket, perm, cls, prior=prior, target_border_idx=tbi)
    exp = _bruteforce_ctr(kind, bucket, perm, cls, prior, tbi, 15)
    for k in ("good", "total", "value", "bin"):
        assert np.array_equal(got[k], exp[k]), k


def test_ctr_hand_scenarios():
    """The read-before-increment scenarios of plain_ctr_oracle_test.rs / tensor_ctr_oracle_test.rs."""
    r = O.ctr_column("Borders", [0, 0, 0, 0], [0, 1, 2, 3], [1, 0, 1, 1], prior=0.5)
    assert r["value"].tolist() == [0.5, 0.75, 0.5, 0.625]
    assert r["bin"].tolist() == [7, 11, 7, 9]
    # (p,x) (p,y) (q,x) (p,x) (q,y) (q,x) as first-seen buckets, identity order
    combo = O.perfect_hash(np.array([0, 1, 2, 0, 3, 2], np.uint32))[0]
    r = O.ctr_column("Borders", combo, np.arange(6), [1, 0, 1, 0, 1, 1], prior=0.5)
    assert r["good"].tolist() == [0, 0, 0, 1, 0, 1] and r["total"].tolist() == [0, 0, 0, 1, 0, 1]
    assert r["value"][3] == 0.75


@pytest.mark.parametrize("name", ["counter", "btmv", "mixed"])
def test_ctr_fit_matches_upstream(name):
    """catboost 1.2.10 CTR fits (Counter / BinarizedTargetMeanValue / Borders, prior 0.5,
    model_size_reg 0.5, Logloss depth 2 x 5, L2): every split (CTR borders in value space) and
    every leaf value reproduced -- online CTR columns under the learn permutation, the
    model_size_reg weights, leaves over the averaging-permutation columns."""
    from tests.trees import ctr_fit_inputs, ctr_tree_matches
    u = G.ctr_fit(name)
    fit = ctr_fit_inputs(u, O)
    P = u["params"]
    r = O.train(fit["bins"], fit["n_borders"], u["y"], loss=P["loss_function"], depth=P["depth"],
                iterations=P["iterations"], learning_rate=P["learning_rate"], l2_leaf_reg=P["l2_leaf_reg"],
                score=P["score_function"], bootstrap_type="No", boost_from_average=P["boost_from_average"],
                random_seed=0, ctr=fit["ctr"])
    for t in range(P["iterations"]):
        assert ctr_tree_matches(u, fit, r["splits"][t], r["leaf_values"][t][0], t, None), f"tree {t}"


def test_ctr_fit_buckets_first_tree_up_to_mirror_tie():
    """The Buckets fit has two complementary columns (class 0 and class 1 counts of one
    projection), whose mirrored splits tie exactly in real arithmetic; the first tree's
    partition and leaf values are reproduced (catboost takes the other side of the tie), later
    trees are not pinned."""
    from tests.trees import ctr_fit_inputs
    u = G.ctr_fit("buckets")
    fit = ctr_fit_inputs(u, O)
    P = u["params"]
    r = O.train(fit["bins"], fit["n_borders"], u["y"], loss=P["loss_function"], depth=P["depth"], iterations=1,
                learning_rate=P["learning_rate"], l2_leaf_reg=P["l2_leaf_reg"], score=P["score_function"],
                bootstrap_type="No", boost_from_average=P["boost_from_average"], random_seed=0, ctr=fit["ctr"])
    F0, av = fit["n_float"], fit["ctr"]["avg_bins"]
    n = u["y"].size
    el, gl = np.zeros(n, int), np.zeros(n, int)
    for l, (is_ctr, idx, border) in enumerate(u["trees"][0]):
        assert is_ctr
        el |= (av[idx] > int(round(border - 1))).astype(int) << l
    for l, (f, b) in enumerate(r["splits"][0]):
        gl |= ((av[f - F0] if f >= F0 else fit["bins"][f]) > b).astype(int) << l
    relabel = {}
    assert all(relabel.setdefault(int(a), int(b)) == int(b) for a, b in zip(el, gl))   # same grouping
    assert len(set(relabel.values())) == len(relabel)
    np.testing.assert_allclose(r["leaf_values"][0][0][gl], u["leaf_values"][0][el], rtol=1e-9, atol=1e-15)
