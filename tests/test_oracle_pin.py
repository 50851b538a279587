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
