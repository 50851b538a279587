"""GPU parity of float-feature preparation: greedy border selection (cbh_select_borders),
device quantization (cbh_quantize) and the raw float channel of the training session
(cbh_session_begin_raw / cbt_open_raw), against the oracle and catboost 1.2.10's borders.

Bars: border sets equal to the oracle's bit for bit (and to the fixtures at f32, the
precision they were stored in); bins bit-exact; a session opened over raw floats grows
exactly the trees, leaves and approximant of a session opened over the same bins.
"""
import numpy as np
import pytest

import catboost_rs_amd as cb
from catboost_rs_amd import datagen
from oracle import oracle as O
from tests import golden_data as G
from tests.test_oracle_pin import oracle_borders_of

pytestmark = pytest.mark.gpu


def _same_sets(got, exp, tag):
    assert len(got) == len(exp), tag
    for f, (a, b) in enumerate(zip(got, exp)):
        assert np.array_equal(np.asarray(a).view(np.uint64), np.asarray(b, np.float64).view(np.uint64)), (tag, f)


def test_select_borders_matches_upstream_fixtures():
    cells, mats = G.borders()
    for c in cells:
        X = mats[c["dataset"]].astype(np.float32)
        got = cb.select_borders(X.T, c["border_count"], c["nan_mode"], c["border_type"])
        exp = [oracle_borders_of(X[:, f], c["border_count"], c["nan_mode"], c["border_type"])
               for f in range(X.shape[1])]
        _same_sets(got, exp, c["stem"])
        for f, want in enumerate(c["borders"]):
            assert np.array_equal(got[f].astype(np.float32), want.astype(np.float32)), (c["stem"], f)


@pytest.mark.parametrize("kind", ["GreedyLogSum", "GreedyMinEntropy"])
def test_select_borders_adversarial_values(kind):
    """Radix-sorted device values give the comparator-sort borders: negatives, -0/+0,
    subnormals, infinities, f32 extremes, heavy duplication (borders_test.rs adversarial)."""
    f32 = np.finfo(np.float32)
    specials = np.array([-np.inf, f32.min, -1.5, -f32.tiny, -0.0, 0.0, f32.tiny, 1e-30, 1.5,
                         f32.max, np.inf, 1e-45, -1e-45], np.float32)
    g = np.random.default_rng(11)
    cols = []
    for j in range(6):
        c = (g.random(8192).astype(np.float32) * 2e3 - 1e3).astype(np.float32)
        m = g.random(8192) < (0.33 + 0.1 * j)
        c[m] = specials[g.integers(0, specials.size, m.sum())]
        cols.append(c)
    X = np.stack(cols)
    for k in (8, 31, 254):
        got = cb.select_borders(X, k, "Min", kind)
        exp = [oracle_borders_of(X[j], k, "Min", kind) for j in range(X.shape[0])]
        _same_sets(got, exp, (kind, k))


@pytest.mark.parametrize("nan_mode", ["Min", "Max", "Forbidden"])
def test_select_borders_sampled_columns(nan_mode):
    """412345 rows (over the 200000-row subset cap): mixed columns -- smooth, lognormal,
    few distinct values, NaN-bearing, constant, all-NaN -- match the oracle."""
    n = 412_345
    g = np.random.default_rng(21)
    cols = [g.standard_normal(n).astype(np.float32),
            np.exp(g.standard_normal(n)).astype(np.float32),
            g.integers(0, 7, n).astype(np.float32),
            np.full(n, 2.5, np.float32),
            np.full(n, np.nan, np.float32)]
    c = g.standard_normal(n).astype(np.float32)
    c[g.random(n) < 0.05] = np.nan
    cols.append(c)
    c = np.round(g.standard_normal(n) * 3).astype(np.float32)
    c[g.random(n) < 1e-5] = np.nan  # NaNs that the subset may miss: the mode still applies
    cols.append(c)
    X = np.stack(cols)
    bc = 254 if nan_mode == "Max" else 255
    got = cb.select_borders(X, bc, nan_mode)
    exp = [oracle_borders_of(X[j], bc, nan_mode, "GreedyLogSum") for j in range(X.shape[0])]
    _same_sets(got, exp, nan_mode)
    # small budget on the same columns
    got = cb.select_borders(X, 16, nan_mode, "GreedyMinEntropy")
    exp = [oracle_borders_of(X[j], 16, nan_mode, "GreedyMinEntropy") for j in range(X.shape[0])]
    _same_sets(got, exp, (nan_mode, 16))


def test_quantize_matches_oracle():
    g = np.random.default_rng(31)
    v = g.standard_normal(1_000_003).astype(np.float32)
    v[g.random(v.size) < 0.01] = np.nan
    v[:6] = [np.inf, -np.inf, 0.0, -0.0, np.float32(np.finfo(np.float32).max), np.nan]
    b = np.unique(g.standard_normal(200).astype(np.float32)).astype(np.float64)
    assert np.array_equal(cb.quantize(v, b), O.quantize(v, b))
    bmax = np.append(b[:100], float(np.finfo(np.float32).max))  # NaN -> top bin
    assert np.array_equal(cb.quantize(v, bmax), O.quantize(v, bmax))
    assert np.array_equal(cb.quantize(v, np.zeros(0)), np.zeros(v.size, np.uint8))
    v[::3] = b[g.integers(0, b.size, v[::3].size)]  # values on a border stay below it
    assert np.array_equal(cb.quantize(v, b), O.quantize(v, b))


def _fit(tr, iterations):
    try:
        splits, leaves = tr.fit(iterations)
        return splits, leaves, tr.approx()
    finally:
        tr.close()


@pytest.mark.parametrize("loss", ["RMSE", "Logloss"])
def test_raw_channel_equals_bin_channel(loss):
    """Device-selected borders -> raw float session == host-binned session (same trees,
    leaves and approximant bit for bit), with NaN-bearing columns under nan_mode=Max."""
    g = np.random.default_rng(41)
    n, F = 60_000, 24
    X = g.standard_normal((F, n)).astype(np.float32)
    X[3, g.random(n) < 0.1] = np.nan
    X[7] = np.round(X[7] * 2)
    w = g.uniform(-1, 1, F)
    z = np.nan_to_num(X).T.astype(np.float64) @ w
    y = z + 0.1 * g.standard_normal(n) if loss == "RMSE" else (g.random(n) < 1 / (1 + np.exp(-z))).astype(float)
    borders = cb.select_borders(X, 64, "Max")
    nb = np.array([b.size for b in borders], np.uint32)
    bins = np.stack([O.quantize(X[f], borders[f]) for f in range(F)])
    kw = dict(loss=loss, depth=6, learning_rate=0.1, l2_leaf_reg=3.0, score="Cosine",
              boost_from_average=loss == "RMSE", bootstrap_type="Bernoulli", subsample=0.7,
              random_seed=5)
    a = _fit(cb.Trainer.from_floats(X, borders, y, **kw), 12)
    b = _fit(cb.Trainer(bins, int(nb.max()) + 1, y, real_folds=nb + 1, **kw), 12)
    assert np.array_equal(a[0], b[0])
    assert np.array_equal(a[1], b[1])
    assert np.array_equal(a[2], b[2])
    oracle = O.train(bins, nb, y, loss=loss, depth=6, iterations=12, learning_rate=0.1,
                     l2_leaf_reg=3.0, score="Cosine", bootstrap_type="Bernoulli", subsample=0.7,
                     boost_from_average=loss == "RMSE", random_seed=5)
    assert np.array_equal(a[0], oracle["splits"])


def test_upstream_fit_from_raw_floats():
    """catboost 1.2.10's regression skeleton fit reproduced over the raw float channel with
    the model's borders: the device bins equal the host bins, so splits and leaves match."""
    u = G.upstream("regression_skeleton")
    P = u["params"]
    X = np.ascontiguousarray(u["X"].T.astype(np.float32))
    tr = cb.Trainer.from_floats(X, u["borders"], u["y"], loss=u["meta"]["loss_function"],
                                depth=P["depth"], learning_rate=P["learning_rate"],
                                l2_leaf_reg=P["l2_leaf_reg"], score=P["score_function"],
                                leaf_method=P["leaf_estimation_method"],
                                boost_from_average=P["boost_from_average"], random_seed=P["random_seed"])
    splits, leaves, approx = _fit(tr, P["iterations"])
    for t in range(P["iterations"]):
        got = [(int(f), np.float32(u["borders"][f][b])) for f, b in splits[t]]
        exp = [(int(f), np.float32(b)) for f, b in zip(u["split_feature"][t], u["split_border"][t])]
        assert got == exp, f"tree {t}"
        np.testing.assert_allclose(leaves[t].reshape(-1), u["leaf_values"][t], rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(approx[0], u["staged"].reshape(P["iterations"], -1)[-1], rtol=1e-5, atol=1e-6)


def test_config1_from_floats_end_to_end():
    """Config 1 from its float matrix: device border selection (128, GreedyLogSum), device
    quantization, 10 trees -- the same trees as the oracle over the oracle's borders."""
    d = datagen.config1()
    P = d["params"]
    X = np.ascontiguousarray(d["features"].T)
    borders = cb.select_borders(X, 128)
    exp_b = [oracle_borders_of(X[f], 128, "Min", "GreedyLogSum") for f in range(X.shape[0])]
    _same_sets(borders, exp_b, "config1")
    tr = cb.Trainer.from_floats(X, borders, d["target"], loss=P["loss"], depth=P["depth"],
                                learning_rate=P["learning_rate"], l2_leaf_reg=P["l2_leaf_reg"],
                                score=P["score"], leaf_method=P["leaf_method"], boost_from_average=True)
    splits, leaves, approx = _fit(tr, 10)
    nb = np.array([b.size for b in exp_b], np.uint32)
    bins = np.stack([O.quantize(X[f], exp_b[f]) for f in range(X.shape[0])])
    exp = O.train(bins, nb, d["target"], loss="RMSE", depth=6, iterations=10, learning_rate=0.1,
                  l2_leaf_reg=3.0, score="Cosine", boost_from_average=True)
    assert np.array_equal(splits, exp["splits"])
    np.testing.assert_allclose(approx, exp["approx"], rtol=1e-5, atol=1e-9)


def test_config2_from_raw_floats_matches_oracle():
    """Config 2 at 200k rows from its raw f32 columns, as the benchmark feeds it: the 254
    GreedyLogSum borders selected on the device equal the oracle's for all 200 columns, and
    the session over the raw float channel (device quantization) grows the oracle's trees."""
    from tests.test_gpu_parity import _close
    d = datagen.config2_raw(n_rows=200_000)
    X, P = d["floats"], d["params"]
    borders = cb.select_borders(X, P["border_count"], "Min", P["border_type"])
    exp_b = [oracle_borders_of(X[f], P["border_count"], "Min", P["border_type"]) for f in range(X.shape[0])]
    _same_sets(borders, exp_b, "config2")
    nb = np.array([b.size for b in exp_b], np.uint32)
    bins = np.stack([O.quantize(X[f], exp_b[f]) for f in range(X.shape[0])])
    kw = dict(loss=P["loss"], depth=P["depth"], learning_rate=P["learning_rate"], l2_leaf_reg=P["l2_leaf_reg"],
              score=P["score"], leaf_method=P["leaf_method"], bootstrap_type=P["bootstrap_type"],
              bagging_temperature=P["bagging_temperature"], boost_from_average=P["boost_from_average"],
              random_seed=P["random_seed"])
    splits, leaves, approx = _fit(cb.Trainer.from_floats(X, borders, d["target"], **kw), 8)
    exp = O.train(bins, nb, d["target"], iterations=8, n_threads=16, **kw)
    assert np.array_equal(splits, exp["splits"])
    _close(leaves, exp["leaf_values"])
    _close(approx, exp["approx"])
