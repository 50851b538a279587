"""GPU parity of the categorical inputs: first-seen bins (cbh_perfect_hash) and online CTR
columns (cbh_ctr_columns) against the oracle and catboost 1.2.10's fixtures.

Bars: bins, counts and CTR bins bit-exact; CTR values bit-equal (the same f64 formula over
the same exact integer counts).
"""
import numpy as np
import pytest

import catboost_rs_amd as cb
from oracle import oracle as O
from tests import golden_data as G

pytestmark = pytest.mark.gpu

SPECS = [("Borders", 0.0), ("Borders", 0.5), ("Borders", 1.0), ("Borders", 0.5, 1), ("Buckets", 0.5, 0),
         ("Buckets", 0.5, 1), ("BinarizedTargetMeanValue", 0.5), ("Counter", 0.0), ("Counter", 0.5),
         ("Borders", 2.0), ("Borders", -0.5)]


def _oracle_cols(bucket, perm, cls, specs, bc=15):
    out = [O.ctr_column(sp[0], bucket, perm, cls, prior=sp[1], target_border_idx=sp[2] if len(sp) > 2 else 0,
                        border_count=bc) for sp in specs]
    return np.stack([o["bin"] for o in out]), np.stack([o["value"] for o in out])


def test_perfect_hash_matches_fixture_and_oracle():
    g = G.categorical()
    h, b = g["cat_hash.hashes"], g["cat_hash.bins"]
    n = h.size // 2
    for c in range(2):
        bins, d = cb.perfect_hash(h[c * n:(c + 1) * n])
        assert np.array_equal(bins, b[c * n:(c + 1) * n])
    rng = np.random.default_rng(2)
    for n, card in ((1, 1), (1000, 3), (2_000_003, 10_000), (300_000, 300_000)):
        vocab = rng.integers(0, 2**32, card, dtype=np.uint64).astype(np.uint32)
        keys = vocab[np.minimum(rng.zipf(1.1, n) - 1, card - 1)]
        got, d = cb.perfect_hash(keys)
        exp, de = O.perfect_hash(keys)
        assert d == de and np.array_equal(got, exp), (n, card)


@pytest.mark.parametrize("n,card", [(1, 1), (7, 1), (5000, 5000), (100_000, 40), (1_000_003, 10_000)])
def test_ctr_columns_match_oracle(n, card):
    rng = np.random.default_rng(n)
    raw = np.minimum(rng.zipf(1.1, n) - 1, card - 1).astype(np.uint32) if card < n else rng.permutation(n).astype(np.uint32)
    bucket, nb = O.perfect_hash(raw)
    perm = O.shuffled_indices(n, 11)
    cls = (rng.random(n) < 0.35).astype(np.uint8)
    bins, vals, cnt = cb.ctr_columns(bucket, perm, cls, SPECS, want_values=True, want_counts=True)
    eb, ev = _oracle_cols(bucket, perm, cls, SPECS)
    assert np.array_equal(bins, eb)
    assert np.array_equal(vals.view(np.uint64), ev.view(np.uint64))
    r = O.ctr_column("Buckets", bucket, perm, cls, prior=0.0, target_border_idx=0)
    assert np.array_equal(cnt[0], r["good"].astype(np.uint32))
    assert np.array_equal(cnt[0] + cnt[1], r["total"].astype(np.uint32))


def test_ctr_columns_hand_scenario_and_bins_at_31_borders():
    bins, vals = cb.ctr_columns(np.zeros(4, np.uint32), np.arange(4), [1, 0, 1, 1], [("Borders", 0.5)],
                                want_values=True)
    assert vals[0].tolist() == [0.5, 0.75, 0.5, 0.625] and bins[0].tolist() == [7, 11, 7, 9]
    rng = np.random.default_rng(4)
    n = 50_000
    bucket, _ = O.perfect_hash(rng.integers(0, 600, n).astype(np.uint32))
    perm = O.shuffled_indices(n, 1)
    cls = (rng.random(n) < 0.5).astype(np.uint8)
    got = cb.ctr_columns(bucket, perm, cls, SPECS, border_count=31)
    eb, _ = _oracle_cols(bucket, perm, cls, SPECS, bc=31)
    assert np.array_equal(got, eb)
