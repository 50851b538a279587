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
