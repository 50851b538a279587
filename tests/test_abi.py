"""CPU-side checks of the C-ABI library: it loads, and it exports every function the
public headers declare (no compute call is made -- there is no GPU here)."""
import os
import re
import subprocess

import pytest

import catboost_rs_amd as cb

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    names = set()
    for h in ("cbhip.h", "cbtrain.h"):
        src = open(os.path.join(ROOT, "include", h)).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b(cb[ht]_\w+)\s*\(", src, re.M):
            names.add(m.group(1))
    return names


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(cb.LIB_PATH):
        pytest.fail("libcbhip.so is not built (run __graft_entry__.build())")
    return cb.load()


def test_library_loads(lib):
    assert lib.cbh_version().decode().startswith("cbhip")


def test_every_declared_symbol_is_exported(lib):
    declared = _declared_functions()
    assert declared, "no declarations parsed"
    assert declared == set(cb.EXPORTS), (declared ^ set(cb.EXPORTS))
    out = subprocess.run(["nm", "-D", "--defined-only", cb.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if l.strip()}
    missing = declared - exported
    assert not missing, f"declared but not exported: {sorted(missing)}"


def test_library_is_gfx950_only():
    out = subprocess.run(["strings", "-n", "8", cb.LIB_PATH], capture_output=True, text=True).stdout
    assert "gfx950" in out
    assert "gfx942" not in out and "gfx90a" not in out


def test_errors_without_device_are_reported_not_faulting(lib):
    """With no GPU, opening a session must fail with a status code, never crash."""
    import ctypes as C
    import numpy as np
    if os.environ.get("HIP_VISIBLE_DEVICES") is None and os.path.exists("/dev/kfd"):
        pytest.skip("a GPU may be present; this check is for GPU-less hosts")
    bins = np.zeros((2, 8), np.uint8)
    cfg = cb.Config(loss=0, score_function=0, leaf_method=0, depth=2, boosting_type_is_plain=1,
                    fold_count=1, approx_dim=1)
    s = C.c_void_p()
    rc = lib.cbh_session_begin_u8(C.byref(cfg), bins.ctypes.data_as(C.c_void_p), None, 8, 2, 4,
                                  0.1, 3.0, C.byref(s))
    assert rc != 0


def test_config_decline_paths(lib):
    """Uncovered configs decline (status 1) before touching the device, like the reference's
    trait defaults (runtime.rs:1497-1529); invalid shapes are typed errors."""
    import ctypes as C
    import numpy as np
    bins = np.zeros((2, 8), np.uint8)
    s = C.c_void_p()

    def begin(**kw):
        base = dict(loss=0, score_function=0, leaf_method=0, depth=2, boosting_type_is_plain=1,
                    fold_count=1, approx_dim=1)
        base.update(kw)
        cfg = cb.Config(**base)
        return lib.cbh_session_begin_u8(C.byref(cfg), bins.ctypes.data_as(C.c_void_p), None, 8, 2, 4,
                                        0.1, 3.0, C.byref(s))

    assert begin(boosting_type_is_plain=0) == cb.DECLINED
    assert begin(fold_count=2) == cb.DECLINED
    assert begin(depth=9) == cb.DECLINED
    assert begin(loss=2, approx_dim=3, leaf_method=0) == cb.DECLINED  # MultiClass needs Newton
    assert begin(approx_dim=2) == -5
    bad = np.full((2, 8), 7, np.uint8)
    cfg = cb.Config(loss=0, score_function=0, leaf_method=0, depth=2, boosting_type_is_plain=1,
                    fold_count=1, approx_dim=1)
    rc = lib.cbh_session_begin_u8(C.byref(cfg), bad.ctypes.data_as(C.c_void_p), None, 8, 2, 4, 0.1,
                                  3.0, C.byref(s))
    assert rc == -2  # bin >= n_bins -> OutOfRange


def test_one_hot_with_bootstrap_is_refused(lib):
    """The caller side refuses one-hot columns with active RNG draws (boosting.rs:5744-5756)
    before any device call."""
    import numpy as np
    bins = np.zeros((2, 8), np.uint8)
    bins[1, ::2] = 1
    with pytest.raises(cb.CbhError) as e:
        cb.Trainer(bins, 2, np.zeros(8), loss="RMSE", depth=2, bootstrap_type="Bernoulli",
                   one_hot_flags=np.array([0, 1], np.uint8), real_folds=np.array([2, 2], np.uint32))
    assert e.value.code == -4


def test_float_preparation_argument_checks(lib):
    """Border selection, quantization and the raw float channel validate their arguments
    before any device call (typed errors, no fault)."""
    import numpy as np
    col = np.array([[0.0, 1.0, 2.0, 3.0]], np.float32)
    for kw, code in ((dict(border_count=0), -2), (dict(border_count=255, nan_mode="Max"), -2),
                     (dict(border_count=256), -2)):
        with pytest.raises(cb.CbhError) as e:
            cb.select_borders(col, **kw)
        assert e.value.code == code
    with pytest.raises(KeyError):
        cb.select_borders(col, border_type="Median")
    with pytest.raises(cb.CbhError) as e:
        cb.quantize(col[0], np.array([2.0, 1.0]))
    assert e.value.code == -2
    with pytest.raises(cb.CbhError) as e:
        cb.quantize(col[0], np.arange(256.0))
    assert e.value.code == -2

    def raw(borders, n_bins=4, **cfg_kw):
        be = cb.HipBackend()
        return be.begin_device_training_raw("RMSE", 2, True, 1, "Cosine", col, borders, None, 4, 1,
                                            n_bins, 0.1, 3.0, **cfg_kw)

    with pytest.raises(cb.CbhError) as e:
        raw([np.array([1.0, 0.5])])
    assert e.value.code == -2  # borders must ascend
    with pytest.raises(cb.CbhError) as e:
        raw([np.array([0.5, 1.5, 2.5, 3.5])])
    assert e.value.code == -2  # n_borders + 1 > n_bins


@pytest.mark.parametrize("n,F", [(1, 1), (63, 3), (1000, 50), (131_073, 17), (300_001, 50)])
def test_columns_from_rows_is_the_transpose(lib, n, F):
    """The row-major ingest (host code, no device) gives every column of the matrix, bit for
    bit: single- and multi-threaded splits, runs of rows not a multiple of the 64-row block."""
    import numpy as np
    x = np.random.default_rng(n + F).standard_normal((n, F)).astype(np.float32)
    x[::7, F // 2] = np.nan
    got = cb.columns_from_rows(x)
    assert got.shape == (F, n)
    assert np.array_equal(got.view(np.uint32), np.ascontiguousarray(x.T).view(np.uint32))


def test_categorical_argument_checks(lib):
    """CTR columns validate the permutation, bucket range and classes before any device call."""
    import numpy as np
    for args, kw in (((np.zeros(3, np.uint32), np.array([0, 0, 1]), np.zeros(3)), {}),
                     ((np.array([0, 5, 1], np.uint32), np.arange(3), np.zeros(3)), dict(n_buckets=2)),
                     ((np.zeros(3, np.uint32), np.arange(3), np.array([0, 2, 1])), {})):
        with pytest.raises(cb.CbhError) as e:
            cb.ctr_columns(*args, [("Borders", 0.5)], **kw)
        assert e.value.code == -2
    with pytest.raises(cb.CbhError) as e:
        cb.ctr_columns(np.zeros(3, np.uint32), np.arange(3), np.zeros(3), [("Borders", 0.5)] * 17)
    assert e.value.code == -2


def test_multiclass_dimensions_without_a_variant_decline(lib):
    """MultiClass dimensions with no compiled kernel variant, and leaf systems larger than one
    workgroup's LDS, decline to the CPU grower (status 1) instead of failing on the device."""
    import ctypes as C
    import numpy as np
    bins = np.zeros((2, 8), np.uint8)
    s = C.c_void_p()
    for k, depth in ((9, 6), (11, 6), (13, 4), (15, 2), (12, 8), (16, 8)):
        cfg = cb.Config(loss=2, score_function=0, leaf_method=1, depth=depth, boosting_type_is_plain=1,
                        fold_count=1, approx_dim=k)
        rc = lib.cbh_session_begin_u8(C.byref(cfg), bins.ctypes.data_as(C.c_void_p), None, 8, 2, 4,
                                      0.1, 3.0, C.byref(s))
        assert rc == cb.DECLINED, (k, depth, rc)


def test_device_ctr_config_admission(lib):
    """The device CTR config declines what ctr_covered declines (gpu_runtime/session.rs:177-215)
    and rejects malformed inputs with typed errors, all before any device call."""
    import ctypes as C
    import numpy as np
    n = 8
    bins = np.zeros((2, n), np.uint8)
    cat = np.array([[0, 1, 0, 2, 1, 0, 2, 2]], np.uint32)
    perm = np.arange(n)[::-1]
    cls = np.array([0, 1, 1, 0, 1, 0, 0, 1])

    def begin(dc, loss="RMSE", n_bins=16):
        be = cb.HipBackend()
        try:
            return be.begin_device_training(loss, 2, True, 1, "Cosine", bins, None, n, 2, n_bins, 0.1, 3.0,
                                            ctr=dc)
        finally:
            be.end_device_training()

    def make(**kw):
        return cb.DeviceCtr(cat, kw.pop("perm", perm), kw.pop("avg", perm), kw.pop("cls", cls),
                            kw.pop("specs", [("Borders", 0.5)]), **kw)

    dc = make()
    dc.config.averaging = None
    assert begin(dc) is False                                   # no averaging half
    assert begin(make(), loss="PairLogit") is False             # pair loss
    assert begin(make(border_count=15), n_bins=8) is False      # border table longer than n_bins - 1
    dc = make()
    dc.columns[0].ctr_type = 3                                  # FloatTargetMeanValue
    assert begin(dc) is False
    dc = make()
    dc.columns[0].n_members = 2                                 # a combination projection
    assert begin(dc) is False
    for mutate, code in ((lambda d: setattr(d.columns[0], "target_border_idx", 2), -2),
                         (lambda d: setattr(d.columns[0], "weight_group", 1), -2),
                         (lambda d: setattr(d.columns[0], "borders", None), -5)):
        dc = make()
        mutate(dc)
        with pytest.raises(cb.CbhError) as e:
            begin(dc)
        assert e.value.code == code
    for kw in (dict(perm=np.zeros(n, np.uint32)), dict(avg=np.array([0] * n)), dict(cls=np.full(n, 2))):
        with pytest.raises(cb.CbhError) as e:
            begin(make(**kw))
        assert e.value.code == -2


def test_ctr_border_table_reproduces_the_oracle_binarization():
    """The border table the caller builds (next_down of the bin edges, boosting.rs:3620-3627)
    binarizes every CTR value the oracle produces to the oracle's own bin for the default
    priors 0, 0.5 and 1: values from skewed buckets and random classes cover tens of thousands
    of (count, total) pairs.  With other priors the table (the reference's device
    binarization, binarize_ctr_kernel) and the oracle's truncation formula (its CPU path) can
    round apart, by one bin, and only for a value that sits exactly on a bin edge -- checked
    in exact rational arithmetic."""
    from fractions import Fraction as Fr

    import numpy as np
    from oracle import oracle as O
    rng = np.random.default_rng(11)
    n = 60_000
    bucket = np.minimum(rng.zipf(1.3, n) - 1, 400).astype(np.uint32)
    bucket, _ = O.perfect_hash(bucket)
    perm = O.shuffled_indices(n, 3)
    cls = (rng.random(n) < 0.4).astype(np.uint8)
    edges_seen = 0
    for kind, tbi in (("Borders", 0), ("Buckets", 0), ("Buckets", 1), ("BinarizedTargetMeanValue", 0),
                      ("Counter", 0)):
        for prior in (0.0, 0.5, 1.0, 2.5, -0.75):
            for bc in (1, 15, 31, 255):
                col = O.ctr_column(kind, bucket, perm, cls, prior=prior, target_border_idx=tbi, border_count=bc)
                table = cb.ctr_borders(prior, bc)
                got = (col["value"][:, None] > table[None, :]).sum(1)
                bad = np.nonzero(got != col["bin"])[0]
                if prior in (0.0, 0.5, 1.0):
                    assert bad.size == 0, (kind, tbi, prior, bc)
                    continue
                pr = Fr(prior)
                shift, norm = -min(Fr(0), pr), max(Fr(1), pr) - min(Fr(0), pr)
                for i in bad:
                    x = (Fr(int(col["good"][i])) + pr) / (Fr(int(col["total"][i])) + 1)
                    assert ((x + shift) / norm * bc).denominator == 1, (kind, prior, bc, i)
                    assert abs(int(got[i]) - int(col["bin"][i])) == 1
                edges_seen += bad.size
    assert edges_seen > 0   # the exact-edge case occurs in this sample
