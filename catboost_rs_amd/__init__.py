"""MI355X (gfx950) oblivious-tree training path of catboost_rs, behind its compute seam.

The product is the shared library ``libcbhip.so`` (HIP kernels + C-ABI, ``include/cbhip.h``)
and the host mirror of cb-train's device branch (``include/cbtrain.h``).  This module is a
thin ctypes front-end used by the tests and ``bench.py``:

* :class:`HipBackend` mirrors ``trait cb_compute::Runtime``'s device-training methods
  (crates/cb-compute/src/runtime.rs:1431-1651): ``compute_gradients``,
  ``begin_device_training``, ``grow_tree_on_device``, ``end_device_training``.
* :class:`Trainer` drives the boosting loop exactly like cb-train's device branch
  (crates/cb-train/src/boosting.rs:6532-7300) through ``cbt_*``.

There is no CPU fallback: if the library is missing or no GPU is present, calls raise.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcbhip.so")

LOSS = {"RMSE": 0, "Logloss": 1, "MultiClass": 2, "CrossEntropy": 3, "PairLogit": 4,
        "PairLogitPairwise": 5}
SCORE = {"Cosine": 0, "L2": 1, "SolarL2": 2, "LOOL2": 3, "SatL2": 4}
LEAF = {"Gradient": 0, "Newton": 1, "Simple": 2}
BOOT = {"No": 0, "Bayesian": 1, "Bernoulli": 2}

OK, DECLINED = 0, 1
ERRORS = {-1: "LengthMismatch", -2: "OutOfRange", -3: "Degenerate", -4: "Unsupported",
          -5: "InvalidArgument", -6: "Device"}


class CbhError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{ERRORS.get(code, code)}: {msg}")
        self.code = code


class Config(C.Structure):
    _fields_ = [("loss", C.c_int32), ("score_function", C.c_int32), ("leaf_method", C.c_int32),
                ("depth", C.c_int32), ("boosting_type_is_plain", C.c_int32),
                ("fold_count", C.c_int32), ("approx_dim", C.c_int32),
                ("bootstrap_type", C.c_int32), ("sample_from_host", C.c_int32),
                ("sample_rate", C.c_float), ("bagging_temperature", C.c_float),
                ("profile", C.c_int32), ("bias", C.c_double), ("rng_seed", C.c_uint64),
                ("one_hot_flags", C.c_void_p), ("real_folds", C.c_void_p),
                ("pairwise_non_diag_reg", C.c_double), ("ctr", C.c_void_p)]


class Family(C.Structure):
    """FamilyTreeArgs::Pairwise / ::MultiOutput (runtime.rs:925-950)."""
    _fields_ = [("kind", C.c_int32), ("n_groups", C.c_uint32), ("group_offsets", C.c_void_p),
                ("pair_winner", C.c_void_p), ("pair_loser", C.c_void_p), ("pair_weight", C.c_void_p),
                ("n_pairs", C.c_uint64), ("approx_k", C.c_void_p), ("approx_dim", C.c_uint32)]


class TreeSampling(C.Structure):
    _fields_ = [("kind", C.c_int32), ("bagging_temperature", C.c_float), ("subsample", C.c_double),
                ("bayesian_seed", C.c_uint64), ("bernoulli_state", C.c_uint64 * 4)]


class TreeOut(C.Structure):
    _fields_ = [("split_feature", C.c_void_p), ("split_bin", C.c_void_p),
                ("split_one_hot", C.c_void_p), ("leaf_values", C.c_void_p),
                ("leaf_of", C.c_void_p), ("split_score", C.c_void_p)]


class Stats(C.Structure):
    _fields_ = [("fill_ms", C.c_double), ("derive_ms", C.c_double), ("score_ms", C.c_double),
                ("partition_ms", C.c_double), ("leaf_ms", C.c_double), ("prepare_ms", C.c_double),
                ("total_ms", C.c_double), ("fill_launches", C.c_uint64), ("fill_rows", C.c_uint64),
                ("fill_row_features", C.c_uint64), ("fill_bytes", C.c_double), ("trees", C.c_uint64),
                ("skip_features", C.c_uint64), ("quantize_ms", C.c_double),
                ("quantize_launches", C.c_uint64), ("quantize_bytes", C.c_double),
                ("fill_mode", C.c_uint32), ("fill_pack_bits", C.c_int32), ("score_shift_der", C.c_int32),
                ("score_shift_w", C.c_int32), ("fill_entries", C.c_uint64),
                ("fill_lane_atomics", C.c_uint64)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}


class CtrInfo(C.Structure):
    _fields_ = [("n_ctr", C.c_uint32), ("averaging_bins", C.c_void_p), ("bucket_count", C.c_void_p),
                ("weight_group", C.c_void_p), ("n_cat", C.c_uint32), ("cat_buckets", C.c_void_p),
                ("cat_bucket_count", C.c_void_p), ("model_size_reg", C.c_double)]


class DeviceCtrColumn(C.Structure):
    """DeviceCtrColumn (runtime.rs:1104-1160)."""
    _fields_ = [("n_members", C.c_uint32), ("member_bins", C.c_void_p), ("prior", C.c_double),
                ("borders", C.c_void_p), ("n_borders", C.c_uint32), ("bucket_count", C.c_uint64),
                ("weight_group", C.c_uint32), ("ctr_type", C.c_int32), ("target_border_idx", C.c_uint32),
                ("projection_members", C.c_void_p), ("n_projection_members", C.c_uint32)]


class DeviceCtrAveraging(C.Structure):
    """DeviceCtrAveraging (runtime.rs:1212-1224)."""
    _fields_ = [("permutation", C.c_void_p), ("target_class", C.c_void_p), ("columns", C.c_void_p),
                ("n_columns", C.c_uint32)]


class DeviceCtrConfig(C.Structure):
    """DeviceCtrConfig (runtime.rs:1174-1200)."""
    _fields_ = [("permutation", C.c_void_p), ("target_class", C.c_void_p), ("columns", C.c_void_p),
                ("n_columns", C.c_uint32), ("averaging", C.c_void_p), ("n_cat", C.c_uint32),
                ("cat_eligible_buckets", C.c_void_p), ("model_size_reg", C.c_double)]


class TrainParams(C.Structure):
    _fields_ = [("loss", C.c_int32), ("score_function", C.c_int32), ("leaf_method", C.c_int32),
                ("depth", C.c_int32), ("bootstrap_type", C.c_int32),
                ("boost_from_average", C.c_int32), ("approx_dim", C.c_int32), ("profile", C.c_int32),
                ("learning_rate", C.c_double), ("l2_leaf_reg", C.c_double), ("subsample", C.c_double),
                ("bagging_temperature", C.c_float), ("pad_", C.c_float), ("random_seed", C.c_uint64),
                ("pairwise_non_diag_reg", C.c_double)]


# Every symbol include/cbhip.h and include/cbtrain.h declare (the ABI test checks them).
EXPORTS = ["cbh_session_begin", "cbh_session_begin_u8", "cbh_session_grow",
           "cbh_session_read_approx", "cbh_session_stats", "cbh_session_reset_stats",
           "cbh_session_end", "cbh_compute_gradients", "cbh_hist_build", "cbh_bootstrap",
           "cbh_apply_oblivious", "cbh_session_begin_raw", "cbh_select_borders", "cbh_quantize", "cbh_perfect_hash", "cbh_ctr_columns", "cbh_shuffled_indices",
           "cbh_version", "cbh_last_error", "cbt_open", "cbt_open_raw", "cbt_set_pairs", "cbt_step",
           "cbt_read_approx", "cbt_stats", "cbt_reset_stats", "cbt_bias", "cbt_close", "cbh_session_set_profile",
           "cbt_set_profile", "cbh_session_set_ctr", "cbt_set_ctr", "cbh_session_read_ctr_bins",
           "cbt_open_ctr", "cbh_hist_build_noalloc", "cbh_session_capture_hists", "cbh_session_level_hist",
           "cbh_columns_from_rows"]

_lib = None


def load(path: str = LIB_PATH):
    """Load libcbhip.so; raises if it was not built (there is no fallback path)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is missing: run `python -m catboost_rs_amd.build`")
    L = C.CDLL(path)
    P = C.c_void_p
    L.cbh_last_error.restype = C.c_char_p
    L.cbh_version.restype = C.c_char_p
    L.cbh_session_begin.argtypes = [C.POINTER(Config), P, P, C.c_uint64, C.c_uint32, C.c_uint32,
                                    C.c_double, C.c_double, C.POINTER(P)]
    L.cbh_session_begin_u8.argtypes = L.cbh_session_begin.argtypes
    L.cbh_session_grow.argtypes = [P, P, P, C.c_uint64, P, C.c_uint64, C.POINTER(TreeSampling),
                                   C.POINTER(Family), C.POINTER(TreeOut)]
    L.cbh_session_read_approx.argtypes = [P, P, C.c_uint64]
    L.cbh_session_stats.argtypes = [P, C.POINTER(Stats)]
    L.cbh_session_reset_stats.argtypes = [P]
    L.cbh_session_reset_stats.restype = None
    L.cbh_session_end.argtypes = [P]
    L.cbh_compute_gradients.argtypes = [C.c_int32, P, P, C.c_uint64, C.c_uint32, P, P]
    L.cbh_hist_build.argtypes = [P, C.c_uint64, C.c_uint32, C.c_uint32, P, P, C.c_uint32, P,
                                 C.c_uint32, P]
    L.cbh_bootstrap.argtypes = [C.POINTER(TreeSampling), C.c_uint64, P, P]
    L.cbh_hist_build_noalloc.argtypes = [P, C.c_uint64, C.c_uint32, C.c_uint32, P, P, C.c_uint32, P, P]
    L.cbt_open.argtypes = [C.POINTER(TrainParams), P, C.c_uint64, C.c_uint32, C.c_uint32, P, P, P,
                           P, C.POINTER(P)]
    L.cbh_apply_oblivious.argtypes = [P, C.c_uint64, C.c_uint32, P, P, P, P, P, C.c_uint32, C.c_uint32,
                                      P, P, P]
    L.cbh_session_begin_raw.argtypes = [C.POINTER(Config), P, P, P, P, C.c_uint64, C.c_uint32, C.c_uint32,
                                        C.c_double, C.c_double, C.POINTER(P)]
    L.cbh_select_borders.argtypes = [P, C.c_uint64, C.c_uint32, C.c_uint32, C.c_int32, C.c_int32, P, P]
    L.cbh_columns_from_rows.argtypes = [P, C.c_uint64, C.c_uint32, P]
    L.cbh_quantize.argtypes = [P, C.c_uint64, P, C.c_uint32, P]
    L.cbh_perfect_hash.argtypes = [P, C.c_uint64, P, P]
    L.cbh_shuffled_indices.argtypes = [C.c_uint64, C.c_uint64, C.c_uint32, P]
    L.cbh_ctr_columns.argtypes = [P, C.c_uint32, C.c_uint64, P, P, P, C.c_uint32, C.c_uint32, P, P, P]
    L.cbt_open_raw.argtypes = [C.POINTER(TrainParams), P, P, P, C.c_uint64, C.c_uint32, P, P, C.POINTER(P)]
    L.cbt_set_pairs.argtypes = [P, P, C.c_uint32, P, P, P, C.c_uint64]
    L.cbt_step.argtypes = [P, P, P, P, P]
    L.cbt_read_approx.argtypes = [P, P]
    L.cbt_stats.argtypes = [P, C.POINTER(Stats)]
    L.cbt_reset_stats.argtypes = [P]
    L.cbt_reset_stats.restype = None
    L.cbt_bias.argtypes = [P]
    L.cbt_bias.restype = C.c_double
    L.cbh_session_set_profile.argtypes = [P, C.c_int32]
    L.cbh_session_capture_hists.argtypes = [P, C.c_int32]
    L.cbh_session_level_hist.argtypes = [P, C.c_uint32, P, C.c_uint64]
    L.cbh_session_set_ctr.argtypes = [P, C.POINTER(CtrInfo)]
    L.cbt_set_ctr.argtypes = [P, C.POINTER(CtrInfo)]
    L.cbt_set_profile.argtypes = [P, C.c_int32]
    L.cbh_session_read_ctr_bins.argtypes = [P, C.c_int32, P, C.c_uint64]
    L.cbt_open_ctr.argtypes = [C.POINTER(TrainParams), P, C.c_uint64, C.c_uint32, C.c_uint32, P, P,
                               C.POINTER(DeviceCtrConfig), P, P, C.POINTER(P)]
    L.cbt_close.argtypes = [P]
    L.cbt_close.restype = None
    _lib = L
    return L


def _check(rc: int):
    if rc != OK:
        raise CbhError(rc, load().cbh_last_error().decode())


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------------------------------
# kernel-level entry points
# ---------------------------------------------------------------------------------------
def compute_gradients(loss: str, approx: np.ndarray, target: np.ndarray, approx_dim: int = 1):
    """Runtime::compute_gradients (runtime.rs:1431): dim-major der1/der2 on the GPU."""
    a = np.ascontiguousarray(approx, np.float64).reshape(-1)
    t = np.ascontiguousarray(target, np.float64)
    n = t.shape[0]
    d1 = np.empty(n * approx_dim)
    pk = approx_dim * (approx_dim + 1) // 2 if loss == "MultiClass" else 1
    d2 = np.empty(n * pk)
    _check(load().cbh_compute_gradients(LOSS[loss], _ptr(a), _ptr(t), n, approx_dim, _ptr(d1), _ptr(d2)))
    return d1, d2


def hist_build(bins_fm, n_bins, der, w, slot_of_row=None, n_slots=1):
    """One histogram fill on the GPU; exact sums returned as f64 [slot][F][bin][K+1]."""
    bins_fm = np.ascontiguousarray(bins_fm, np.uint8)
    F, n = bins_fm.shape
    der = np.ascontiguousarray(der, np.float64)
    K = 1 if der.ndim == 1 else der.shape[0]
    w = np.ascontiguousarray(w, np.float64)
    slot = None if slot_of_row is None else np.ascontiguousarray(slot_of_row, np.uint32)
    out = np.empty((n_slots, F, n_bins, K + 1), np.float64)
    _check(load().cbh_hist_build(_ptr(bins_fm), n, F, n_bins, _ptr(der), _ptr(w), K, _ptr(slot),
                                 n_slots, _ptr(out)))
    return out


def bootstrap(kind: str, n: int, *, bayesian_seed=0, bernoulli_state=(0, 1, 0, 1), subsample=1.0,
              temperature=1.0):
    s = TreeSampling(kind=BOOT[kind], bagging_temperature=temperature, subsample=subsample,
                     bayesian_seed=bayesian_seed)
    for i, v in enumerate(bernoulli_state):
        s.bernoulli_state[i] = v
    sw = np.empty(n)
    ctrl = np.empty(n, np.uint8)
    _check(load().cbh_bootstrap(C.byref(s), n, _ptr(sw), _ptr(ctrl)))
    return sw, ctrl.astype(bool)


# ---------------------------------------------------------------------------------------
# The Runtime seam (begin / grow / end)
# ---------------------------------------------------------------------------------------
def apply_oblivious(features_fm, split_features, split_borders, tree_split_offsets, leaf_values,
                    tree_leaf_offsets, approx_dim=1, bias=None, nan_as_true=None):
    """Raw predictions [approx_dim][n] of an oblivious float ensemble on the device
    (``cbh_apply_oblivious``); features_fm is f32 [F][n], model arrays are flat CSR."""
    x = np.ascontiguousarray(features_fm, np.float32)
    F, n = x.shape
    sf = np.ascontiguousarray(split_features, np.uint32)
    sb = np.ascontiguousarray(split_borders, np.float64)
    so = np.ascontiguousarray(tree_split_offsets, np.uint32)
    lv = np.ascontiguousarray(leaf_values, np.float64)
    lo = np.ascontiguousarray(tree_leaf_offsets, np.uint32)
    b = None if bias is None else np.ascontiguousarray(np.broadcast_to(bias, (approx_dim,)), np.float64)
    na = None if nan_as_true is None else np.ascontiguousarray(nan_as_true, np.uint8)
    out = np.zeros((approx_dim, n))
    _check(load().cbh_apply_oblivious(_ptr(x), n, F, _ptr(sf), _ptr(sb), _ptr(so), _ptr(lv), _ptr(lo),
                                      so.shape[0] - 1, approx_dim, _ptr(b), _ptr(na), _ptr(out)))
    return out


BORDER_TYPE = {"GreedyLogSum": 0, "GreedyMinEntropy": 1}
NAN_MODE = {"Min": 0, "Max": 1, "Forbidden": 2}


def _column_ptrs(columns):
    """f32 feature-major matrix [F][n] -> (kept array, C array of F column pointers)."""
    x = np.ascontiguousarray(columns, np.float32)
    if x.ndim != 2:
        raise ValueError("columns must be a [n_features][n] matrix")
    ptrs = (C.c_void_p * max(x.shape[0], 1))()
    for f in range(x.shape[0]):
        ptrs[f] = x.ctypes.data + f * x.strides[0]
    return x, ptrs


def _border_ptrs(borders):
    bs = [np.ascontiguousarray(b, np.float64) for b in borders]
    ptrs = (C.c_void_p * max(len(bs), 1))()
    for f, b in enumerate(bs):
        ptrs[f] = b.ctypes.data if b.size else None
    nb = np.array([b.size for b in bs], np.uint32)
    return bs, ptrs, nb


def columns_from_rows(rows):
    """Per-feature f32 columns [F][n] of a row-major (n, F) matrix (``cbh_columns_from_rows``,
    a threaded host copy)."""
    x = np.ascontiguousarray(rows, np.float32)
    if x.ndim != 2:
        raise ValueError("rows must be an (n_rows, n_features) matrix")
    n, F = x.shape
    out = np.empty((F, n), np.float32)
    _check(load().cbh_columns_from_rows(_ptr(x), n, F, _ptr(out)))
    return out


def select_borders(columns, border_count=254, nan_mode="Min", border_type="GreedyLogSum"):
    """Greedy border sets of f32 columns [F][n] (``cbh_select_borders``): a list of F
    ascending f64 arrays, sentinels of ``nan_mode`` included for NaN-bearing columns."""
    x, ptrs = _column_ptrs(columns)
    F, n = x.shape
    out = np.zeros((F, border_count + 1))
    cnt = np.zeros(F, np.uint32)
    _check(load().cbh_select_borders(ptrs, n, F, border_count, NAN_MODE[nan_mode],
                                     BORDER_TYPE[border_type], _ptr(out), _ptr(cnt)))
    return [out[f, :cnt[f]].copy() for f in range(F)]


def quantize(column, borders):
    """u8 bins of one f32 column over ascending borders (``cbh_quantize``)."""
    c = np.ascontiguousarray(column, np.float32)
    b = np.ascontiguousarray(borders, np.float64)
    out = np.zeros(c.shape[0], np.uint8)
    _check(load().cbh_quantize(_ptr(c), c.shape[0], _ptr(b) if b.size else None, b.size, _ptr(out)))
    return out


CTR_TYPE = {"Borders": 0, "Buckets": 1, "BinarizedTargetMeanValue": 2, "Counter": 4}


class CtrSpec(C.Structure):
    _fields_ = [("ctr_type", C.c_int32), ("target_border_idx", C.c_uint32), ("prior_num", C.c_double),
                ("prior_denom", C.c_double)]


def shuffled_indices(n, seed, count=1):
    """Learn permutations [count][n] (``cbh_shuffled_indices``, host)."""
    out = np.zeros((count, n), np.uint32)
    _check(load().cbh_shuffled_indices(n, seed, count, _ptr(out)))
    return out[0] if count == 1 else out


def perfect_hash(keys):
    """First-seen dense bins of u32 keys on the device (``cbh_perfect_hash``)."""
    k = np.ascontiguousarray(keys, np.uint32)
    out = np.zeros(k.shape[0], np.uint32)
    d = C.c_uint32()
    _check(load().cbh_perfect_hash(_ptr(k), k.shape[0], _ptr(out), C.byref(d)))
    return out, int(d.value)


def ctr_columns(buckets, permutation, target_class, specs, border_count=15, n_buckets=None,
                want_values=False, want_counts=False):
    """Online CTR columns of one categorical feature on the device (``cbh_ctr_columns``).
    ``specs``: list of (ctr_type, prior) or (ctr_type, prior, target_border_idx).  Returns
    bins [n_specs][n] u8 (and values [n_specs][n], counts [2][n] when asked)."""
    b = np.ascontiguousarray(buckets, np.uint32)
    pm = np.ascontiguousarray(permutation, np.uint32)
    tc = np.ascontiguousarray(target_class, np.uint8)
    n = b.shape[0]
    nb = (int(b.max()) + 1 if n else 1) if n_buckets is None else int(n_buckets)
    arr = (CtrSpec * len(specs))()
    for k, sp in enumerate(specs):
        arr[k] = CtrSpec(CTR_TYPE[sp[0]], sp[2] if len(sp) > 2 else 0, float(sp[1]), 1.0)
    bins = np.zeros((len(specs), n), np.uint8)
    vals = np.zeros((len(specs), n)) if want_values else None
    cnt = np.zeros((2, n), np.uint32) if want_counts else None
    _check(load().cbh_ctr_columns(_ptr(b), nb, n, _ptr(pm), _ptr(tc), arr, len(specs), border_count,
                                  _ptr(bins), _ptr(vals), _ptr(cnt)))
    out = [bins]
    if want_values:
        out.append(vals)
    if want_counts:
        out.append(cnt)
    return out[0] if len(out) == 1 else tuple(out)


def ctr_bin_columns(cat_keys, permutation, target_class, specs=(("Borders", 0.5),), border_count=15):
    """CTR bin columns of every categorical column [n_cat][n] (category keys) on the device:
    first-seen buckets, then the online CTR of each spec over the learn permutation.
    Returns (bins [n_cat * n_specs][n] u8, feature-major in (column, spec) order, and the
    bucket count of each column)."""
    keys = np.ascontiguousarray(cat_keys, np.uint32)
    out, counts = [], []
    for j in range(keys.shape[0]):
        bucket, d = perfect_hash(keys[j])
        out.append(ctr_columns(bucket, permutation, target_class, list(specs), border_count=border_count,
                               n_buckets=d))
        counts.append(d)
    return np.concatenate(out, 0), np.array(counts, np.int64)


def ctr_borders(prior, border_count=15):
    """Border table of a CTR column as build_device_ctr_config makes it (boosting.rs:3620-3627):
    next_down((k + 1) * norm / border_count - shift), shift/norm = calc_normalization(prior)."""
    left, right = min(0.0, float(prior)), max(1.0, float(prior))
    shift, norm = -left, right - left
    k = np.arange(border_count, dtype=np.float64)
    return np.nextafter((k + 1.0) * norm / border_count - shift, -np.inf)


class DeviceCtr:
    """A DeviceCtrConfig (``cbh_device_ctr_config``) and the host arrays it points into.

    Built as cb-train's build_device_ctr_config does (boosting.rs:3590-3707) for simple
    projections: one column per (categorical column, spec) in that order, each spec
    (ctr_type, prior[, target_border_idx]); the border table of ``ctr_borders``; one weight
    group per (ctr type, categorical column); the averaging half the same specs under the
    averaging permutation.  ``cat_buckets`` [n_cat][n] are the first-seen buckets of the
    CTR-eligible columns, which are also their member bins."""

    def __init__(self, cat_buckets, permutation, averaging_permutation, target_class, specs,
                 border_count=15, bucket_counts=None, model_size_reg=0.5):
        cat = np.ascontiguousarray(cat_buckets, np.uint32)
        n_cat, n = cat.shape
        if bucket_counts is None:
            bucket_counts = [int(c.max()) + 1 if n else 0 for c in cat]
        keep = [cat]
        self.perm = np.ascontiguousarray(permutation, np.uint32)
        self.avg_perm = np.ascontiguousarray(averaging_permutation, np.uint32)
        self.cls = np.ascontiguousarray(target_class, np.uint32)
        keep += [self.perm, self.avg_perm, self.cls]
        member_ptrs = [(C.c_void_p * 1)(cat[j].ctypes.data) for j in range(n_cat)]
        proj = [np.array([j], np.uint32) for j in range(n_cat)]
        keep += [member_ptrs, proj]
        groups = {}
        specs = [tuple(sp) for sp in specs]
        m = n_cat * len(specs)
        cols = (DeviceCtrColumn * m)()
        k = 0
        for j in range(n_cat):
            for sp in specs:
                ctype = CTR_TYPE[sp[0]]
                b = ctr_borders(sp[1], border_count)
                keep.append(b)
                g = groups.setdefault((ctype, j), len(groups))
                cols[k] = DeviceCtrColumn(1, C.cast(member_ptrs[j], C.c_void_p), float(sp[1]), _ptr(b),
                                          b.shape[0], int(bucket_counts[j]), g, ctype,
                                          sp[2] if len(sp) > 2 else 0, _ptr(proj[j]), 1)
                k += 1
        self.n_columns = m
        self.columns = cols
        self.averaging = DeviceCtrAveraging(_ptr(self.avg_perm), _ptr(self.cls), C.cast(cols, C.c_void_p), m)
        cat_ptrs = (C.c_void_p * max(n_cat, 1))(*[cat[j].ctypes.data for j in range(n_cat)])
        keep.append(cat_ptrs)
        self.config = DeviceCtrConfig(_ptr(self.perm), _ptr(self.cls), C.cast(cols, C.c_void_p), m,
                                      C.cast(C.pointer(self.averaging), C.c_void_p), n_cat,
                                      C.cast(cat_ptrs, C.c_void_p), float(model_size_reg))
        self._keep = keep

    def ref(self):
        return C.byref(self.config)

    def as_pointer(self):
        return C.cast(C.pointer(self.config), C.c_void_p)


def _family_arrays(group_offsets, winner, loser, weight=None):
    go = np.ascontiguousarray(group_offsets, np.uint32)
    w = np.ascontiguousarray(winner, np.uint32)
    l = np.ascontiguousarray(loser, np.uint32)
    wt = None if weight is None else np.ascontiguousarray(weight, np.float64)
    return go, w, l, wt


def _family(go, w, l, wt):
    return Family(kind=1, n_groups=go.shape[0] - 1, group_offsets=_ptr(go), pair_winner=_ptr(w),
                  pair_loser=_ptr(l), pair_weight=_ptr(wt), n_pairs=w.shape[0])


class HipBackend:
    """Mirror of ``GpuBackend: Runtime`` (crates/cb-backend/src/gpu_backend.rs:196-425)."""

    def __init__(self):
        self._s = C.c_void_p()
        self.n = 0
        self.depth = 0
        self.K = 1

    def compute_gradients(self, loss, approx, target, approx_dimension=1):
        return compute_gradients(loss, approx, target, approx_dimension)

    def begin_device_training(self, loss, depth, boosting_type_is_plain, fold_count, score_function,
                              bins_feature_major, weight, n, n_features, n_bins, learning_rate,
                              scaled_l2, *, approx_dim=1, bias=0.0, leaf_method="Gradient",
                              bootstrap_type="No", sample_from_host=False, profile=False,
                              one_hot_flags=None, real_folds=None, pairwise_non_diag_reg=0.1,
                              ctr=None) -> bool:
        """Returns True when the session opened, False when the config is declined.  ``ctr``: a
        ``DeviceCtr`` (DeviceTrainConfig.ctr); its columns follow the n_features base features."""
        self._keep = [ctr]
        oh = None if one_hot_flags is None else np.ascontiguousarray(one_hot_flags, np.uint8)
        rf = None if real_folds is None else np.ascontiguousarray(real_folds, np.uint32)
        self._keep += [oh, rf]
        cfg = Config(loss=LOSS[loss], score_function=SCORE[score_function], leaf_method=LEAF[leaf_method],
                     depth=depth, boosting_type_is_plain=int(boosting_type_is_plain),
                     fold_count=fold_count, approx_dim=approx_dim, bootstrap_type=BOOT[bootstrap_type],
                     sample_from_host=int(sample_from_host), profile=int(profile), bias=bias,
                     one_hot_flags=_ptr(oh), real_folds=_ptr(rf),
                     pairwise_non_diag_reg=pairwise_non_diag_reg,
                     ctr=None if ctr is None else ctr.as_pointer())
        bins = np.ascontiguousarray(bins_feature_major)
        w = None if weight is None else np.ascontiguousarray(weight, np.float64)
        fn = load().cbh_session_begin_u8 if bins.dtype == np.uint8 else load().cbh_session_begin
        if bins.dtype not in (np.uint8, np.uint32):
            bins = bins.astype(np.uint32)
        rc = fn(C.byref(cfg), _ptr(bins), _ptr(w), n, n_features, n_bins, learning_rate, scaled_l2,
                C.byref(self._s))
        if rc == DECLINED:
            return False
        _check(rc)
        self.n, self.depth, self.K = n, depth, approx_dim
        self.n_ctr = 0 if ctr is None else ctr.n_columns
        return True

    def read_ctr_bins(self, averaging=False):
        """The session's CTR bins [n_ctr][n] of the structure (or averaging) materialization."""
        out = np.zeros((self.n_ctr, self.n), np.uint8)
        _check(load().cbh_session_read_ctr_bins(self._s, int(bool(averaging)), _ptr(out), out.size))
        return out

    def begin_device_training_raw(self, loss, depth, boosting_type_is_plain, fold_count, score_function,
                                  float_columns, feature_borders, weight, n, n_features, n_bins,
                                  learning_rate, scaled_l2, *, approx_dim=1, bias=0.0,
                                  leaf_method="Gradient", bootstrap_type="No", sample_from_host=False,
                                  profile=False, real_folds=None, pairwise_non_diag_reg=0.1) -> bool:
        """Raw float channel (runtime.rs:1546): f32 columns [F][n] + per-feature borders; the
        device quantizes.  Returns True when the session opened, False when declined."""
        rf = None if real_folds is None else np.ascontiguousarray(real_folds, np.uint32)
        x, cp = _column_ptrs(float_columns)
        bs, bp, nb = _border_ptrs(feature_borders)
        w = None if weight is None else np.ascontiguousarray(weight, np.float64)
        self._keep = [rf, x, cp, bs, bp, nb, w]
        cfg = Config(loss=LOSS[loss], score_function=SCORE[score_function], leaf_method=LEAF[leaf_method],
                     depth=depth, boosting_type_is_plain=int(boosting_type_is_plain),
                     fold_count=fold_count, approx_dim=approx_dim, bootstrap_type=BOOT[bootstrap_type],
                     sample_from_host=int(sample_from_host), profile=int(profile), bias=bias,
                     one_hot_flags=None, real_folds=_ptr(rf),
                     pairwise_non_diag_reg=pairwise_non_diag_reg)
        rc = load().cbh_session_begin_raw(C.byref(cfg), cp, bp, _ptr(nb), _ptr(w), n, n_features, n_bins,
                                          learning_rate, scaled_l2, C.byref(self._s))
        if rc == DECLINED:
            return False
        _check(rc)
        self.n, self.depth, self.K = n, depth, approx_dim
        return True

    def grow_tree_on_device(self, approx=None, target=None, sample=None, sampling=None,
                            want_leaf_of=False, family=None):
        """``family`` = (group_offsets, winner, loser[, weight]) for a pair loss (first tree), or
        dict(approx_k=[K][n], approx_dim=K) for FamilyTreeArgs::MultiOutput."""
        d = self.depth
        sf = np.zeros(d, np.uint32)
        sb = np.zeros(d, np.uint32)
        so = np.zeros(d, np.uint8)
        sc = np.zeros(d, np.float64)
        lv = np.zeros((1 << d) * self.K, np.float64)
        lo = np.zeros(self.n, np.uint32) if want_leaf_of else None
        out = TreeOut(_ptr(sf), _ptr(sb), _ptr(so), _ptr(lv), _ptr(lo), _ptr(sc))
        a = None if approx is None else np.ascontiguousarray(approx, np.float64)
        t = None if target is None else np.ascontiguousarray(target, np.float64)
        s = None if sample is None else np.ascontiguousarray(sample, np.float64)
        fam = None
        if isinstance(family, dict):
            ak = np.ascontiguousarray(family["approx_k"], np.float64)
            self._fam_keep = ak
            fam = Family(kind=2, approx_k=_ptr(ak), approx_dim=int(family["approx_dim"]))
        elif family is not None:
            arrs = _family_arrays(*family)
            self._fam_keep = arrs
            fam = _family(*arrs)
        _check(load().cbh_session_grow(self._s, _ptr(a), _ptr(t), self.n, _ptr(s),
                                       0 if s is None else s.shape[0],
                                       None if sampling is None else C.byref(sampling),
                                       None if fam is None else C.byref(fam), C.byref(out)))
        return {"splits": [(int(f), int(b), bool(o)) for f, b, o in zip(sf, sb, so)],
                "leaf_values": lv.reshape(1 << d, self.K), "leaf_of": lo, "scores": sc}

    def read_approx(self):
        a = np.zeros(self.n * self.K)
        _check(load().cbh_session_read_approx(self._s, _ptr(a), a.shape[0]))
        return a.reshape(self.K, self.n)

    def capture_hists(self, on=True):
        """Keep every later tree's level histograms (cbh_session_capture_hists)."""
        _check(load().cbh_session_capture_hists(self._s, int(bool(on))))

    def level_hist(self, level, n_features, n_bins):
        """Level ``level`` of the last tree: bin sums [2^level][F][n_bins][K+1] (channel K the
        weight), the reference's layout."""
        out = np.zeros(((1 << level), n_features, n_bins, self.K + 1), np.float64)
        _check(load().cbh_session_level_hist(self._s, level, _ptr(out), out.size))
        return out

    def stats(self):
        st = Stats()
        _check(load().cbh_session_stats(self._s, C.byref(st)))
        return st.as_dict()

    def end_device_training(self):
        if self._s:
            _check(load().cbh_session_end(self._s))
        self._s = C.c_void_p()


class Trainer:
    """cb-train's device branch over the C-ABI (host RNG phase, draw replay)."""

    def __init__(self, bins_fm, n_bins, target, *, loss="RMSE", depth=6, learning_rate=0.1,
                 l2_leaf_reg=3.0, score="Cosine", leaf_method="Gradient", bootstrap_type="No",
                 subsample=0.66, bagging_temperature=1.0, boost_from_average=False, random_seed=0,
                 weight=None, approx_dim=1, profile=False, real_folds=None, one_hot_flags=None,
                 pairs=None, group_offsets=None, pairwise_non_diag_reg=0.1, float_columns=None,
                 float_borders=None, ctr=None, device_ctr=None):
        """``pairs`` = (winner, loser[, weight]) and ``group_offsets`` (CSR over row order) for
        PairLogit / PairLogitPairwise.  With ``bins_fm`` None the trainer opens over the raw
        float channel: ``float_columns`` f32 [F][n] and ``float_borders`` (F arrays).  ``ctr`` =
        dict(avg_bins [n_ctr][n], bucket_count, group, cat_buckets [n_cat][n], cat_bucket_count,
        model_size_reg) when the last n_ctr columns are CTR columns (``cbt_set_ctr``);
        ``device_ctr`` = a ``DeviceCtr`` whose columns the session builds on the device and
        appends after the base features (``cbt_open_ctr``)."""
        raw = bins_fm is None
        if raw:
            x, cp = _column_ptrs(float_columns)
            bs, bp, nb = _border_ptrs(float_borders)
            self.bins = None
            F, n = x.shape
        else:
            self.bins = np.ascontiguousarray(bins_fm, np.uint8)
            F, n = self.bins.shape
        self.n, self.F, self.depth = n, F, depth
        self.K = approx_dim if loss == "MultiClass" else 1
        p = TrainParams(loss=LOSS[loss], score_function=SCORE[score], leaf_method=LEAF[leaf_method],
                        depth=depth, bootstrap_type=BOOT[bootstrap_type],
                        boost_from_average=int(boost_from_average), approx_dim=self.K,
                        profile=int(profile), learning_rate=learning_rate, l2_leaf_reg=l2_leaf_reg,
                        subsample=subsample, bagging_temperature=bagging_temperature,
                        random_seed=random_seed, pairwise_non_diag_reg=pairwise_non_diag_reg)
        t = np.ascontiguousarray(target, np.float64)
        w = None if weight is None else np.ascontiguousarray(weight, np.float64)
        rf = None if real_folds is None else np.ascontiguousarray(real_folds, np.uint32)
        oh = None if one_hot_flags is None else np.ascontiguousarray(one_hot_flags, np.uint8)
        self._keep = (t, w, rf, oh)
        self._h = C.c_void_p()
        if raw:
            if real_folds is not None or one_hot_flags is not None:
                raise ValueError("the raw float channel takes its folds from the borders and has no one-hot columns")
            self._keep += (x, cp, bs, bp, nb)
            _check(load().cbt_open_raw(C.byref(p), cp, bp, _ptr(nb), n, F, _ptr(t), _ptr(w), C.byref(self._h)))
        elif device_ctr is not None:
            self._keep += (device_ctr,)
            _check(load().cbt_open_ctr(C.byref(p), _ptr(self.bins), n, F, n_bins, _ptr(rf), _ptr(oh),
                                       device_ctr.ref(), _ptr(t), _ptr(w), C.byref(self._h)))
            self.F = F + device_ctr.n_columns
        else:
            _check(load().cbt_open(C.byref(p), _ptr(self.bins), n, F, n_bins, _ptr(rf), _ptr(oh), _ptr(t),
                                   _ptr(w), C.byref(self._h)))
        if ctr is not None:
            self._set_ctr(ctr, n)
        if pairs is not None:
            go, pw_, pl_, pwt = _family_arrays(group_offsets, *pairs)
            _check(load().cbt_set_pairs(self._h, _ptr(go), go.shape[0] - 1, _ptr(pw_), _ptr(pl_),
                                        _ptr(pwt), pw_.shape[0]))

    def _set_ctr(self, ctr, n):
        avg = np.ascontiguousarray(ctr["avg_bins"], np.uint8)
        m = avg.shape[0]
        bc = np.ascontiguousarray(ctr["bucket_count"], np.uint32)
        grp = np.ascontiguousarray(ctr.get("group", np.arange(m)), np.uint32)
        cat = np.ascontiguousarray(ctr.get("cat_buckets", np.zeros((0, n))), np.uint32)
        cnb = np.ascontiguousarray(ctr.get("cat_bucket_count",
                                           [int(c.max()) + 1 if c.size else 0 for c in cat]), np.uint32)
        self._ctr_keep = (avg, bc, grp, cat, cnb)
        info = CtrInfo(m, _ptr(avg), _ptr(bc), _ptr(grp), cat.shape[0], _ptr(cat) if cat.shape[0] else None,
                       _ptr(cnb) if cat.shape[0] else None, float(ctr.get("model_size_reg", 0.5)))
        _check(load().cbt_set_ctr(self._h, C.byref(info)))

    @classmethod
    def from_floats(cls, float_columns, float_borders, target, **kw):
        """Trainer over the raw float channel (the device quantizes the columns)."""
        return cls(None, None, target, float_columns=float_columns, float_borders=float_borders, **kw)

    def step(self):
        d = self.depth
        sf = np.zeros(d, np.uint32)
        sb = np.zeros(d, np.uint32)
        so = np.zeros(d, np.uint8)
        lv = np.zeros((self.K, 1 << d), np.float64)
        _check(load().cbt_step(self._h, _ptr(sf), _ptr(sb), _ptr(so), _ptr(lv)))
        return np.stack([sf, sb], 1).astype(np.int32), lv, so

    def fit(self, iterations, with_one_hot=False):
        """Grow ``iterations`` trees; returns (splits [it][depth][2], leaves [it][K][2^d]) and,
        with ``with_one_hot``, the per-level one-hot flags [it][depth]."""
        splits, leaves, kinds = [], [], []
        for _ in range(iterations):
            s, lv, so = self.step()
            splits.append(s)
            leaves.append(lv)
            kinds.append(so.astype(bool))
        if with_one_hot:
            return np.array(splits), np.array(leaves), np.array(kinds)
        return np.array(splits), np.array(leaves)

    def approx(self):
        a = np.zeros(self.n * self.K)
        _check(load().cbt_read_approx(self._h, _ptr(a)))
        return a.reshape(self.K, self.n)

    @property
    def bias(self):
        return load().cbt_bias(self._h)

    def stats(self):
        st = Stats()
        _check(load().cbt_stats(self._h, C.byref(st)))
        return st.as_dict()

    def reset_stats(self):
        load().cbt_reset_stats(self._h)

    def set_profile(self, on):
        """Per-stage HIP-event timing on (eager trees) or off (recorded trees replayed)."""
        _check(load().cbt_set_profile(self._h, int(bool(on))))

    def close(self):
        if self._h:
            load().cbt_close(self._h)
        self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
