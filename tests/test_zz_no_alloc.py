"""The no-allocation histogram entry (cbh_hist_build_noalloc) against cbh_hist_build: device
buffers in and out, scratch in the library's static device array, two calls in a row (the
second smaller, so stale scratch contents from the first would show), and the size limit."""
import ctypes as C

import numpy as np
import pytest

import catboost_rs_amd as cb

pytestmark = pytest.mark.gpu


def _case(seed, n, F, B, K):
    g = np.random.default_rng(seed)
    bins = g.integers(0, B, (F, n)).astype(np.uint8)
    der = g.standard_normal((K, n))
    w = g.uniform(0.0, 2.0, n)
    return bins, der, w


def _hip():
    """The HIP runtime the library itself links (one runtime per process: torch bundles
    another, which cannot share the device with it)."""
    cb.load()
    L = C.CDLL("/opt/rocm/lib/libamdhip64.so.7")
    L.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    L.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    L.hipFree.argtypes = [C.c_void_p]
    return L


def _noalloc(bins, n_bins, der, w):
    """The caller allocates the device inputs and the output; the entry allocates nothing."""
    L = _hip()
    F, n = bins.shape
    K = der.shape[0]
    out = np.full((F, n_bins, K + 1), np.nan)
    host = [np.ascontiguousarray(a) for a in (bins, der, w, out)]
    dev = []
    try:
        for a in host:
            p = C.c_void_p()
            assert L.hipMalloc(C.byref(p), a.nbytes) == 0
            dev.append(p)
            assert L.hipMemcpy(p, a.ctypes.data_as(C.c_void_p), a.nbytes, 1) == 0
        cb._check(cb.load().cbh_hist_build_noalloc(dev[0], n, F, n_bins, dev[1], dev[2], K, dev[3], None))
        assert L.hipDeviceSynchronize() == 0
        assert L.hipMemcpy(host[3].ctypes.data_as(C.c_void_p), dev[3], host[3].nbytes, 2) == 0
    finally:
        for p in dev:
            L.hipFree(p)
    return host[3]


def test_noalloc_hist_matches_hist_build_twice():
    for seed, n, F, B, K in ((1, 150_000, 40, 200, 1), (2, 20_000, 13, 33, 3)):
        bins, der, w = _case(seed, n, F, B, K)
        exp = cb.hist_build(bins, B, der, w)[0]
        got = _noalloc(bins, B, der, w)
        assert got.shape == exp.shape
        np.testing.assert_allclose(got, exp, rtol=1e-12, atol=1e-12 * np.abs(exp).max())
        # the weight channel sums to the total weight per feature, exactly as the entry's own
        np.testing.assert_allclose(got[:, :, K].sum(1), np.full(F, w.sum()), rtol=1e-12)


def test_noalloc_hist_rejects_inputs_beyond_the_scratch():
    n, F, B, K = 1_000_000, 64, 256, 1   # 24 MB of rows + 16 MB of statistics > 32 MiB
    with pytest.raises(cb.CbhError) as e:
        cb._check(cb.load().cbh_hist_build_noalloc(C.c_void_p(8), n, F, B, C.c_void_p(8), C.c_void_p(8), K,
                                                   C.c_void_p(8), None))
    assert e.value.code == -2
