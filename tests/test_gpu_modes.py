"""GPU: gpu_math="fast" and the reference's GPU knobs that this backend
honours (hist_streams, resident_blocks)."""

from __future__ import annotations

import numpy as np
import pytest

from helpers import assert_same_models, product_params

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fb():
    import ferrisboost_amd as fb
    from ferrisboost_amd import _native as N

    if not N.device_available(0):
        pytest.fail("no gfx950 device: the GPU suite needs an MI355X")
    return fb


def _pairs(N, objective, gpu_math, margin, labels, weights=None):
    out = np.zeros(2 * margin.size, np.float32)
    N.check_hip(N.hip().fbh_gradient_pairs(0, objective, gpu_math, N.ptr(margin), N.ptr(labels),
                                           N.ptr(weights), margin.size, N.ptr(out)))
    return out


def _binned(oracle, x, max_bin=255):
    """Column-major u8 bins under the oracle's sketch: #{cuts <= v}, NaN the
    sentinel (find_bin, src/data/columns.rs:335-341)."""
    vals, offs = oracle.sketch_cuts(x, max_bin)
    nf = x.shape[1]
    bins = np.empty((nf, x.shape[0]), np.uint8)
    hoffs = np.zeros(nf + 1, np.uint32)
    for f in range(nf):
        c = vals[offs[f]:offs[f + 1]]
        b = np.searchsorted(c, x[:, f], side="right").astype(np.int64)
        b[np.isnan(x[:, f])] = 0xFF
        bins[f] = b
        hoffs[f + 1] = hoffs[f] + c.size + 1
    return bins, hoffs


def test_fast_pairs_keep_per_bin_sums_within_1e6(fb, oracle):
    """gpu_math="fast" (apply_delta_and_gradient, src/backend/cuda/
    histogram.cu:673-783): deterministic, and every per-bin histogram sum of
    the narrow 10.5M x 28 workload's shape (here 1M rows, margins spread as
    after training) within 1e-6 of the exact sum, relative to the bin's
    magnitude. The exact pairs equal the oracle's host gradients bit for bit."""
    from ferrisboost_amd import _native as N
    from ferrisboost_amd import datasets

    x, y, _, _ = datasets.narrow_binary(1_000_000, seed=12)
    rng = np.random.default_rng(5)
    margin = (rng.normal(0.0, 2.5, size=y.size)).astype(np.float32)
    exact = _pairs(N, 1, 0, margin, y)
    fast = _pairs(N, 1, 1, margin, y)
    assert np.array_equal(fast.view(np.uint32), _pairs(N, 1, 1, margin, y).view(np.uint32))
    want = np.zeros_like(exact)
    oracle.lib().orc_gradients(oracle._p(margin), oracle._p(y), None, y.size, 1, oracle._p(want))
    assert np.array_equal(exact.view(np.uint32), want.view(np.uint32))
    assert not np.array_equal(exact.view(np.uint32), fast.view(np.uint32))  # a different exp
    bins, offs = _binned(oracle, x)
    scales = oracle.quantizer_scales(float(np.abs(exact[0::2]).max()),
                                     float(np.abs(exact[1::2]).max()), y.size)
    qe, _ = oracle.quantize(exact, scales)
    qf, _ = oracle.quantize(fast, scales)
    he = oracle.hist_build(bins, offs, qe).reshape(-1, 2).astype(np.float64)
    hf = oracle.hist_build(bins, offs, qf).reshape(-1, 2).astype(np.float64)
    mag = oracle.hist_build(bins, offs, np.abs(qe)).reshape(-1, 2).astype(np.float64)
    rel = np.abs(hf - he) / np.maximum(mag, 1.0)
    assert rel.max() <= 1e-6, rel.max()
    # Relative to the exact sum itself, over bins whose sum does not cancel
    # below 10 % of their magnitude (a cancelling bin's exact sum can be
    # near zero, where no relative bound holds).
    keep = np.abs(he) >= 0.1 * mag
    rel_exact = np.abs(hf - he)[keep] / np.abs(he)[keep]
    print(f"fast per-bin error: {rel.max():.3e} of the bin's magnitude, "
          f"{rel_exact.max():.3e} of the exact sum over {keep.mean():.1%} of the bins")
    assert rel_exact.max() <= 1e-5, rel_exact.max()


def test_fast_keeps_structure_on_the_reference_fixture(fb):
    """gpu_math_fast_keeps_structure_and_stays_deterministic
    (tests/gpu_histogram.rs:1411-1476) on its 3000 x 6 fixture: fast runs
    repeat byte for byte, the trees keep exact mode's structure (leaf flags,
    split features, thresholds, missing directions, children) and leaf values
    differ from exact mode's by less than 1e-3 relative."""
    n, nf = 3000, 6
    r = np.arange(n)[:, None]
    f = np.arange(nf)[None, :]
    x = ((r * 13 + f * 29) % 37).astype(np.float32)
    y = (((np.arange(n) * 17) % 23) < 11).astype(np.float32)
    p = {"max_depth": 4, "max_bin": 32, "cols_per_block": 3, "objective": "binary:logistic"}
    exact = fb.train(p, x, y, 3)
    fast = fb.train(dict(p, gpu_math="fast"), x, y, 3)
    again = fb.train(dict(p, gpu_math="fast"), x, y, 3)
    assert fast.to_json() == again.to_json()
    for te, tf in zip(exact.trees(), fast.trees()):
        assert te.size == tf.size
        assert np.array_equal(te["is_leaf"], tf["is_leaf"])
        s = te["is_leaf"] == 0
        for field in ("feat", "split_cond", "default_left", "left", "right"):
            assert np.array_equal(te[field][s], tf[field][s]), field
        lv = ~s
        d = np.abs(te["leaf_value"][lv] - tf["leaf_value"][lv])
        rel = d / np.maximum(np.abs(te["leaf_value"][lv]), 1e-12)
        assert rel.max() < 1e-3, rel.max()


def test_multiclass_fast_pairs_match_the_host_softmax(fb, oracle):
    """gpu_multiclass_fast_gradient_matches_host_softmax
    (tests/gpu_histogram.rs:2662-2738): from the same class margins, each
    class's fast device pairs quantize with the host softmax pairs' scales
    and their root sums differ by at most one fixed-point unit a row; the
    row sample (keyed on the tree index) selects the host's rows."""
    import ctypes as C

    from ferrisboost_amd import _native as N

    k, n = 5, 3000
    rows = np.arange(n)
    s = ((rows * 13) % 41) + ((rows * 5) % 7)
    labels = np.minimum(s * k // 48, k - 1).astype(np.float32)
    weights = np.array([0.5, 1.0, 2.0, 0.25, 3.0], np.float32)[(rows * 3) % 5]
    margins = (0.3 * np.arange(k, dtype=np.float32) - np.float32(0.7)).astype(np.float32)
    L = N.hip()
    width = np.ones(4, np.uint8)
    nbins = np.full(4, 19, np.uint32)
    shape = N.Shape(4, N.ptr(width), N.ptr(nbins), None)
    cfg = N.Config()
    cfg.n_outputs = k
    ctx = C.c_void_p()
    N.check_hip(L.fbh_ctx_create(0, n, C.byref(shape), C.byref(cfg), C.byref(ctx)))
    try:
        N.check_hip(L.fbh_set_multiclass(ctx, k, N.ptr(labels), N.ptr(weights), N.ptr(margins)))
        N.check_hip(L.fbh_set_gpu_math(ctx, 1))
        dev = np.zeros(k * n, np.float32)
        N.check_hip(L.fbh_download_margin(ctx, N.ptr(dev)))
        assert np.array_equal(dev.reshape(k, n), np.repeat(margins[:, None], n, axis=1))
        N.check_hip(L.fbh_multiclass_begin_round(ctx))
        class_margins = np.repeat(margins[:, None], n, axis=1)
        for rate, cls in ((1.0, 0), (1.0, 3), (0.6, 2)):
            tree = 7 * k + cls
            th = int(oracle.lib().orc_threshold_for(rate))
            host = oracle.softmax_pairs(class_margins, labels, weights, cls)
            sel = np.array([oracle.lib().orc_row_selected(i, th, 11, tree) for i in range(n)], bool)
            host[0::2][~sel] = 0.0
            host[1::2][~sel] = 0.0
            hs = oracle.quantizer_scales(float(np.abs(host[0::2]).max()),
                                         float(np.abs(host[1::2]).max()), n)
            hq, hsum = oracle.quantize(host, hs)
            N.check_hip(L.fbh_set_output(ctx, cls))
            scales = np.zeros(2, np.float64)
            root = np.zeros(2, np.int64)
            N.check_hip(L.fbh_gradient_exchange(ctx, None, None, th, 11, tree, N.ptr(scales),
                                                N.ptr(root)))
            assert scales.tolist() == list(hs), (cls, scales, hs)
            assert abs(int(root[0]) - int(hsum[0])) <= n and abs(int(root[1]) - int(hsum[1])) <= n
        with pytest.raises(ValueError):
            N.check_hip(L.fbh_set_output(ctx, k))
    finally:
        L.fbh_ctx_destroy(ctx)


def test_fast_training_is_deterministic(fb):
    from ferrisboost_amd import datasets

    x, y, params, _ = datasets.narrow_binary(300_000, seed=13, max_bin=255)
    p = dict(params, gpu_math="fast")
    a = fb.train(p, x, y, num_boost_round=12)
    b = fb.train(p, x, y, num_boost_round=12)
    assert_same_models(a, b)
    n = y.size
    assert np.array_equal(a.train_margins(n).view(np.uint32), b.train_margins(n).view(np.uint32))
    assert a.stats["device_sigmoid"] == 1
    # squared error has no exponential: fast equals exact
    sq = dict(params, objective="reg:squarederror")
    assert_same_models(fb.train(sq, x, y, num_boost_round=3),
                       fb.train(dict(sq, gpu_math="fast"), x, y, num_boost_round=3))


@pytest.mark.parametrize("knobs", [{"resident_blocks": 0}, {"resident_blocks": 1},
                                   {"resident_blocks": 0, "hist_streams": 1},
                                   {"hist_streams": 1, "gpu_memory_budget": None}])
def test_resident_blocks_and_hist_streams_keep_the_model(fb, oracle, knobs):
    """resident_blocks caps the resident tiles (0: everything streams) and
    hist_streams picks one or two streaming windows; trees and margins stay
    those of the all-resident run and the oracle."""
    rng = np.random.default_rng(101)
    n, nf = 60_013, 36
    x = rng.normal(size=(n, nf)).astype(np.float32)
    x[rng.random((n, nf)) < 0.03] = np.nan
    y = (np.nan_to_num(x[:, 1]) + np.nan_to_num(x[:, 20]) * np.nan_to_num(x[:, 33])
         + 0.4 * rng.normal(size=n) > 0).astype(np.float32)
    p = {"n_rounds": 3, "max_depth": 5, "eta": 0.3, "max_bin": 255}
    pp = product_params(p)
    ref = fb.train(pp, x, y, num_boost_round=3)
    kn = {k: v for k, v in knobs.items() if v is not None}
    got = fb.train(dict(pp, **kn), x, y, num_boost_round=3)
    if "resident_blocks" in kn:
        assert got.stats["resident_tiles"] == kn["resident_blocks"]
        assert got.stats["streamed_bytes"] > 0
    assert_same_models(ref, got)
    assert np.array_equal(got.train_margins(n).view(np.uint32), ref.train_margins(n).view(np.uint32))
    assert_same_models(oracle.train(x, y, oracle.make_params(**p)), got)


@pytest.mark.parametrize("kind", ["numeric", "categorical_wide"])
def test_subtraction_inside_the_scan_keeps_the_model(fb, oracle, monkeypatch, kind):
    """Device-grown levels subtract siblings inside the split scan (the larger
    child's bins from its parent's slot, stored back for the next level);
    FB_HIP_NO_SUB_IN_SCAN=1 runs the subtraction as its own launch. Both give
    the same trees and margins, with a per-node feature mask too (a feature
    masked out of the larger child still has its bins subtracted and stored,
    since the next level scans them), for numeric features of at most 256
    bins and for categorical and 257-1024-bin ones."""
    rng = np.random.default_rng(202)
    n = 40_000
    if kind == "numeric":
        nf = 24
        x = rng.normal(size=(n, nf)).astype(np.float32)
        types = None
        p = {"max_depth": 6, "eta": 0.3, "max_bin": 255, "colsample_bynode": 0.6}
    else:
        nf = 12
        x = rng.normal(size=(n, nf)).astype(np.float32)
        x[:, 8:] = rng.integers(0, 300, size=(n, 4)).astype(np.float32)
        types = ["q"] * 8 + ["c"] * 4
        p = {"max_depth": 6, "eta": 0.3, "max_bin": 1000, "colsample_bynode": 0.6,
             "max_cat_to_onehot": 4}
    x[rng.random((n, nf)) < 0.03] = np.nan
    y = (np.nan_to_num(x[:, 1]) + np.nan_to_num(x[:, 5]) * 0.5
         + 0.3 * rng.normal(size=n) > 0).astype(np.float32)
    pp = dict(product_params(p), seed=7)
    if types:
        pp["feature_types"] = types
    fused = fb.train(pp, x, y, num_boost_round=4)
    monkeypatch.setenv("FB_HIP_NO_SUB_IN_SCAN", "1")
    apart = fb.train(pp, x, y, num_boost_round=4)
    assert_same_models(fused, apart)
    assert np.array_equal(fused.train_margins(n).view(np.uint32),
                          apart.train_margins(n).view(np.uint32))
