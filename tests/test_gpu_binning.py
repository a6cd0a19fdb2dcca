"""GPU: binning of row-major f32 rows on the device (fbh_set_cuts,
fbh_upload_rows, fbh_finish_rows) gives the host's bins (find_bin /
quantize_value, src/data/columns.rs:335-356; categorical::code_to_bin):
checked through the root histogram of random fixed-point pairs against the
oracle's histogram of the host-binned columns, and through whole trainings,
device-binned against host-binned, byte for byte."""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from helpers import assert_same_models

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fb_mod():
    import ferrisboost_amd as fb

    return fb


@pytest.fixture(scope="module")
def N():
    from ferrisboost_amd import _native as N

    if not N.device_available(0):
        pytest.fail("no gfx950 device: the GPU suite needs an MI355X")
    return N


def _host_bins(x, cuts, offsets, cat, width):
    """The host engine's bins of every column (Cuts::bin_of)."""
    n, nf = x.shape
    out = []
    for f in range(nf):
        v = x[:, f]
        miss = 0xFF if width[f] == 1 else 0xFFFF
        nb = int(offsets[f + 1] - offsets[f]) + 1
        if cat[f]:
            with np.errstate(invalid="ignore"):
                ok = (v >= 0) & (v < np.float32(nb))
            b = np.where(ok, np.nan_to_num(v, nan=0.0).astype(np.int64), miss - 1)
        else:
            b = np.searchsorted(cuts[offsets[f]:offsets[f + 1]], v, side="right")
        b = np.where(np.isnan(v), miss, b)
        out.append(b.astype(np.uint8 if width[f] == 1 else np.uint16))
    return out


def _edge_matrix(n, seed):
    """Numeric columns with NaN, +-inf, -0.0 and values equal to their cuts;
    categorical columns with in-range, negative, too large, fractional and
    NaN codes; widths u8 (200 bins, 60 codes) and u16 (700 bins, 400 codes)."""
    rng = np.random.default_rng(seed)
    specs = [("q", 200), ("q", 700), ("c", 60), ("c", 400), ("q", 2), ("q", 255), ("c", 254)]
    nf = len(specs)
    x = np.empty((n, nf), np.float32)
    cuts, offsets, cat = [], [0], []
    for f, (kind, nb) in enumerate(specs):
        if kind == "q":
            c = np.sort(rng.choice(np.linspace(-3, 3, 5 * nb, dtype=np.float32), nb - 1,
                                   replace=False))
            v = rng.normal(size=n).astype(np.float32) * 1.5
            pick = rng.random(n)
            v[pick < 0.15] = c[rng.integers(0, c.size, size=n)][pick < 0.15]  # exactly a cut
            v[(pick >= 0.15) & (pick < 0.2)] = np.nan
            v[(pick >= 0.2) & (pick < 0.21)] = np.inf
            v[(pick >= 0.21) & (pick < 0.22)] = -np.inf
            v[(pick >= 0.22) & (pick < 0.23)] = -0.0
            cat.append(0)
        else:
            c = np.arange(1, nb, dtype=np.float32)
            v = rng.integers(0, nb, size=n).astype(np.float32)
            pick = rng.random(n)
            v[pick < 0.05] = -1.0
            v[(pick >= 0.05) & (pick < 0.1)] = nb + rng.integers(0, 5, size=n)[(pick >= 0.05) & (pick < 0.1)]
            v[(pick >= 0.1) & (pick < 0.12)] = np.nan
            v[(pick >= 0.12) & (pick < 0.14)] = 2.5
            v[(pick >= 0.14) & (pick < 0.15)] = 1e9
            cat.append(1)
        x[:, f] = v
        cuts.append(c)
        offsets.append(offsets[-1] + c.size)
    return (x, np.concatenate(cuts).astype(np.float32), np.array(offsets, np.uint32),
            np.array(cat, np.uint8))


@pytest.mark.parametrize("n", [5_003, 70_000])
def test_device_bins_give_the_host_histogram(N, oracle, n):
    x, cuts, offsets, cat = _edge_matrix(n, seed=n)
    nf = x.shape[1]
    nbins = (np.diff(offsets.astype(np.int64)) + 1).astype(np.uint32)
    width = np.array([1 if nb <= (254 if c else 255) else 2 for nb, c in zip(nbins, cat)],
                     np.uint8)
    want_bins = _host_bins(x, cuts, offsets, cat, width)
    rng = np.random.default_rng(n + 1)
    fixed = rng.integers(-(1 << 40), 1 << 40, size=2 * n).astype(np.int64)
    fixed[1::2] = np.abs(fixed[1::2])
    hist_off = np.concatenate([[0], np.cumsum(nbins)]).astype(np.uint32)
    # The unseen-category code (past the feature's bins) is in no histogram
    # bin, as the missing code: give the oracle the missing code for it.
    want = []
    for f, b in enumerate(want_bins):
        miss = 0xFF if width[f] == 1 else 0xFFFF
        b = np.where(b >= nbins[f], miss, b).astype(b.dtype)
        want.append(oracle.hist_build(b.reshape(1, -1), np.array([0, nbins[f]], np.uint32), fixed))
    want = np.concatenate(want)
    # the device bins hold unseen codes where the host's do
    assert any((b == (0xFE if width[f] == 1 else 0xFFFE)).any() for f, b in enumerate(want_bins)
               if cat[f])

    L = N.hip()
    shape = N.Shape(nf, N.ptr(width), N.ptr(nbins), N.ptr(cat))
    cfg = N.Config()
    ctx = C.c_void_p()
    N.check_hip(L.fbh_ctx_create(0, n, C.byref(shape), C.byref(cfg), C.byref(ctx)))
    try:
        N.check_hip(L.fbh_set_cuts(ctx, N.ptr(cuts), N.ptr(offsets), N.ptr(cat)))
        assert L.fbh_rows_staging_bytes(ctx) > 0
        # three chunks of uneven sizes
        cuts_at = [0, n // 3 + 1, 2 * n // 3 + 7, n]
        xc = np.ascontiguousarray(x)
        for a, b in zip(cuts_at[:-1], cuts_at[1:]):
            N.check_hip(L.fbh_upload_rows(ctx, N.ptr(xc[a:b]), a, b - a))
        N.check_hip(L.fbh_finish_rows(ctx))
        scales = np.array([1.0, 1.0])
        N.check_hip(L.fbh_upload_gpair_fixed(ctx, N.ptr(fixed), N.ptr(scales)))
        root = N.Span()
        N.check_hip(L.fbh_begin_tree(ctx, None, 0, None, 0, C.byref(root)))
        node = N.NodeReq()
        node.rows = root
        node.sum[0] = int(fixed[0::2].sum())
        node.sum[1] = int(fixed[1::2].sum())
        node.lower, node.upper = -3.4028234663852886e38, 3.4028234663852886e38
        node.slot, node.subtract_parent, node.subtract_sibling = 0, -1, -1
        sp = N.SplitParams()
        sp.lambda_ = 1.0
        sp.max_cat_to_onehot, sp.max_cat_threshold = 4, 64
        out = N.SplitOut()
        words = np.zeros(64, np.uint64)
        N.check_hip(L.fbh_eval_nodes(ctx, C.byref(node), 1, C.byref(sp), None, C.byref(out),
                                     N.ptr(words), C.c_uint32(words.size)))
        got = np.zeros(2 * int(hist_off[-1]), np.int64)
        w = C.c_uint64()
        N.check_hip(L.fbh_download_histogram(ctx, 0, N.ptr(got), C.byref(w)))
    finally:
        L.fbh_ctx_destroy(ctx)
    assert w.value == hist_off[-1]
    assert np.array_equal(got, want)


@pytest.mark.parametrize("case", ["narrow_u8", "u16_categorical", "sampled"])
def test_device_binned_training_equals_host_binned(case):
    import ferrisboost_amd as fb
    from ferrisboost_amd import datasets

    if case == "narrow_u8":
        X, y, params, _ = datasets.narrow_binary(60_001)
        params = dict(params, max_bin=255)
        X[::11, 3] = np.nan
        X[::13, 5] = np.inf
    elif case == "u16_categorical":
        X, y, params, _ = datasets.widebin_cat(40_000, n_num=10, n_cat=4, n_codes=300)
        params = dict(params, max_bin=700, max_leaves=0, max_depth=6)
    else:
        X, y, params, _ = datasets.wide_binary(12_000, n_features=120)
    rounds = 4
    dev = fb.train(params, X, y, num_boost_round=rounds)
    host = fb.train(dict(params, hip_host_binning=True), X, y, num_boost_round=rounds)
    assert dev.stats["device_binning"] == 1 and host.stats["device_binning"] == 0
    assert_same_models(host, dev)
    n = y.size
    assert np.array_equal(dev.train_margins(n).view(np.uint32), host.train_margins(n).view(np.uint32))


def test_streamed_plan_bins_on_the_device(fb_mod, N, monkeypatch):
    """A plan that streams tiles from pinned host memory bins on the device
    too: each chunk of rows is binned into a stage, resident tiles are packed
    in place and streamed tiles' records and columns are copied back to their
    pinned memory. The model equals the host-binned one at the same budget
    and the all-resident one, byte for byte."""
    from test_gpu_parity import _streaming_budgets

    fb = fb_mod
    rng = np.random.default_rng(71)
    n, nf = 120_007, 40
    x = rng.normal(size=(n, nf)).astype(np.float32)
    x[rng.random((n, nf)) < 0.04] = np.nan
    y = (np.nan_to_num(x[:, 0]) - np.nan_to_num(x[:, 7]) * np.nan_to_num(x[:, 31])
         + 0.3 * rng.normal(size=n) > 0).astype(np.float32)
    p = {"objective": "binary:logistic", "max_depth": 6, "eta": 0.3, "max_bin": 255}
    ref = fb.train(p, x, y, num_boost_round=4)
    assert ref.stats["resident_tiles"] == ref.stats["n_tiles"] and ref.stats["device_binning"]
    some, _ = _streaming_budgets(N, ref, n, 32)
    # small row stages, so the budget's room left by the plan holds them
    monkeypatch.setenv("FB_HIP_STAGE_ROWS", "2048")
    for k in range(64):
        budget = some + k * (1 << 18)
        dev = fb.train(dict(p, gpu_memory_budget=budget), x, y, num_boost_round=4)
        if dev.stats["resident_tiles"] == dev.stats["n_tiles"]:
            break
        if dev.stats["device_binning"]:
            assert dev.stats["streamed_bytes"] > 0 and dev.stats["device_bytes"] <= budget
            host = fb.train(dict(p, gpu_memory_budget=budget, hip_host_binning=True), x, y,
                            num_boost_round=4)
            assert host.stats["device_binning"] == 0
            assert host.stats["resident_tiles"] == dev.stats["resident_tiles"]
            assert_same_models(host, dev)
            assert_same_models(ref, dev)
            assert np.array_equal(dev.train_margins(n).view(np.uint32),
                                  ref.train_margins(n).view(np.uint32))
            return
    pytest.fail("no budget between streaming and full residency left room for device binning")
