"""GPU parity: the HIP path against the CPU oracle, through the C ABI.

Integer work (histograms, partitions, node sums, split packets, trees) must
be bit-identical; margins are compared bit for bit with the oracle and with
the reference's XGBoost-3.4.1 golden margins.
"""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from helpers import (assert_same_models, case_params, golden_cases, load_case,
                     product_params)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fb():
    import ferrisboost_amd as fb
    from ferrisboost_amd import _native as N

    if not N.device_available(0):
        pytest.fail("no gfx950 device: the GPU suite needs an MI355X")
    return fb


@pytest.fixture(scope="module")
def N(fb):
    from ferrisboost_amd import _native as N

    return N


def _device_hist(N, bins, offsets, gpair, rows=None):
    bins = np.ascontiguousarray(bins)
    nf, n = bins.shape
    out = np.zeros(2 * int(offsets[-1]), np.int64)
    r = None if rows is None else np.ascontiguousarray(rows, np.uint32)
    N.check_hip(N.hip().fbh_build_histogram(
        0, N.ptr(bins), bins.dtype.itemsize, n, nf, N.ptr(np.ascontiguousarray(offsets, np.uint32)),
        N.ptr(np.ascontiguousarray(gpair, np.int64)), N.ptr(r), 0 if r is None else r.size,
        N.ptr(out)))
    return out


@pytest.mark.parametrize("width", [1, 2])
@pytest.mark.parametrize("n_feats", [1, 3, 7, 28, 63])
def test_histogram_matches_oracle(N, oracle, width, n_feats):
    rng = np.random.default_rng(100 + n_feats * 3 + width)
    n = 4203
    n_bins = rng.integers(1, 255 if width == 1 else 1200, size=n_feats)
    offsets = np.concatenate([[0], np.cumsum(n_bins)]).astype(np.uint32)
    dtype = np.uint8 if width == 1 else np.uint16
    miss = 0xFF if width == 1 else 0xFFFF
    bins = np.empty((n_feats, n), dtype)
    for f in range(n_feats):
        b = rng.integers(0, n_bins[f], size=n)
        b[rng.random(n) < 0.1] = miss
        bins[f] = b
    big = 1 << 42
    g = rng.integers(-big, big, size=n)
    h = rng.integers(0, big, size=n)
    gpair = np.stack([g, h], axis=1).reshape(-1).astype(np.int64)
    for rows in (None, np.sort(rng.choice(n, size=n // 7, replace=False)),
                 np.array([0, 4202, 0, 2048, 2048, 17], np.uint32), np.array([2047], np.uint32)):
        got = _device_hist(N, bins, offsets, gpair, rows)
        want = oracle.hist_build(bins, offsets, gpair, rows)
        assert np.array_equal(got, want)


@pytest.mark.parametrize("n_feats", [9, 17, 40])
def test_histogram_interleaved_16bit_matches_oracle(N, oracle, n_feats):
    """16-bit features of at most 256 bins share interleaved tiles of 16
    cells (32-byte records): bins 0..255, the all-ones missing code, bin
    counts from 1 to 256."""
    rng = np.random.default_rng(700 + n_feats)
    n = 5001
    n_bins = rng.integers(1, 257, size=n_feats)
    n_bins[0] = 256
    offsets = np.concatenate([[0], np.cumsum(n_bins)]).astype(np.uint32)
    bins = np.empty((n_feats, n), np.uint16)
    for f in range(n_feats):
        b = rng.integers(0, n_bins[f], size=n)
        b[rng.random(n) < 0.08] = 0xFFFF
        bins[f] = b
    gpair = rng.integers(-(1 << 41), 1 << 41, size=2 * n).astype(np.int64)
    for rows in (None, np.sort(rng.choice(n, size=n // 5, replace=False)).astype(np.uint32)):
        got = _device_hist(N, bins, offsets, gpair, rows)
        assert np.array_equal(got, oracle.hist_build(bins, offsets, gpair, rows))


def test_histogram_wide_features_use_global_path(N, oracle):
    # 16-bit features whose histogram exceeds an LDS tile, mixed with small ones.
    rng = np.random.default_rng(55)
    n = 20_000
    n_bins = np.array([5000, 7, 60000, 300], np.int64)
    offsets = np.concatenate([[0], np.cumsum(n_bins)]).astype(np.uint32)
    bins = np.empty((4, n), np.uint16)
    for f in range(4):
        b = rng.integers(0, n_bins[f], size=n)
        b[rng.random(n) < 0.05] = 0xFFFF
        bins[f] = b
    gpair = rng.integers(-(1 << 40), 1 << 40, size=2 * n).astype(np.int64)
    for rows in (None, np.sort(rng.choice(n, 3000, replace=False)).astype(np.uint32)):
        got = _device_hist(N, bins, offsets, gpair, rows)
        assert np.array_equal(got, oracle.hist_build(bins, offsets, gpair, rows))


def test_histogram_low_word_carry(N, oracle):
    # Values whose low 32 bits overflow when summed: exact 64-bit wrapping sums.
    n = 9000
    bins = np.zeros((1, n), np.uint8)
    bins[0] = np.arange(n) % 3
    v = np.full(n, (1 << 32) - 1, np.int64)
    gpair = np.stack([v, v // 3], axis=1).reshape(-1)
    offsets = np.array([0, 3], np.uint32)
    got = _device_hist(N, bins, offsets, gpair)
    assert np.array_equal(got, oracle.hist_build(bins, offsets, gpair))
    # wrapping: near i64 limits
    v2 = np.full(n, (1 << 62), np.int64)
    gpair2 = np.stack([v2, -v2], axis=1).reshape(-1)
    got2 = _device_hist(N, bins, offsets, gpair2)
    assert np.array_equal(got2, oracle.hist_build(bins, offsets, gpair2))


@pytest.mark.parametrize("width", [1, 2])
def test_partition_matches_oracle(N, oracle, width):
    rng = np.random.default_rng(7 + width)
    n = 10_037
    nb = 200 if width == 1 else 3000
    dtype = np.uint8 if width == 1 else np.uint16
    miss = 0xFF if width == 1 else 0xFFFF
    col = rng.integers(0, nb, size=n).astype(dtype)
    col[rng.random(n) < 0.15] = miss
    for rows in (np.arange(n, dtype=np.uint32), np.sort(rng.choice(n, 5000, replace=False)).astype(np.uint32)):
        for split_bin, ml in ((0, True), (nb // 3, False), (nb // 3, True), (nb, False)):
            out = np.zeros_like(rows)
            nl = C.c_uint64()
            N.check_hip(N.hip().fbh_partition_rows(0, N.ptr(col), width, n, N.ptr(rows), rows.size,
                                                   split_bin, int(ml), None, 0, N.ptr(out),
                                                   C.byref(nl)))
            want, wl = oracle.partition(rows, col, split_bin, ml)
            assert nl.value == wl
            assert np.array_equal(out, want)
        # categorical set
        cats = np.zeros((nb + 63) // 64, np.uint64)
        for c in rng.choice(nb, nb // 4, replace=False):
            cats[c >> 6] |= np.uint64(1) << np.uint64(c & 63)
        out = np.zeros_like(rows)
        nl = C.c_uint64()
        N.check_hip(N.hip().fbh_partition_rows(0, N.ptr(col), width, n, N.ptr(rows), rows.size, 0,
                                               1, N.ptr(cats), cats.size, N.ptr(out), C.byref(nl)))
        want, wl = oracle.partition(rows, col, 0, True, cats)
        assert nl.value == wl and np.array_equal(out, want)


CASES = golden_cases()


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_golden_training_is_bit_exact(fb, oracle, case):
    x, y, w, want = load_case(case)
    p = case_params(case)
    mono = case.get("monotone_constraints")
    om = oracle.train(x, y, oracle.make_params(**p), weights=w, monotone=mono)
    pp = product_params(p)
    if mono:
        pp["monotone_constraints"] = mono
    pm = fb.train(pp, x, y, weight=w, num_boost_round=p["n_rounds"])
    assert_same_models(om, pm)
    got = pm.predict(x, output_margin=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(pm.train_margins(x.shape[0]).view(np.uint32),
                          om.train_margins(x.shape[0]).view(np.uint32))


def _synthetic(kind, n):
    from ferrisboost_amd import datasets

    return getattr(datasets, kind)(n)


def test_device_sigmoid_equals_host_libm_on_every_float(N, oracle):
    """The device sigmoid (expf restated from glibc's method) against the
    host libm's 1 / (1 + expf(-x)) on all 2^32 float inputs, compared by
    fingerprints of four 2^30-input ranges."""
    import os

    threads = max(1, min(16, os.cpu_count() or 1))
    for k in range(4):
        b, e = k << 30, (k + 1) << 30
        dev = C.c_uint64()
        N.check_hip(N.hip().fbh_sigmoid_checksum(0, b, e, C.byref(dev)))
        host = oracle.lib().orc_sigmoid_checksum(b, e, threads)
        assert dev.value == host, f"range {k}: device {dev.value:#x} host {host:#x}"
    # denormal and saturated outputs element by element
    x = np.array([-88.0, -87.5, -88.7, -89.0, -103.0, 0.0, -0.0, 1e-30, 20.0, 88.0, -20.0,
                  np.inf, -np.inf], np.float32)
    got = np.empty_like(x)
    want = np.empty_like(x)
    N.check_hip(N.hip().fbh_sigmoid_device(0, N.ptr(x), x.size, N.ptr(got)))
    oracle.lib().orc_sigmoid(oracle._p(x), x.size, oracle._p(want))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("objective, depth, host_sigmoid", [
    ("binary:logistic", 6, False), ("reg:squarederror", 6, False), ("binary:logistic", 10, False),
    ("binary:logistic", 6, True), ("binary:logistic", 10, True)])
def test_sampled_weighted_rounds_match_oracle(fb, oracle, objective, depth, host_sigmoid):
    """Device margins, leaf ids (u8 up to 256 leaves, u16 beyond), the device
    sigmoid or the chunked host-sigmoid exchange, and on-device gradient pairs
    reproduce the host round (subsample, row weights, scale_pos_weight,
    missing values)."""
    rng = np.random.default_rng(depth * 7 + len(objective))
    n, nf = 40_037, 7
    x = rng.normal(size=(n, nf)).astype(np.float32)
    x[rng.random((n, nf)) < 0.05] = np.nan
    z = np.nan_to_num(x[:, 0]) - 0.7 * np.nan_to_num(x[:, 1]) * np.nan_to_num(x[:, 2])
    if objective == "binary:logistic":
        y = (z + 0.3 * rng.normal(size=n) > 0).astype(np.float32)
    else:
        y = (z + 0.1 * rng.normal(size=n)).astype(np.float32)
    w = rng.uniform(0.2, 3.0, size=n).astype(np.float32)
    p = {"n_rounds": 7, "max_depth": depth, "eta": 0.3, "subsample": 0.7, "seed": 11,
         "max_bin": 64, "objective": objective, "min_child_weight": 0.5}
    if objective == "binary:logistic":
        p.update(scale_pos_weight=2.5, base_score=0.4)
    om = oracle.train(x, y, oracle.make_params(**p), weights=w)
    pm = fb.train(dict(product_params(p), hip_host_sigmoid=host_sigmoid), x, y, weight=w,
                  num_boost_round=p["n_rounds"])
    assert_same_models(om, pm)
    if objective == "binary:logistic":
        assert pm.stats["device_sigmoid"] == (0 if host_sigmoid else 1)
    if depth > 8:
        assert max(int(t["is_leaf"].sum()) for t in pm.trees()) > 256
    assert np.array_equal(pm.train_margins(n).view(np.uint32), om.train_margins(n).view(np.uint32))


@pytest.mark.parametrize("case", ["budget", "monotone", "categorical", "sampled_deep", "stump",
                                  "squared", "walk_budget", "walk_categorical", "walk_squared",
                                  "walk_u16", "lg_plain", "lg_monotone", "lg_categorical",
                                  "lg_sampled_deep", "lg_cap64", "lg_cap11", "lg_cap9_categorical",
                                  "walk_lg_cap11", "lg_cap20_monotone"])
def test_device_grown_trees_match_host_levels_and_oracle(fb, oracle, case):
    """Whole depthwise trees grown on the device (the max_leaves budget, node
    ids, weights, bounds, slots, partitions and leaves decided by kernels)
    equal the trees the host grows level by level and the CPU oracle's, node
    for node, with margins equal bit for bit. The walk_ cases use 4 KiB tiles:
    two features a tile, three tiles in one 16-byte row bundle, so leaves and
    margins come from the row-order walk of the finished tree instead of a
    last-level partition; walk_u16 has 300 bins (16-bit cells, three
    features a 16 KiB tile, two tiles in one 16-byte bundle). The lg_ cases
    grow lossguide trees: whose leaf cap cannot bind (max_leaves 0, or 64 at
    depth 6), where the device grows every split and the host numbers the
    nodes in best-first order; and under a binding cap (9, 11, 20 leaves at
    depth 6), where the host keeps the splits best-first expansion takes
    before the cap and the device adds the kept leaves' values to the rows
    afterwards; against the host's expansion-by-expansion growth."""
    walk = case.startswith("walk_")
    case = case[5:] if walk else case
    lossguide = case.startswith("lg_")
    case = case[3:] if lossguide else case
    wide_bins = case == "u16"
    rng = np.random.default_rng(sum(map(ord, case)))
    n, nf = 30_011, 6
    x = rng.normal(size=(n, nf)).astype(np.float32)
    x[rng.random((n, nf)) < 0.04] = np.nan
    z = np.nan_to_num(x[:, 0]) - 0.8 * np.nan_to_num(x[:, 1]) + 0.5 * np.nan_to_num(x[:, 2]) ** 2
    y = (z + 0.4 * rng.normal(size=n) > 0.3).astype(np.float32)
    p = {"n_rounds": 5, "max_depth": 6, "eta": 0.3, "max_bin": 64,
         "objective": "binary:logistic"}
    w = None
    mono = None
    cat = None
    if case == "budget":
        p.update(max_leaves=11)
    elif case == "monotone":
        mono = [1, -1, 0, 1, 0, 0]
    elif case == "categorical":
        x[:, 5] = rng.integers(0, 40, n)
        y = ((x[:, 5] % 3 == 1) | (np.nan_to_num(x[:, 0]) > 1)).astype(np.float32)
        cat = [0, 0, 0, 0, 0, 1]
    elif case == "sampled_deep":
        p.update(max_depth=10, subsample=0.6, seed=3, min_child_weight=0.3)
        w = rng.uniform(0.5, 2.0, size=n).astype(np.float32)
    elif case == "stump":
        p.update(max_depth=1)
    elif case == "squared":
        p.update(objective="reg:squarederror")
        y = z.astype(np.float32)
    elif case == "u16":
        p.update(max_bin=300)
    elif case == "cap64":
        p.update(max_leaves=64)
    elif case == "cap11":
        p.update(max_leaves=11)
    elif case == "cap9_categorical":
        x[:, 5] = rng.integers(0, 40, n)
        y = ((x[:, 5] % 3 == 1) | (np.nan_to_num(x[:, 0]) > 1)).astype(np.float32)
        cat = [0, 0, 0, 0, 0, 1]
        p.update(max_leaves=9)
    elif case == "cap20_monotone":
        mono = [1, -1, 0, 1, 0, 0]
        p.update(max_leaves=20)
    if lossguide:
        p.update(grow_policy="lossguide")
    om = oracle.train(x, y, oracle.make_params(**p), weights=w, monotone=mono, categorical=cat)
    pp = product_params(p)
    if walk:
        pp["hip_tile_bytes"] = 16384 if wide_bins else 4096
    if mono:
        pp["monotone_constraints"] = mono
    if cat:
        pp["feature_types"] = ["c" if c else "q" for c in cat]
    dev = fb.train(pp, x, y, weight=w, num_boost_round=p["n_rounds"])
    host = fb.train(dict(pp, hip_host_levels=True), x, y, weight=w, num_boost_round=p["n_rounds"])
    assert dev.stats["device_trees"] == p["n_rounds"]
    assert host.stats["device_trees"] == 0
    assert_same_models(om, dev)
    assert_same_models(om, host)
    want = om.train_margins(n).view(np.uint32)
    assert np.array_equal(dev.train_margins(n).view(np.uint32), want)
    assert np.array_equal(host.train_margins(n).view(np.uint32), want)


class _TreeNode(C.Structure):
    _fields_ = [("feat", C.c_uint32), ("bin", C.c_uint32), ("left", C.c_int32),
                ("right", C.c_int32), ("leaf_value", C.c_float), ("sum_hess", C.c_float),
                ("gain", C.c_float), ("flags", C.c_uint32), ("cat_offset", C.c_uint32),
                ("n_cat_words", C.c_uint32), ("value_as_leaf", C.c_float),
                ("leaf_pos", C.c_uint32)]


class _GrowParams(C.Structure):
    _fields_ = [("max_depth", C.c_uint32), ("max_leaves", C.c_uint32),
                ("learning_rate", C.c_float), ("flags", C.c_uint32)]


@pytest.mark.parametrize("tile_bytes", [0, 4096])
def test_device_grown_tree_from_host_pairs_matches_oracle_splits(N, oracle, tile_bytes):
    """A whole tree grown through the C ABI from fixed-point pairs the host
    quantized (no device objective: leaves land in the prediction delta),
    against a depthwise grower built from the oracle's histogram, split and
    partition: every split (feature, bin, missing direction, gain bit for
    bit), the children's Hessian sums, node numbering, and each row's delta
    equal to the value of the leaf the oracle's partitions put it in. With
    4 KiB tiles the five features share one row bundle and the leaves come
    from the row-order walk; with the default tile they come from the leaf
    spans."""
    rng = np.random.default_rng(77 + tile_bytes)
    n, nf, nb, depth = 20_011, 5, 41, 4
    bins = rng.integers(0, nb, size=(nf, n)).astype(np.uint8)
    bins[rng.random((nf, n)) < 0.05] = 0xFF
    g = rng.integers(-(1 << 30), 1 << 30, size=n)
    g += (bins[0].astype(np.int64) - nb // 2) << 26  # make feature 0 informative
    h = rng.integers(1, 1 << 30, size=n)
    fixed = np.stack([g, h], axis=1).reshape(-1).astype(np.int64)
    scales = np.array([2.0 ** 24, 2.0 ** 26])
    offsets = np.arange(nf + 1, dtype=np.uint32) * nb
    feat_ids = np.arange(nf, dtype=np.uint32)
    lam, mcw, eta = 1.0, 0.5, 0.3
    op = oracle.make_params(**{"lambda": lam, "gamma": 0.0, "min_child_weight": mcw})

    # The oracle's depthwise tree: levels in order, children ids tree_size + 2s.
    want = {}  # node id -> (feat, bin, missing_left, gain bits, left id, right id)
    leaf_rows = {}
    level = [(0, np.arange(n, dtype=np.uint32), np.array([g.sum(), h.sum()], np.int64))]
    size = 1
    for d in range(depth):
        nxt = []
        for node, rows, ssum in level:
            sp = None
            if rows.size:
                hist = oracle.hist_build(bins, offsets, fixed, rows)
                sp = oracle.best_split(hist, feat_ids, offsets, ssum, scales, op)
            if sp is None or not sp.found:
                leaf_rows[node] = rows
                continue
            out, nl = oracle.partition(rows, bins[sp.feat], sp.bin, bool(sp.missing_left))
            lid, rid = size, size + 1
            size += 2
            want[node] = (sp.feat, sp.bin, bool(sp.missing_left),
                          np.float32(sp.gain).view(np.uint32), lid, rid,
                          np.array(sp.left, np.int64), np.array(sp.right, np.int64))
            nxt.append((lid, out[:nl], np.array(sp.left, np.int64)))
            nxt.append((rid, out[nl:], np.array(sp.right, np.int64)))
        level = nxt
    for node, rows, _ in level:
        leaf_rows[node] = rows

    L = N.hip()
    width = np.ones(nf, np.uint8)
    nbins = np.full(nf, nb, np.uint32)
    shape = N.Shape(nf, N.ptr(width), N.ptr(nbins), None)
    cfg = N.Config()
    cfg.tile_bytes = tile_bytes
    ctx = C.c_void_p()
    N.check_hip(L.fbh_ctx_create(0, n, C.byref(shape), C.byref(cfg), C.byref(ctx)))
    try:
        N.check_hip(L.fbh_upload_block(ctx, N.ptr(feat_ids), nf, 1, N.ptr(np.ascontiguousarray(bins))))
        N.check_hip(L.fbh_upload_gpair_fixed(ctx, N.ptr(fixed), N.ptr(scales)))
        root = N.Span()
        N.check_hip(L.fbh_begin_tree(ctx, None, 0, None, 0, C.byref(root)))
        sp = N.SplitParams()
        sp.lambda_, sp.gamma, sp.min_child_weight = lam, 0.0, mcw
        gp = _GrowParams(depth, 0, eta, 0)
        cap = (2 << depth) - 1
        nodes = (_TreeNode * cap)()
        vals = np.zeros(1 << depth, np.float32)
        cats = np.zeros(1, np.uint64)
        nn, nlv = C.c_uint32(), C.c_uint32()
        root_sum = np.array([g.sum(), h.sum()], np.int64)
        N.check_hip(L.fbh_grow_depthwise(ctx, C.byref(gp), C.byref(sp), N.ptr(root_sum), nodes,
                                         C.c_uint32(cap), C.byref(nn), N.ptr(cats), C.c_uint32(1),
                                         N.ptr(vals), C.c_uint32(vals.size), C.byref(nlv)))
        delta = np.empty(n, np.float32)
        N.check_hip(L.fbh_download_delta(ctx, N.ptr(delta)))
    finally:
        L.fbh_ctx_destroy(ctx)

    assert nn.value == size
    assert want, "the oracle tree has no split"
    inv_h = 1.0 / scales[1]
    for node in range(size):
        t = nodes[node]
        if node in want:
            f, b, ml, gain, lid, rid, ls, rs = want[node]
            assert (t.flags & 1) == 0, node
            assert (t.feat, t.bin, bool(t.flags & 2)) == (f, b, ml), node
            assert np.float32(t.gain).view(np.uint32) == gain, node
            assert (t.left, t.right) == (lid, rid), node
            assert np.float32(nodes[lid].sum_hess) == np.float32(ls[1] * inv_h), node
            assert np.float32(nodes[rid].sum_hess) == np.float32(rs[1] * inv_h), node
        else:
            assert t.flags & 1, node
            rows = leaf_rows[node]
            assert np.all(delta[rows].view(np.uint32) == np.float32(t.leaf_value).view(np.uint32)), node
    assert sum(r.size for r in leaf_rows.values()) == n


@pytest.mark.parametrize("host_levels", [False, True])
def test_nonfinite_gradients_stop_training(fb, host_levels):
    """Gradients that overflow f32 (labels near the f32 maximum times a
    weight of 10) stop training with the reference's error, whether the
    quantizer scales come back to the host every round (host-grown levels)
    or stay on the device (device-grown trees, checked when the tree is
    collected)."""
    from ferrisboost_amd import _native as N

    rng = np.random.default_rng(5)
    n = 4096
    x = rng.normal(size=(n, 3)).astype(np.float32)
    y = np.where(np.arange(n) % 2 == 0, 3e38, -3e38).astype(np.float32)
    w = np.full(n, 10.0, np.float32)
    params = {"objective": "reg:squarederror", "max_depth": 3, "max_bin": 16,
              "hip_host_levels": host_levels}
    with pytest.raises(N.InputError, match="non-finite gradient"):
        fb.train(params, x, y, weight=w, num_boost_round=2)


@pytest.mark.parametrize("max_bin", [255, 256])
def test_plumbing_config_matches_oracle(fb, oracle, max_bin):
    X, y, params, _ = _synthetic("plumbing", 30_000)
    params = dict(params, max_bin=max_bin)
    rounds = 12
    om = oracle.train(X, y, oracle.make_params(n_rounds=rounds, **params))
    pm = fb.train(params, X, y, num_boost_round=rounds)
    assert_same_models(om, pm)
    assert np.array_equal(pm.train_margins(X.shape[0]), om.train_margins(X.shape[0]))


@pytest.mark.parametrize("max_bin, rate, n_rows", [(256, 0.5, 6_000), (64, 0.5, 6_000),
                                                    (256, 0.3, 6_001), (64, 0.3, 6_002),
                                                    (64, 0.8, 6_000)])
def test_wide_colsample_matches_oracle(fb, oracle, max_bin, rate, n_rows):
    """Column sampling over interleaved tiles of 16-bit (max_bin 256) and
    8-bit (64) cells: at rates 0.5 and 0.3 each tree's features are packed
    into fresh tiles (four rows a thread when the row count is a multiple of
    8, else one), at 0.8 the tiles are used as they are."""
    from ferrisboost_amd import datasets

    X, y, params, _ = datasets.wide_binary(n_rows, n_features=300)
    rounds = 6
    params = dict(params, max_depth=6, max_bin=max_bin, colsample_bytree=rate)
    om = oracle.train(X, y, oracle.make_params(n_rounds=rounds, **params))
    pm = fb.train(params, X, y, num_boost_round=rounds)
    assert_same_models(om, pm)


def test_lossguide_categorical_matches_oracle(fb, oracle):
    from ferrisboost_amd import datasets

    X, y, params, _ = datasets.widebin_cat(20_000, n_num=12, n_cat=4, n_codes=500)
    # one low-cardinality categorical column takes the one-hot path
    X[:, -1] = np.floor(X[:, -1]) % 3
    rounds = 5
    params = dict(params, max_leaves=31, max_bin=300)
    cat = [1 if t == "c" else 0 for t in params["feature_types"]]
    op = {k: v for k, v in params.items() if k != "feature_types"}
    om = oracle.train(X, y, oracle.make_params(n_rounds=rounds, **op), categorical=cat)
    pm = fb.train(params, X, y, num_boost_round=rounds)
    assert_same_models(om, pm)
    assert np.array_equal(pm.train_margins(X.shape[0]), om.train_margins(X.shape[0]))


@pytest.mark.parametrize("knobs", [
    {},                                             # device-grown, row walk (one bundle)
    {"hip_host_levels": True},                      # host-driven levels
    {"grow_policy": "lossguide", "max_leaves": 20},  # capped lossguide
    {"resident_blocks": 0},                         # everything streamed
    {"colsample_bytree": 0.6},                      # packed interleaved tiles
])
def test_full_byte_cells_match_oracle(fb, oracle, knobs):
    """max_bin 256 on continuous features without missing values: 256 bins a
    feature, stored as 8-bit cells in which every byte is a bin (no missing
    code); one feature with a NaN keeps 16-bit cells. Trees and margins equal
    the oracle's, whose bins are 16-bit as the reference's."""
    rng = np.random.default_rng(77)
    n, nf = 40_000, 20
    x = rng.normal(size=(n, nf)).astype(np.float32)
    x[5, 3] = np.nan  # feature 3 has a missing value: 16-bit cells
    y = (x[:, 0] + np.nan_to_num(x[:, 3]) * x[:, 7] - 0.5 * x[:, 12] + 0.3 * rng.normal(size=n)
         > 0).astype(np.float32)
    p = {"max_depth": 6, "eta": 0.3, "max_bin": 256}
    kw = dict(knobs)
    op = {k: v for k, v in dict(p, **kw).items() if not k.startswith("hip_") and
          k != "resident_blocks"}
    om = oracle.train(x, y, oracle.make_params(n_rounds=4, **op))
    pm = fb.train(dict(p, **kw), x, y, 4)
    assert_same_models(om, pm)
    assert np.array_equal(pm.train_margins(n).view(np.uint32), om.train_margins(n).view(np.uint32))
    # the bins reach 255: the last bin is a real one
    t = pm.trees()
    assert any((tr["is_leaf"] == 0).any() for tr in t)


@pytest.mark.parametrize("policy", ["lossguide", "depthwise"])
def test_tile_major_root_matches_oracle(fb, oracle, policy):
    """Many planar tiles sharing each row bundle (wide-bin numeric and
    categorical features, as C4): the root reads tile-major copies of the
    records in long chunks, the deeper levels the bundles."""
    from ferrisboost_amd import datasets

    X, y, params, _ = datasets.widebin_cat(150_000, n_num=40, n_cat=8, n_codes=300)
    params = dict(params, grow_policy=policy, max_depth=5, max_leaves=0 if policy ==
                  "depthwise" else 255)
    cat = [1 if t == "c" else 0 for t in params["feature_types"]]
    op = {k: v for k, v in params.items() if k != "feature_types"}
    om = oracle.train(X, y, oracle.make_params(n_rounds=3, **op), categorical=cat)
    pm = fb.train(params, X, y, num_boost_round=3)
    assert_same_models(om, pm)
    assert np.array_equal(pm.train_margins(X.shape[0]).view(np.uint32),
                          om.train_margins(X.shape[0]).view(np.uint32))


def test_depthwise_categorical_partition_path(fb, oracle):
    from ferrisboost_amd import datasets

    X, y, params, _ = datasets.widebin_cat(15_000, n_num=6, n_cat=3, n_codes=40)
    params = dict(params, grow_policy="depthwise", max_depth=5, max_leaves=0, max_bin=64,
                  max_cat_threshold=8)
    cat = [1 if t == "c" else 0 for t in params["feature_types"]]
    op = {k: v for k, v in params.items() if k != "feature_types"}
    om = oracle.train(X, y, oracle.make_params(n_rounds=4, **op), categorical=cat)
    pm = fb.train(params, X, y, num_boost_round=4)
    assert_same_models(om, pm)


@pytest.mark.parametrize("threshold", [2, 64, 1000])
def test_categorical_scan_directions_and_ties(fb, oracle, threshold):
    """Sorted-category prefix scans in both directions, up to every category
    (max_cat_threshold above the category count), with categories of equal
    weight: each category code repeats one of a few label patterns exactly,
    so weights and candidate gains tie."""
    rng = np.random.default_rng(71 + threshold)
    n, n_codes = 24_000, 300
    codes = rng.integers(0, n_codes, n)
    X = np.zeros((n, 3), np.float32)
    X[:, 0] = codes
    X[:, 1] = rng.standard_normal(n)
    X[:, 2] = rng.integers(0, 7, n)
    # four groups of categories by code % 4, two of them label-pure
    y = ((codes % 4 == 1) | ((codes % 4 == 2) & (X[:, 1] > 0))).astype(np.float32)
    X[rng.random(n) < 0.05, 0] = np.nan
    params = dict(objective="binary:logistic", max_depth=5, learning_rate=0.3, max_bin=512,
                  grow_policy="lossguide", max_leaves=24, max_cat_to_onehot=4,
                  max_cat_threshold=threshold, feature_types=["c", "q", "c"])
    cat = [1, 0, 1]
    op = {k: v for k, v in params.items() if k != "feature_types"}
    om = oracle.train(X, y, oracle.make_params(n_rounds=4, **op), categorical=cat)
    pm = fb.train(params, X, y, num_boost_round=4)
    assert_same_models(om, pm)
    assert np.array_equal(pm.train_margins(n), om.train_margins(n))


def test_shap_matches_oracle_and_is_additive(fb, oracle):
    X, y, params, _ = _synthetic("plumbing", 8_000)
    X[::7, 3] = np.nan
    rounds = 8
    om = oracle.train(X, y, oracle.make_params(n_rounds=rounds, **params))
    pm = fb.train(params, X, y, num_boost_round=rounds)
    assert_same_models(om, pm)
    rows = X[:2000]
    got = pm.predict(rows, pred_contribs=True)
    want = om.shap(rows)
    assert np.max(np.abs(got - want)) <= 1e-5
    margin = pm.predict(rows, output_margin=True).astype(np.float64)
    assert np.max(np.abs(got.astype(np.float64).sum(axis=1) - margin)) <= 1e-4


def _plan_for(N, model, n_rows, slots, budget, categorical=None):
    """The plan the trainer makes for this model's shape under a budget."""
    vals, offs = model.cuts()
    nb = (np.diff(offs.astype(np.int64)) + 1).astype(np.uint32)
    w = np.where(nb > 255, 2, 1).astype(np.uint8)
    cat = None if categorical is None else np.ascontiguousarray(categorical, np.uint8)
    shape = N.Shape(nb.size, N.ptr(w), N.ptr(nb), N.ptr(cat))
    cfg = N.Config()
    cfg.memory_budget = budget
    cfg.hist_slots = slots
    out = N.Plan()
    N.check_hip(N.hip().fbh_plan_memory(n_rows, C.byref(shape), C.byref(cfg), 0, C.byref(out)))
    return out


def _streaming_budgets(N, model, n_rows, slots, categorical=None):
    """A budget keeping some tiles resident and one keeping none."""
    big = _plan_for(N, model, n_rows, slots, 1 << 40, categorical)
    assert big.n_tiles >= 3, big.n_tiles
    lo = big.fixed_bytes
    some = none = None
    for step in range(0, 4000):
        b = lo + step * (1 << 18)
        try:
            p = _plan_for(N, model, n_rows, slots, b, categorical)
        except ValueError:
            continue
        if p.resident_tiles == 0 and none is None:
            none = b
        if 0 < p.resident_tiles < p.n_tiles:
            some = b
            break
    assert some and none, (some, none)
    return some, none


@pytest.mark.parametrize("kind", ["depthwise", "lossguide_categorical"])
def test_streaming_matches_resident_and_oracle(fb, oracle, N, kind):
    """gpu_memory_budget forces tiles to stream from pinned host memory
    (record windows for histograms, columns for partitions): the models are
    byte-identical to the all-resident run and to the CPU oracle, and the
    context stays within the budget."""
    rng = np.random.default_rng(61 if kind == "depthwise" else 62)
    n = 120_007
    if kind == "depthwise":
        nf = 40
        x = rng.normal(size=(n, nf)).astype(np.float32)
        x[rng.random((n, nf)) < 0.04] = np.nan
        y = (np.nan_to_num(x[:, 0]) - np.nan_to_num(x[:, 7]) * np.nan_to_num(x[:, 31])
             + 0.3 * rng.normal(size=n) > 0).astype(np.float32)
        p = {"n_rounds": 4, "max_depth": 6, "eta": 0.3, "max_bin": 255}
        slots, cat = 32, None
    else:
        nf = 24
        x = rng.random((n, nf)).astype(np.float32)
        x[:, 18:] = rng.integers(0, 300, size=(n, 6))
        x[rng.random((n, nf)) < 0.05] = np.nan
        y = (np.nan_to_num(x[:, 0]) + (np.nan_to_num(x[:, 20]) % 7 == 3) + 0.1 * rng.normal(size=n)
             ).astype(np.float32)
        p = {"n_rounds": 3, "max_bin": 1024, "grow_policy": "lossguide", "max_leaves": 31,
             "objective": "reg:squarederror", "eta": 0.3}
        slots = 33
        cat = np.array([0] * 18 + [1] * 6, np.uint8)
    pp = product_params(p)
    if cat is not None:
        pp["feature_types"] = ["c" if c else "q" for c in cat]
    ref = fb.train(pp, x, y, num_boost_round=p["n_rounds"])
    assert ref.stats["resident_tiles"] == ref.stats["n_tiles"]
    some, none = _streaming_budgets(N, ref, n, slots, cat)
    om = oracle.train(x, y, oracle.make_params(**p), categorical=cat)
    for budget in (some, none):
        st = fb.train(dict(pp, gpu_memory_budget=budget), x, y, num_boost_round=p["n_rounds"])
        assert st.stats["budget_bytes"] == budget
        assert st.stats["resident_tiles"] < st.stats["n_tiles"]
        assert st.stats["streamed_bytes"] > 0
        assert st.stats["device_bytes"] <= budget
        assert_same_models(ref, st)
        assert_same_models(om, st)
        assert np.array_equal(st.train_margins(n).view(np.uint32), ref.train_margins(n).view(np.uint32))
