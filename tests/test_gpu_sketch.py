"""GPU: the quantile sketch on the device (fbh_sketch_create / push_rows /
cuts) gives the host sketch's cuts bit for bit (SketchSet, FeatureSketch,
src/data/sketch.rs:72-560; the product's host sketch equals the oracle's,
tests/test_host.py): max_bin from 2 to 1024, row counts around the batch
size and with many batches, NaN, +-inf, heavy duplicates, ties across
batches, rows pushed in uneven pieces, categorical codes and their errors,
zeros of both signs, and whole trainings
sketched on the device against the host sketch."""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from helpers import assert_same_models

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def N():
    from ferrisboost_amd import _native as N

    if not N.device_available(0):
        pytest.fail("no gfx950 device: the GPU suite needs an MI355X")
    return N


def _host(N, x, max_bin, cat=None):
    n, nf = x.shape
    cap = sum(65534 if (cat is not None and cat[f]) else max(max_bin, 2) for f in range(nf))
    vals = np.zeros(cap + 1, np.float32)
    offs = np.zeros(nf + 1, np.uint32)
    c = None if cat is None else np.ascontiguousarray(cat, np.uint8)
    N.check_train(N.train_lib().fbt_sketch_cuts(N.ptr(x), n, nf, max_bin, None, N.ptr(c),
                                                N.ptr(vals), N.ptr(offs)))
    return vals[: offs[-1]].copy(), offs


def _device(N, x, max_bin, cat=None, pieces=None):
    L = N.hip()
    n, nf = x.shape
    c = None if cat is None else np.ascontiguousarray(cat, np.uint8)
    h = C.c_void_p()
    N.check_hip(L.fbh_sketch_create(0, n, nf, max_bin, N.ptr(c), 0, C.byref(h)))
    try:
        bounds = [0, n] if pieces is None else [0, *pieces, n]
        for a, b in zip(bounds[:-1], bounds[1:]):
            part = np.ascontiguousarray(x[a:b])
            N.check_hip(L.fbh_sketch_push_rows(h, N.ptr(part), b - a))
        cap = sum(65533 if (cat is not None and cat[f]) else max(max_bin - 1, 0)
                  for f in range(nf))
        vals = np.zeros(cap + 1, np.float32)
        offs = np.zeros(nf + 1, np.uint32)
        host = np.zeros(max(nf, 1), np.uint8)
        N.check_hip(L.fbh_sketch_cuts(h, N.ptr(vals), cap, N.ptr(offs), N.ptr(host)))
        return vals[: offs[-1]].copy(), offs, host[:nf]
    finally:
        L.fbh_sketch_destroy(h)


def _both_zero_signs(col):
    z = col[col == 0]
    return bool(np.signbit(z).any() and not np.signbit(z).all())


def _same(N, x, max_bin, cat=None, pieces=None):
    """Device cuts equal the host's for every feature the device decides;
    a feature it leaves to the host holds both zero signs and a zero cut."""
    x = np.ascontiguousarray(x, np.float32)
    hv, ho = _host(N, x, max_bin, cat)
    dv, do, flags = _device(N, x, max_bin, cat, pieces)
    for f in range(x.shape[1]):
        want = hv[ho[f]:ho[f + 1]]
        if flags[f]:
            assert do[f + 1] == do[f]
            assert _both_zero_signs(x[:, f]) and (want == 0).any(), f
            continue
        got = dv[do[f]:do[f + 1]]
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f
    return dv, do, flags


def _mixed(n, seed):
    """Columns of every kind the sketch meets."""
    rng = np.random.default_rng(seed)
    cols = [
        rng.standard_normal(n),
        rng.integers(0, 7, n),                                    # few distinct values
        rng.integers(0, 5000, n),                                 # ties across batches
        np.round(rng.standard_normal(n) * 30) + 0.0,              # heavy duplicates
        np.where(rng.random(n) < 0.3, np.nan, rng.random(n)),    # missing values
        np.where(rng.random(n) < 0.02, np.inf, rng.standard_exponential(n)),
        np.where(rng.random(n) < 0.02, -np.inf, rng.lognormal(0, 4, n)),
        np.full(n, np.nan),                                       # no value at all
        np.full(n, 2.5),                                          # one value
        rng.standard_normal(n) * 1e-39,                           # subnormals
        np.where(rng.random(n) < 0.5, 3e38, -3e38),               # midpoints overflow
    ]
    return np.stack([np.asarray(c, np.float64) for c in cols], axis=1).astype(np.float32)


@pytest.mark.parametrize("max_bin", [2, 3, 16, 255, 256, 1024])
@pytest.mark.parametrize("n", [1, 31, 4080, 4081, 8161, 61_237])
def test_device_sketch_equals_host_sketch(N, max_bin, n):
    _same(N, _mixed(n, n + max_bin), max_bin)


@pytest.mark.parametrize("max_bin", [4, 255])
def test_many_batches_and_uneven_pushes(N, max_bin):
    """max_bin 4 puts 64 values in a batch: 300k rows make 4688 batches, 13
    levels of merges and every set bit of the batch count in the collapse."""
    x = _mixed(300_000, 5 + max_bin)
    one = _same(N, x, max_bin)
    pieces = _same(N, x, max_bin, pieces=[1, 64, 65, 100_003, 100_004, 299_999])
    assert np.array_equal(one[0].view(np.uint32), pieces[0].view(np.uint32))
    assert np.array_equal(one[1], pieces[1])


def test_device_sketch_equals_oracle(N, oracle):
    x = _mixed(20_011, 3)
    for max_bin in (16, 256):
        dv, do, _ = _same(N, x, max_bin)
        ov, oo = oracle.sketch_cuts(x, max_bin)
        assert np.array_equal(do, oo)
        assert np.array_equal(dv.view(np.uint32), ov.view(np.uint32))


def test_categorical_codes_and_invalid_codes(N):
    rng = np.random.default_rng(11)
    n = 50_000
    x = np.stack([rng.standard_normal(n), rng.integers(0, 700, n),
                  np.where(rng.random(n) < 0.2, np.nan, rng.integers(0, 9, n)),
                  np.full(n, np.nan)], axis=1).astype(np.float32)
    cat = np.array([0, 1, 1, 1], np.uint8)
    dv, do, _ = _same(N, x, 256, cat)
    assert do[2] - do[1] == x[:, 1].max()  # codes 1..max_code
    for bad in (-1.0, 2.5, 65534.0):
        y = x.copy()
        y[777, 2] = bad
        with pytest.raises(N.InputError, match="categorical feature #2 contains a value"):
            _device(N, y, 256, cat)
    y = x.copy()
    y[5, 1] = 65533.0
    _same(N, y, 256, cat)


def test_both_zero_signs(N):
    """Zeros of both signs form one entry whose sign only a zero cut shows:
    low-cardinality data (midpoint cuts) and a zero never chosen are decided
    on the device; a mass of mixed zeros chosen as a cut goes to the host."""
    rng = np.random.default_rng(2)
    n = 30_000
    a = np.round(rng.standard_normal(n) * 3).astype(np.float32)       # midpoint cuts
    z = np.where(rng.random(n) < 0.3, np.round(rng.standard_normal(n)) * 0.0,
                 rng.standard_normal(n)).astype(np.float32)            # zero is a cut
    b = (rng.standard_normal(n) + 3.0).astype(np.float32)             # zero in the tail
    b[::997] = 0.0
    b[1::997] = -0.0                                                   # zero not a cut
    c = np.abs(a)                                                      # +0.0 only
    m = np.where(rng.random(n) < 0.3, np.float32(-0.0),
                 rng.standard_normal(n)).astype(np.float32)            # -0.0 only, a cut
    x = np.ascontiguousarray(np.stack([a, z, b, c, m], axis=1))
    assert all(_both_zero_signs(x[:, f]) for f in (0, 1, 2))
    dv, do, flags = _same(N, x, 64)
    assert flags.tolist() == [0, 1, 0, 0, 0]
    cut = dv[do[4]:do[5]]
    assert ((cut == 0) & np.signbit(cut)).any()  # a -0.0 cut decided on the device


def test_pushing_past_the_created_rows_is_an_input_error(N):
    L = N.hip()
    x = np.zeros((10, 2), np.float32)
    h = C.c_void_p()
    N.check_hip(L.fbh_sketch_create(0, 5, 2, 16, None, 0, C.byref(h)))
    try:
        with pytest.raises(N.InputError, match="more rows"):
            N.check_hip(L.fbh_sketch_push_rows(h, N.ptr(x), 10))
    finally:
        L.fbh_sketch_destroy(h)
    assert L.fbh_sketch_device_bytes(10, 2, 2048, None) == 0
    assert L.fbh_sketch_fits(0, 10, 2, 2048, None, 0) == 0
    assert L.fbh_sketch_fits(0, 10, 2, 256, None, 0) == 1


@pytest.mark.parametrize("case", ["narrow", "widebin", "zero_signs"])
def test_device_sketched_training_equals_host_sketched(case):
    import ferrisboost_amd as fb
    from ferrisboost_amd import datasets

    if case == "narrow":
        X, y, params, _ = datasets.narrow_binary(80_001)
        params = dict(params, max_bin=255)
    elif case == "widebin":
        X, y, params, _ = datasets.widebin_cat(60_000, n_num=12, n_cat=4, n_codes=300)
        params = dict(params, max_leaves=0, max_depth=6)
    else:
        X, y, params, _ = datasets.plumbing(30_000)
        X[:, 2] = np.round(X[:, 2] * 3)  # both zero signs: sketched on the host
    rounds = 4
    dev = fb.train(params, X, y, num_boost_round=rounds)
    host = fb.train(dict(params, hip_host_sketch=True), X, y, num_boost_round=rounds)
    assert dev.stats["device_sketch"] == 1 and host.stats["device_sketch"] == 0
    assert_same_models(host, dev)
    assert dev.to_json() == host.to_json()
    weighted = fb.train(params, X, y, num_boost_round=1, weight=np.ones(y.size, np.float32))
    assert weighted.stats["device_sketch"] == 0


@pytest.mark.parametrize("workload", ["narrow", "widebin"])
def test_full_size_device_sketch_equals_host(N, workload):
    """The cuts of the 10.5M x 28 narrow matrix at max_bin 255 and of the
    2M x 100 wide-bin matrix (80 numeric with NaN, 20 categorical) at 1024."""
    from ferrisboost_amd import datasets

    if workload == "narrow":
        X, _, params, _ = datasets.narrow_binary()
        cat = None
    else:
        X, _, params, _ = datasets.widebin_cat()
        cat = np.array([t == "c" for t in params["feature_types"]], np.uint8)
    _same(N, X, params["max_bin"], cat)


def test_device_sketch_in_the_exact_regime_equals_exact_rank_cuts(N):
    """The exact-summary regime of tests/test_sketch_pins.py on the device:
    D distinct values with max_bin < D <= 16 * max_bin, so the cuts are fixed
    by the exact ranks (numpy's unique counts), in several batch orders."""
    from test_sketch_pins import EXACT, _exact_case, expected_cuts

    for case in EXACT:
        max_bin, d, n, order, weighted = case
        if weighted:
            continue  # weighted rows are sketched on the host
        col, _ = _exact_case(*case, seed=d)
        want = expected_cuts(col, None, max_bin)
        dv, do, flags = _device(N, col.reshape(-1, 1), max_bin)
        assert not flags[0]
        assert np.array_equal(dv.view(np.uint32), want.view(np.uint32)), case
