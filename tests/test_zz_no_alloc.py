"""fbh_shap_contribs_noalloc: the explanation entry point that allocates no
device memory, checked through the C ABI against fbh_shap_contribs (same
kernels, bit for bit) on two calls in a row, the second smaller, plus the
size limit."""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from helpers import product_params

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    from ferrisboost_amd import _native as N

    if not N.device_available(0):
        pytest.fail("no gfx950 device: the GPU suite needs an MI355X")
    return N


def _flat_model(N, model, n_features, bias):
    """fbh_shap_model_create arguments from a trained model's trees."""
    trees = model.trees()
    words = model.cat_words()
    nodes = np.concatenate(trees)
    offs = np.concatenate([[0], np.cumsum([t.size for t in trees])]).astype(np.uint32)
    cols = {
        "feat": np.ascontiguousarray(nodes["feat"], np.uint32),
        "cond": np.ascontiguousarray(nodes["split_cond"], np.float32),
        "left": np.ascontiguousarray(nodes["left"], np.int32),
        "right": np.ascontiguousarray(nodes["right"], np.int32),
        "dl": np.ascontiguousarray(nodes["default_left"], np.uint8),
        "leaf": np.ascontiguousarray(nodes["is_leaf"], np.uint8),
        "val": np.ascontiguousarray(nodes["leaf_value"], np.float32),
        "hess": np.ascontiguousarray(nodes["sum_hess"], np.float32),
        "coff": np.ascontiguousarray(nodes["cat_begin"], np.uint32),
        "clen": np.ascontiguousarray(nodes["cat_len"], np.uint32),
        "words": np.ascontiguousarray(words if words.size else np.zeros(1, np.uint32), np.uint32),
    }
    h = C.c_void_p()
    N.check_hip(N.hip().fbh_shap_model_create(
        0, len(trees), N.ptr(offs), N.ptr(cols["feat"]), N.ptr(cols["cond"]),
        N.ptr(cols["left"]), N.ptr(cols["right"]), N.ptr(cols["dl"]), N.ptr(cols["leaf"]),
        N.ptr(cols["val"]), N.ptr(cols["hess"]), N.ptr(cols["coff"]), N.ptr(cols["clen"]),
        N.ptr(cols["words"]), int(words.size), n_features, float(bias), C.byref(h)))
    return h


def test_noalloc_contribs_equal_the_allocating_entry_point(lib):
    import ferrisboost_amd as fb

    N = lib
    rng = np.random.default_rng(91)
    n, nf = 30_000, 40
    x = rng.normal(size=(n, nf)).astype(np.float32)
    x[rng.random((n, nf)) < 0.05] = np.nan
    y = (np.nan_to_num(x[:, 0]) - np.nan_to_num(x[:, 3]) * np.nan_to_num(x[:, 9]) > 0)
    m = fb.train(product_params({"max_depth": 6, "eta": 0.3}), x, y.astype(np.float32),
                 num_boost_round=12)
    h = _flat_model(N, m, nf, m.base_margin)
    try:
        # 32 MiB of scratch hold 102,297 rows of 40 features (328 bytes a
        # row): the first call needs two batches, the second (smaller) one.
        big = np.concatenate([x, x[::-1], x, x[::-1]])
        for rows in (big, x[5000:5000 + 7001]):
            rows = np.ascontiguousarray(rows)
            k = rows.shape[0]
            margin = np.linspace(-1, 1, k).astype(np.float32)
            for mg in (None, margin):
                want = np.zeros((k, nf + 1), np.float32)
                got = np.full((k, nf + 1), np.nan, np.float32)
                # the entry point under test runs first on a fresh model, so
                # no launch of the allocating one has prepared anything for it
                N.check_hip(N.hip().fbh_shap_contribs_noalloc(h, N.ptr(rows), k, N.ptr(mg),
                                                              N.ptr(got)))
                N.check_hip(N.hip().fbh_shap_contribs(h, N.ptr(rows), k, N.ptr(mg), N.ptr(want)))
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (k, mg is None)
    finally:
        N.hip().fbh_shap_model_destroy(h)


def test_noalloc_rejects_rows_wider_than_its_scratch(lib):
    """A row that cannot fit the fixed scratch is an input error before any
    device work."""
    N = lib
    nf = (32 << 20) // 8  # 8 * nf + 8 bytes a row exceed the scratch
    offs = np.array([0, 1], np.uint32)
    one = lambda dt, v: np.array([v], dt)  # noqa: E731
    h = C.c_void_p()
    N.check_hip(N.hip().fbh_shap_model_create(
        0, 1, N.ptr(offs), N.ptr(one(np.uint32, 0)), N.ptr(one(np.float32, 0.0)),
        N.ptr(one(np.int32, -1)), N.ptr(one(np.int32, -1)), N.ptr(one(np.uint8, 0)),
        N.ptr(one(np.uint8, 1)), N.ptr(one(np.float32, 0.5)), N.ptr(one(np.float32, 1.0)),
        None, None, None, 0, nf, 0.0, C.byref(h)))
    try:
        row = np.zeros((1, nf), np.float32)
        out = np.zeros((1, nf + 1), np.float32)
        with pytest.raises(ValueError, match="scratch"):
            N.check_hip(N.hip().fbh_shap_contribs_noalloc(h, N.ptr(row), 1, None, N.ptr(out)))
    finally:
        N.hip().fbh_shap_model_destroy(h)
