"""GPU prediction and explanation against the oracle, through the C ABI:
margins and probabilities (GpuPredictor), leaf ids, Saabas and SHAP
interaction values (GpuExplainModel), base margins, tree ranges, and a saved
model loaded back. (Device margins of the golden cases are checked by
test_gpu_parity.py::test_golden_training_is_bit_exact, whose predict() runs
on the device.)"""

from __future__ import annotations

import os

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


def _sigmoid(oracle, m):
    out = np.zeros_like(m)
    oracle.lib().orc_sigmoid(oracle._p(m), m.size, oracle._p(out))
    return out


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _trained(fb, oracle, seed, n=6000, nf=7, rounds=6, depth=5, categorical=False,
             objective="binary:logistic"):
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(n, nf)).astype(np.float32)
    x[rng.random((n, nf)) < 0.08] = np.nan
    cat = None
    if categorical:
        x[:, 2] = rng.integers(0, 40, size=n)
        x[:, 5] = rng.integers(0, 7, size=n)
        cat = np.zeros(nf, np.uint8)
        cat[[2, 5]] = 1
    y = (np.nan_to_num(x[:, 0]) + np.isin(x[:, 2], [1, 5, 9, 30]) - 0.5 * np.nan_to_num(x[:, 3])
         + 0.3 * rng.normal(size=n) > 0.2).astype(np.float32)
    p = {"n_rounds": rounds, "max_depth": depth, "eta": 0.3, "max_bin": 64, "objective": objective}
    pp = product_params(p)
    if cat is not None:
        pp["feature_types"] = ["c" if c else "q" for c in cat]
    om = oracle.train(x, y, oracle.make_params(**p), categorical=cat)
    pm = fb.train(pp, x, y, num_boost_round=rounds)
    assert_same_models(om, pm)
    return om, pm, x


@pytest.mark.parametrize("categorical", [False, True])
def test_margins_values_and_leaves_match_oracle(fb, oracle, categorical):
    om, pm, x = _trained(fb, oracle, 71 + categorical, categorical=categorical)
    rows = x.copy()
    rows[:50, 2] = -3.0   # unseen / negative codes
    rows[50:100, 2] = 1e9
    margin = pm.predict(rows, output_margin=True)
    assert np.array_equal(_bits(margin), _bits(om.predict_margin(rows)))
    prob = pm.predict(rows)
    assert np.array_equal(_bits(prob), _bits(_sigmoid(oracle, margin)))
    host = pm.predict(rows, use_gpu=False)
    assert np.array_equal(_bits(prob), _bits(host))
    leaf = pm.predict(rows, pred_leaf=True)
    assert leaf.shape == (rows.shape[0], pm.num_trees)
    assert np.array_equal(leaf, om.explain(rows, "leaf"))
    assert pm.predict(rows, pred_leaf=True, strict_shape=True).shape == (rows.shape[0], pm.num_trees, 1, 1)


@pytest.mark.parametrize("categorical", [False, True])
def test_saabas_matches_oracle(fb, oracle, categorical):
    om, pm, x = _trained(fb, oracle, 73 + categorical, categorical=categorical)
    rows = x[:3000]
    got = pm.predict(rows, pred_contribs=True, approx_contribs=True)
    want = om.explain(rows, "approx")
    assert got.shape == want.shape
    assert np.max(np.abs(got - want)) <= 1e-6
    margin = pm.predict(rows, output_margin=True).astype(np.float64)
    assert np.max(np.abs(got.astype(np.float64).sum(axis=1) - margin)) <= 1e-4


@pytest.mark.parametrize("categorical", [False, True])
def test_interactions_match_oracle(fb, oracle, categorical):
    om, pm, x = _trained(fb, oracle, 75 + categorical, nf=6, rounds=5, depth=4,
                         categorical=categorical)
    rows = x[:400]
    got = pm.predict(rows, pred_interactions=True)
    want = om.explain(rows, "interactions")
    assert got.shape == (rows.shape[0], 7, 7)
    assert np.max(np.abs(got - want)) <= 1e-5
    assert np.array_equal(got, np.transpose(got, (0, 2, 1)))
    shap = pm.predict(rows, pred_contribs=True)
    assert np.max(np.abs(got.sum(axis=2) - shap)) <= 1e-4
    assert pm.predict(rows[:3], pred_interactions=True, strict_shape=True).shape == (3, 1, 7, 7)


def test_base_margin_and_tree_ranges_match_oracle(fb, oracle):
    """A per-row base margin replaces the intercept; n_trees takes a prefix
    and iteration_range a slice of the trees (src/python/mod.rs:1993-2029)."""
    om, pm, x = _trained(fb, oracle, 77, rounds=8, categorical=True)
    rows = x[:2000]
    bm = np.linspace(-2, 2, rows.shape[0]).astype(np.float32)
    got = pm.predict(rows, output_margin=True, base_margin=bm)
    trees = om.trees()
    words = om.cat_words()
    acc = bm.copy()
    leaf = om.explain(rows, "leaf").astype(np.int64)
    for t, tr in enumerate(trees):
        acc = (acc + tr["leaf_value"][leaf[:, t]]).astype(np.float32)
    assert np.array_equal(_bits(got), _bits(acc))
    for kind, kw in (("contribs", {"pred_contribs": True}),
                     ("approx", {"pred_contribs": True, "approx_contribs": True})):
        g = pm.predict(rows, base_margin=bm, **kw)
        w = om.explain(rows, kind, margin=bm)
        assert np.max(np.abs(g - w)) <= 1e-5, kind
    # slices [b, e) against an oracle model of exactly those trees
    for b, e in ((0, 3), (2, 6), (5, 5), (0, 8)):
        if e == b:
            want = np.full(rows.shape[0], np.float32(om.base_margin), np.float32)
        else:
            sub = oracle.model_from_nodes(trees[b:e], words, "binary:logistic",
                                          float(om.base_score))
            want = sub.predict_margin(rows)
        if b == 0:
            got = pm.predict(rows, output_margin=True, n_trees=e)
        else:
            got = pm.predict(rows, output_margin=True, iteration_range=(b, e))
        assert np.array_equal(_bits(got), _bits(want)), (b, e)
        if e > b:
            g = pm.predict(rows[:300], pred_contribs=True, iteration_range=(b, e))
            assert np.max(np.abs(g - sub.shap(rows[:300]))) <= 1e-5, (b, e)


def test_saved_model_predicts_and_explains_identically(fb, oracle, tmp_path):
    """save_model -> load_model: same trees, margins and SHAP values bit for bit."""
    om, pm, x = _trained(fb, oracle, 79, rounds=10, depth=6, categorical=True)
    path = os.path.join(tmp_path, "m.json")
    pm.save_model(path)
    back = fb.Model.load_model(path)
    assert back.num_trees == pm.num_trees and back.objective == pm.objective
    for a, b in zip(pm.trees(), back.trees()):
        for f in ("feat", "split_cond", "left", "right", "default_left", "is_leaf", "leaf_value",
                  "gain", "sum_hess"):
            assert np.array_equal(a[f], b[f]), f
    rows = x[:3000]
    assert np.array_equal(_bits(back.predict(rows, output_margin=True)),
                          _bits(pm.predict(rows, output_margin=True)))
    assert np.array_equal(_bits(back.predict(rows, pred_contribs=True)),
                          _bits(pm.predict(rows, pred_contribs=True)))
    assert np.array_equal(back.predict(rows, pred_leaf=True), pm.predict(rows, pred_leaf=True))
    with open(path) as f:
        assert back.to_json() == f.read()


def test_squared_error_values_are_margins(fb, oracle):
    om, pm, x = _trained(fb, oracle, 81, objective="reg:squarederror")
    rows = x[:1000]
    assert np.array_equal(_bits(pm.predict(rows)), _bits(om.predict_margin(rows)))


@pytest.mark.parametrize("nf", [7, 222, 240, 300])
def test_prediction_kernels_by_row_width(fb, oracle, nf):
    """The row width picks the walk: up to 223 features four waves share the
    rows staged in LDS (and add each run of trees' leaf values in tree
    order), up to 255 one wave stages them, wider rows are read in place.
    Every one gives the oracle's margins and leaf ids, bit for bit, also for
    a row count that leaves a partial last block and more trees than one run
    of 32."""
    om, pm, x = _trained(fb, oracle, 90 + nf, n=3001, nf=nf, rounds=37, depth=4)
    margin = pm.predict(x, output_margin=True)
    assert np.array_equal(_bits(margin), _bits(om.predict_margin(x)))
    leaf = om.explain(x, "leaf").astype(np.int64)
    assert np.array_equal(pm.predict(x, pred_leaf=True), leaf)
    # a per-row base margin, then every tree's leaf in tree order (f32 adds)
    acc = np.linspace(-1, 1, x.shape[0]).astype(np.float32)
    got = pm.predict(x, output_margin=True, base_margin=acc.copy())
    for t, tr in enumerate(om.trees()):
        acc = (acc + tr["leaf_value"][leaf[:, t]]).astype(np.float32)
    assert np.array_equal(_bits(got), _bits(acc))
