"""GPU: column sampling beyond colsample_bytree, feature weights and
starting margins on the device path, equal to the oracle bit for bit.

* colsample_bylevel / colsample_bynode (NestedSampler, src/data/colsample.rs:
  203-286): each node's split scan masked to its own feature set
  (split_cached_features_masked, src/backend/cuda/histogram.cu:482-494),
  depthwise and lossguide, with and without colsample_bytree, one output and
  several;
* feature_weights (src/data/colsample.rs:119-195) in each sampler;
* base_margin (src/training/mod.rs:1831-1852, 2605-2616): every row starts
  at its own margin, one output and several;
* the reference's train() argument order: fb.train(p, X, y, 100) trains
  100 rounds.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import assert_same_models

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fb():
    import ferrisboost_amd as fb
    from ferrisboost_amd import _native as N

    if not N.device_available(0):
        pytest.fail("no gfx950 device: the GPU suite needs an MI355X")
    return fb


def _data(n=20_000, nf=12, seed=3, cat=False):
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(n, nf)).astype(np.float32)
    x[rng.random((n, nf)) < 0.05] = np.nan
    if cat:
        x[:, nf - 1] = rng.integers(0, 9, n).astype(np.float32)
    z = np.nan_to_num(x) @ rng.normal(size=nf) + 0.5 * rng.normal(size=n)
    return x, z.astype(np.float32)


W = [1.0, 0.0, 2.0, 3.0, 1.0, 0.5, 4.0, 1.0, 2.0, 1.0, 0.0, 3.0]

CASES = {
    "bylevel": dict(colsample_bylevel=0.5),
    "bynode": dict(colsample_bynode=0.5),
    "tree_level_node": dict(colsample_bytree=0.8, colsample_bylevel=0.7, colsample_bynode=0.6),
    "lossguide_bynode": dict(colsample_bynode=0.5, grow_policy="lossguide", max_leaves=20),
    "lossguide_uncapped_bylevel": dict(colsample_bylevel=0.5, grow_policy="lossguide"),
    "weights_bytree": dict(colsample_bytree=0.5, feature_weights=W),
    "weights_nested": dict(colsample_bylevel=0.6, colsample_bynode=0.5, feature_weights=W),
    "weights_equal": dict(colsample_bytree=0.5, colsample_bynode=0.5, feature_weights=[2.0] * 12),
    "categorical_bynode": dict(colsample_bynode=0.5, cat=True),
    "multiclass_bylevel": dict(colsample_bylevel=0.5, objective="multi:softprob", num_class=3),
    "quantile_bynode": dict(colsample_bynode=0.5, objective="reg:quantileerror",
                            quantile_alpha=[0.2, 0.8]),
}


def _labels(obj, z):
    if obj == "binary:logistic":
        return (z > 0).astype(np.float32)
    if obj.startswith("multi:"):
        return np.digitize(z, np.quantile(z, [1 / 3, 2 / 3])).astype(np.float32)
    return z


@pytest.mark.parametrize("name", list(CASES))
def test_sampled_columns_equal_the_oracle(fb, oracle, name):
    kw = dict(CASES[name])
    cat = kw.pop("cat", False)
    x, z = _data(cat=cat)
    obj = kw.pop("objective", "binary:logistic")
    y = _labels(obj, z)
    p = dict(max_depth=6, eta=0.3, max_bin=64, seed=11, objective=obj, **kw)
    rounds = 6
    types = ["q"] * 11 + ["c"] if cat else None
    om = oracle.train(x, y, oracle.make_params(n_rounds=rounds, cols_per_block=4, nthread=4, **p),
                      categorical=None if not cat else np.array([t == "c" for t in types], np.uint8))
    pm = fb.train(dict(p, **({"feature_types": types} if types else {})), x, y, rounds)
    assert_same_models(om, pm)
    n = y.size
    assert np.array_equal(pm.train_margins(n).view(np.uint32), om.train_margins(n).view(np.uint32))


@pytest.mark.parametrize("obj", ["binary:logistic", "reg:squarederror", "multi:softprob",
                                 "reg:quantileerror"])
def test_base_margin_equals_the_oracle(fb, oracle, obj):
    x, z = _data(seed=5)
    y = _labels(obj, z)
    k = 3 if obj.startswith("multi:") else (2 if obj == "reg:quantileerror" else 1)
    extra = {"num_class": 3} if k == 3 else ({"quantile_alpha": [0.3, 0.7]} if k == 2 else {})
    rng = np.random.default_rng(8)
    margin = rng.normal(scale=0.5, size=(y.size, k)).astype(np.float32)
    p = dict(max_depth=5, eta=0.3, max_bin=64, objective=obj, **extra)
    om = oracle.train(x, y, oracle.make_params(n_rounds=4, base_margin=margin.T.copy(), **p))
    pm = fb.train(p, x, y, 4, base_margin=margin if k > 1 else margin[:, 0])
    assert_same_models(om, pm)
    assert pm.base_score == om.base_score
    assert np.array_equal(pm.train_margins(y.size).view(np.uint32),
                          om.train_margins(y.size).view(np.uint32))


def test_positional_num_boost_round(fb):
    x, z = _data(n=3000)
    m = fb.train({"max_depth": 3}, x, (z > 0).astype(np.float32), 100)
    assert m.num_trees == 100
