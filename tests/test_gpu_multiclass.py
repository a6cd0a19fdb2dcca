"""GPU: multiclass training (multi:softprob / multi:softmax) on the device
against the oracle's restatement of train_multiclass_rounds
(src/training/mod.rs:2578-2850) and Objective::softmax_gradients
(src/training/objective.rs:1175-1219): byte-identical trees and training
margins in gpu_math="exact" (the device exp is glibc's expf restated), over
depthwise and lossguide growth, weights, sampling, categorical features, a
given base_score and host-driven levels; gpu_math="fast" deterministic;
predictions, probabilities and class indices, per-class TreeSHAP, JSON round
trips and round ranges."""

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


def _data(n, k, seed, n_feat=8, cat=False):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, n_feat)).astype(np.float32)
    x[rng.random((n, n_feat)) < 0.05] = np.nan
    score = np.stack([x[:, j % n_feat] * (1 + j) - 0.5 * np.nan_to_num(x[:, (j + 3) % n_feat])
                      for j in range(k)], axis=1)
    score += rng.gumbel(size=score.shape)
    y = np.nanargmax(np.nan_to_num(score, nan=-1e9), axis=1).astype(np.float32)
    types = None
    if cat:
        x[:, -1] = rng.integers(0, 12, n).astype(np.float32)
        y = np.where(x[:, -1] % 3 == 0, 0, y).astype(np.float32)
        types = ["q"] * (n_feat - 1) + ["c"]
    return x, y, types


CASES = {
    "softprob_depthwise": dict(n=6000, k=3, params={"max_depth": 6}),
    "softmax_weighted": dict(n=5000, k=4, weights=True,
                             params={"objective": "multi:softmax", "max_depth": 5}),
    "sampled": dict(n=8000, k=3, params={"max_depth": 6, "subsample": 0.7,
                                          "colsample_bytree": 0.6, "seed": 11}),
    "lossguide_uncapped": dict(n=5000, k=3, params={"grow_policy": "lossguide", "max_depth": 5,
                                                     "max_leaves": 0}),
    "lossguide_capped": dict(n=5000, k=3, params={"grow_policy": "lossguide", "max_depth": 6,
                                                   "max_leaves": 11}),
    "categorical": dict(n=6000, k=3, cat=True, params={"max_depth": 5}),
    "base_score": dict(n=3000, k=5, params={"max_depth": 4, "base_score": 0.25}),
    "host_levels": dict(n=4000, k=3, params={"max_depth": 5, "hip_host_levels": True}),
    "depth_zero": dict(n=2000, k=3, params={"max_depth": 0}),
}


def _train_both(fb, oracle, case):
    spec = CASES[case]
    x, y, types = _data(spec["n"], spec["k"], seed=len(case), cat=spec.get("cat", False))
    w = (np.random.default_rng(5).uniform(0.3, 2.0, y.size).astype(np.float32)
         if spec.get("weights") else None)
    params = {"objective": "multi:softprob", "num_class": spec["k"], "eta": 0.3,
              "max_bin": 64, "min_child_weight": 0.5}
    params.update(spec["params"])
    rounds = 4
    pm = fb.train(dict(params, **({"feature_types": types} if types else {})), x, y, weight=w,
                  num_boost_round=rounds)
    op = {k: v for k, v in params.items() if not k.startswith("hip_")}
    cat = None if types is None else np.array([t == "c" for t in types], np.uint8)
    om = oracle.train(x, y, oracle.make_params(n_rounds=rounds, nthread=1, **op), weights=w,
                      categorical=cat)
    return x, y, w, pm, om


@pytest.mark.parametrize("case", list(CASES))
def test_multiclass_equals_oracle(fb, oracle, case):
    x, y, w, pm, om = _train_both(fb, oracle, case)
    k = CASES[case]["k"]
    assert pm.num_class == k and om.num_outputs == k
    assert np.array_equal(pm.class_margins().view(np.uint32), om.class_margins().view(np.uint32))
    assert_same_models(om, pm)
    assert np.array_equal(pm.train_margins(y.size).view(np.uint32),
                          om.train_margins(y.size).view(np.uint32))
    pred = pm.predict(x, output_margin=True)
    assert pred.shape == (y.size, k)
    assert np.array_equal(pred.view(np.uint32), om.predict_margin(x).view(np.uint32))


def test_fast_mode_is_deterministic_and_close(fb):
    x, y, _ = _data(20_000, 4, seed=3)
    p = {"objective": "multi:softprob", "num_class": 4, "max_depth": 6, "gpu_math": "fast"}
    a = fb.train(p, x, y, num_boost_round=6)
    b = fb.train(p, x, y, num_boost_round=6)
    assert a.to_json() == b.to_json()
    exact = fb.train(dict(p, gpu_math="exact"), x, y, num_boost_round=6)
    pa, pe = a.predict(x), exact.predict(x)
    assert np.abs(pa - pe).max() < 1e-2
    assert (pa.argmax(1) == pe.argmax(1)).mean() > 0.99


def test_probabilities_classes_and_host_scoring(fb, oracle):
    x, y, _, pm, om = _train_both(fb, oracle, "softprob_depthwise")
    k = 3
    m = pm.predict(x, output_margin=True)
    assert np.array_equal(m.view(np.uint32), pm.predict(x, output_margin=True,
                                                        use_gpu=False).view(np.uint32))
    prob = pm.predict(x)
    assert prob.shape == (y.size, k)
    assert np.array_equal(prob.view(np.uint32), pm.predict(x, use_gpu=False).view(np.uint32))
    e = np.exp(m.astype(np.float64) - m.max(1, keepdims=True))
    assert np.allclose(prob, e / e.sum(1, keepdims=True), rtol=0, atol=1e-6)
    assert np.allclose(prob.sum(1), 1.0, atol=1e-6)
    sm = fb.Model.from_json(pm.to_json().replace('"multi:softprob"', '"multi:softmax"'))
    cls = sm.predict(x)
    assert cls.shape == (y.size,)
    assert np.array_equal(cls, m.argmax(1).astype(np.float32))


def test_json_round_trip_keeps_classes(fb, oracle):
    x, y, _, pm, _ = _train_both(fb, oracle, "softmax_weighted")
    text = pm.to_json()
    assert '"num_class":"4"' in text and '"multi:softmax"' in text
    assert '"tree_info":[0,1,2,3,0,1,2,3' in text
    back = fb.Model.from_json(text)
    assert back.num_class == 4
    assert np.array_equal(back.class_margins().view(np.uint32),
                          pm.class_margins().view(np.uint32))
    assert back.to_json() == text
    assert np.array_equal(back.predict(x, output_margin=True).view(np.uint32),
                          pm.predict(x, output_margin=True).view(np.uint32))


def test_round_range_and_base_margin(fb, oracle):
    x, y, _, pm, om = _train_both(fb, oracle, "softprob_depthwise")
    k = 3
    full = pm.predict(x, output_margin=True)
    two = pm.predict(x, output_margin=True, iteration_range=(0, 2))
    trees = pm.trees()
    want = np.tile(pm.class_margins(), (y.size, 1)).astype(np.float32)
    for t in range(2 * k):
        single = oracle.model_from_nodes([trees[t]], np.zeros(0, np.uint32), "reg:squarederror",
                                         0.0)
        want[:, t % k] += single.predict_margin(x)
    assert np.array_equal(two.view(np.uint32), want.view(np.uint32))
    # rows started from the first two rounds' margins, scored by the last two
    got = pm.predict(x, output_margin=True, iteration_range=(2, 4), base_margin=two)
    assert np.array_equal(got.view(np.uint32), full.view(np.uint32))


def test_per_class_shap_equals_the_oracle_and_adds_up(fb, oracle):
    x, y, _, pm, _ = _train_both(fb, oracle, "categorical")
    k = 3
    xs = x[:500]
    phi = pm.predict(xs, pred_contribs=True)
    assert phi.shape == (500, k, x.shape[1] + 1)
    margin = pm.predict(xs, output_margin=True)
    assert np.allclose(phi.sum(axis=2), margin, atol=1e-4)
    trees, words = pm.trees(), pm.cat_words()
    for c in range(k):
        ct = trees[c::k]
        # the class's own trees, category words renumbered from 0
        base = 0
        rebuilt = []
        all_words = []
        for t in range(len(trees)):
            if t % k != c:
                continue
            node = trees[t].copy()
            has = node["cat_len"] > 0
            for i in np.nonzero(has)[0]:
                b, ln = node["cat_begin"][i], node["cat_len"][i]
                all_words.append(words[b:b + ln])
                node["cat_begin"][i] = base
                base += ln
            rebuilt.append(node)
        cw = np.concatenate(all_words) if all_words else np.zeros(0, np.uint32)
        om = oracle.model_from_nodes(rebuilt, cw, "reg:squarederror",
                                     float(pm.class_margins()[c]))
        assert len(ct) == len(rebuilt)
        assert np.array_equal(phi[:, c, :].view(np.uint32), om.shap(xs).view(np.uint32))


def test_labels_outside_the_classes_are_value_errors(fb):
    x, y, _ = _data(500, 3, seed=1)
    for bad in (3.0, -1.0, 0.5):
        yy = y.copy()
        yy[10] = bad
        with pytest.raises(ValueError, match="integers in"):
            fb.train({"objective": "multi:softprob", "num_class": 3}, x, yy, num_boost_round=1)


def test_large_first_rounds_equal_oracle(fb, oracle):
    """2M rows x 12 features, 4 classes, depth 8: the softmax statistics and
    class pairs at size, against the oracle's first rounds."""
    x, y, _ = _data(2_000_000, 4, seed=41, n_feat=12)
    params = {"objective": "multi:softprob", "num_class": 4, "max_depth": 8, "eta": 0.1,
              "max_bin": 255}
    pm = fb.train(params, x, y, num_boost_round=2)
    om = oracle.train(x, y, oracle.make_params(n_rounds=2, nthread=8, **params))
    assert_same_models(om, pm)
    assert np.array_equal(pm.train_margins(y.size).view(np.uint32),
                          om.train_margins(y.size).view(np.uint32))
