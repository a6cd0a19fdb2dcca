"""GPU: reg:quantileerror on the device against the oracle's restatement of
Objective::quantile_scale / quantile_gradient (src/training/objective.rs:
1002-1160), the single-output round loop and, for several quantile_alpha,
train_multiclass_rounds (src/training/mod.rs:2578-2890): byte-identical trees
and training margins in gpu_math="exact" (the scale's terms summed on the
host in row order in double, tanh as glibc's tanhf restated), over one and
several alphas, weights, sampling, lossguide, categorical features, a given
base_score and host-driven levels; the device tanhf equal to the host's on
all 2^32 inputs; gpu_math="fast" deterministic; sorted multi-quantile
predictions, JSON round trips and per-quantile TreeSHAP."""

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


def _data(n, seed, n_feat=8, cat=False):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, n_feat)).astype(np.float32)
    x[rng.random((n, n_feat)) < 0.05] = np.nan
    y = (np.nan_to_num(x[:, 0]) * 1.5 - np.nan_to_num(x[:, 1]) ** 2
         + rng.standard_exponential(n) * (1 + np.abs(np.nan_to_num(x[:, 2])))).astype(np.float32)
    types = None
    if cat:
        x[:, -1] = rng.integers(0, 12, n).astype(np.float32)
        y = (y + (x[:, -1] % 4)).astype(np.float32)
        types = ["q"] * (n_feat - 1) + ["c"]
    return x, y, types


CASES = {
    "median_depthwise": dict(n=6000, alpha=0.5, params={"max_depth": 6}),
    "upper_weighted": dict(n=5000, alpha=0.9, weights=True, params={"max_depth": 5}),
    "lower_sampled": dict(n=8000, alpha=0.1, params={"max_depth": 6, "subsample": 0.7,
                                                     "colsample_bytree": 0.6, "seed": 11}),
    "lossguide_uncapped": dict(n=5000, alpha=0.7, params={"grow_policy": "lossguide",
                                                          "max_depth": 5, "max_leaves": 0}),
    "lossguide_capped": dict(n=5000, alpha=0.3, params={"grow_policy": "lossguide",
                                                        "max_depth": 6, "max_leaves": 11}),
    "categorical": dict(n=6000, alpha=0.8, cat=True, params={"max_depth": 5}),
    "base_score": dict(n=3000, alpha=0.5, params={"max_depth": 4, "base_score": 0.25}),
    "host_levels": dict(n=4000, alpha=0.6, params={"max_depth": 5, "hip_host_levels": True}),
    "depth_zero": dict(n=2000, alpha=0.95, params={"max_depth": 0}),
    "three_alphas": dict(n=6000, alpha=[0.1, 0.5, 0.9], params={"max_depth": 5}),
    "alphas_weighted_sampled": dict(n=5000, alpha=[0.05, 0.5, 0.5, 0.95], weights=True,
                                    params={"max_depth": 4, "subsample": 0.8, "seed": 3}),
    # every output's scale sum is started by the first output's call: these take the
    # deferred leaf values (capped lossguide) and the host-driven levels with several alphas
    "alphas_lossguide_capped": dict(n=5000, alpha=[0.2, 0.5, 0.8],
                                    params={"grow_policy": "lossguide", "max_leaves": 11,
                                            "max_depth": 6}),
    "alphas_host_levels": dict(n=4000, alpha=[0.3, 0.7],
                               params={"max_depth": 4, "hip_host_levels": True}),
}


def _train_both(fb, oracle, case, rounds=4):
    spec = CASES[case]
    x, y, types = _data(spec["n"], seed=len(case), cat=spec.get("cat", False))
    w = (np.random.default_rng(5).uniform(0.3, 2.0, y.size).astype(np.float32)
         if spec.get("weights") else None)
    params = {"objective": "reg:quantileerror", "quantile_alpha": spec["alpha"], "eta": 0.3,
              "max_bin": 64, "min_child_weight": 0.5}
    params.update(spec["params"])
    pm = fb.train(dict(params, **({"feature_types": types} if types else {})), x, y, weight=w,
                  num_boost_round=rounds)
    op = {k: v for k, v in params.items() if not k.startswith("hip_")}
    cat = None if types is None else np.array([t == "c" for t in types], np.uint8)
    om = oracle.train(x, y, oracle.make_params(n_rounds=rounds, nthread=1, **op), weights=w,
                      categorical=cat)
    return x, y, w, pm, om


def test_device_tanh_equals_the_host_libm_on_every_float(fb, oracle):
    from ferrisboost_amd import _native as N
    import ctypes as C

    got = C.c_uint64()
    N.check_hip(N.hip().fbh_tanh_checksum(0, 0, 1 << 32, C.byref(got)))
    want = oracle.lib().orc_tanh_checksum(0, 1 << 32, 16)
    assert got.value == want


@pytest.mark.parametrize("case", list(CASES))
def test_quantile_equals_oracle(fb, oracle, case):
    x, y, w, pm, om = _train_both(fb, oracle, case)
    alphas = np.atleast_1d(np.asarray(CASES[case]["alpha"], np.float32))
    k = alphas.size
    assert pm.num_class == k and om.num_outputs == k
    assert pm.quantile_alpha == [float(a) for a in alphas]
    if k > 1:
        assert np.array_equal(pm.class_margins().view(np.uint32),
                              om.class_margins().view(np.uint32))
    else:
        assert np.float32(pm.base_score).view(np.uint32) == np.float32(om.base_score).view(np.uint32)
    assert_same_models(om, pm)
    assert np.array_equal(pm.train_margins(y.size).view(np.uint32),
                          om.train_margins(y.size).view(np.uint32))
    pred = pm.predict(x, output_margin=True)
    assert pred.shape == ((y.size, k) if k > 1 else (y.size,))
    assert np.array_equal(pred.view(np.uint32), om.predict_margin(x).view(np.uint32))


@pytest.mark.parametrize("alpha", [0.75, [0.2, 0.5, 0.8]])
def test_full_size_first_rounds_equal_oracle(fb, oracle, alpha):
    """400k rows: the host's serial scale sums (one output, or several summed side by
    side on host threads over chunked downloads) and the device pairs at size."""
    x, y, _ = _data(400_000, seed=21, n_feat=12)
    params = {"objective": "reg:quantileerror", "quantile_alpha": alpha, "max_depth": 8,
              "eta": 0.1, "max_bin": 255}
    pm = fb.train(params, x, y, num_boost_round=3)
    om = oracle.train(x, y, oracle.make_params(n_rounds=3, nthread=8, **params))
    assert_same_models(om, pm)
    assert np.array_equal(pm.train_margins(y.size).view(np.uint32),
                          om.train_margins(y.size).view(np.uint32))


def test_fast_mode_is_deterministic_and_close(fb):
    x, y, _ = _data(50_000, seed=3)
    p = {"objective": "reg:quantileerror", "quantile_alpha": [0.2, 0.8], "max_depth": 6,
         "gpu_math": "fast"}
    a = fb.train(p, x, y, num_boost_round=8)
    b = fb.train(p, x, y, num_boost_round=8)
    assert a.to_json() == b.to_json()
    exact = fb.train(dict(p, gpu_math="exact"), x, y, num_boost_round=8)
    pa = a.predict(x, output_margin=True)
    pe = exact.predict(x, output_margin=True)
    assert np.abs(pa - pe).max() < 1e-3 * max(1.0, np.abs(pe).max())


def test_predictions_sorted_json_round_trip_and_coverage(fb, oracle):
    x, y, _, pm, _ = _train_both(fb, oracle, "three_alphas", rounds=30)
    m = pm.predict(x, output_margin=True)
    v = pm.predict(x)
    assert v.shape == m.shape == (y.size, 3)
    assert np.array_equal(v, np.sort(m, axis=1))
    assert np.array_equal(v.view(np.uint32), pm.predict(x, use_gpu=False).view(np.uint32))
    cover = [(y <= v[:, j]).mean() for j in range(3)]
    assert abs(cover[0] - 0.1) < 0.12 and abs(cover[1] - 0.5) < 0.12 and abs(cover[2] - 0.9) < 0.12
    text = pm.to_json()
    assert '"num_target":"3"' in text and '"num_class":"0"' in text
    assert '"quantile_alpha":"[0.1,0.5,0.9]"' in text
    back = fb.Model.from_json(text)
    assert back.quantile_alpha == pm.quantile_alpha and back.num_class == 3
    assert back.to_json() == text
    assert np.array_equal(back.predict(x).view(np.uint32), v.view(np.uint32))
    single = fb.Model.from_json(_train_both(fb, oracle, "median_depthwise")[3].to_json())
    assert single.quantile_alpha == [0.5] and single.num_class == 1


def test_per_quantile_shap_adds_up(fb, oracle):
    x, y, _, pm, _ = _train_both(fb, oracle, "three_alphas")
    xs = x[:400]
    phi = pm.predict(xs, pred_contribs=True)
    assert phi.shape == (400, 3, x.shape[1] + 1)
    assert np.allclose(phi.sum(axis=2), pm.predict(xs, output_margin=True), atol=1e-4)
    trees = pm.trees()
    for c in range(3):
        om = oracle.model_from_nodes(trees[c::3], np.zeros(0, np.uint32), "reg:squarederror",
                                     float(pm.class_margins()[c]))
        assert np.array_equal(phi[:, c, :].view(np.uint32), om.shap(xs).view(np.uint32))


def test_quantile_parameters_are_checked(fb):
    x, y, _ = _data(300, seed=1)
    with pytest.raises(ValueError, match="needs quantile_alpha"):
        fb.train({"objective": "reg:quantileerror"}, x, y, num_boost_round=1)
    with pytest.raises(ValueError, match="ascending"):
        fb.train({"objective": "reg:quantileerror", "quantile_alpha": [0.6, 0.4]}, x, y,
                 num_boost_round=1)
