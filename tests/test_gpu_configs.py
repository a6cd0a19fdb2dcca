"""GPU: every benchmark configuration at its stated size against the oracle
(or, for the streamed configuration, against the all-resident run).

  C1  100,000 x 28, depth 6, 100 rounds, max_bin 255 and 256 (u8 / u16)
  C2  10,500,000 x 28 narrow, depth 8: the first rounds against the oracle at
      max_bin 255 (u8) and 256 (u16); 500 rounds twice, exact and fast,
      identical run to run
  C3  400,000 x 2,000 wide, colsample_bytree 0.5: the first rounds
  C4  2,000,000 x 100 wide-bin categorical lossguide, max_leaves 255: the
      first rounds
  C5  50,000,000 x 200 under a 4 GiB budget: streamed models identical to the
      all-resident ones (max_bin 256 and 255), and TreeSHAP of the 100-tree
      depth-8 ensemble on 1M rows (20k rows against the oracle, additivity on
      all of them)
"""

from __future__ import annotations

import gc
import sys
import time
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from helpers import assert_same_models, uncaptured

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fb():
    import ferrisboost_amd as fb
    from ferrisboost_amd import _native as N

    if not N.device_available(0):
        pytest.fail("no gfx950 device: the GPU suite needs an MI355X")
    return fb


_T0 = time.time()


def _say(msg: str) -> None:
    """A progress line, shown at once (the long steps here run for minutes)."""
    with uncaptured():
        sys.stdout.write(f"[configs {time.time() - _T0:7.1f}s] {msg}\n")
        sys.stdout.flush()


def _oracle_params(oracle, params, rounds):
    p = {k: v for k, v in params.items() if k not in ("feature_types", "gpu_math")}
    return oracle.make_params(n_rounds=rounds, nthread=16, **p)


def _categorical(params):
    ft = params.get("feature_types")
    return None if ft is None else np.array([1 if t == "c" else 0 for t in ft], np.uint8)


def _same_margins(a, b, n):
    assert np.array_equal(a.train_margins(n).view(np.uint32), b.train_margins(n).view(np.uint32))


def _check_against_oracle(fb, oracle, X, y, params, rounds):
    cat = _categorical(params)
    _say(f"oracle: {X.shape[0]} x {X.shape[1]}, {rounds} rounds")
    om = oracle.train(X, y, _oracle_params(oracle, params, rounds), categorical=cat)
    _say("device")
    pm = fb.train(params, X, y, num_boost_round=rounds)
    assert_same_models(om, pm)
    n = y.size
    assert np.array_equal(pm.train_margins(n).view(np.uint32), om.train_margins(n).view(np.uint32))
    return pm


@pytest.mark.parametrize("max_bin", [255, 256])
def test_c1_plumbing_100k_100_rounds(fb, oracle, max_bin):
    from ferrisboost_amd import datasets

    X, y, params, extra = datasets.plumbing(100_000)
    assert extra["rounds"] == 100
    pm = _check_against_oracle(fb, oracle, X, y, dict(params, max_bin=max_bin), 100)
    assert pm.num_trees == 100


@pytest.fixture(scope="module")
def narrow():
    from ferrisboost_amd import datasets

    X, y, params, _ = datasets.narrow_binary(10_500_000)
    _say("narrow data generated")
    yield X, y, params
    del X, y
    gc.collect()


@pytest.mark.parametrize("max_bin", [255, 256])
def test_c2_narrow_first_rounds_match_oracle(fb, oracle, narrow, max_bin):
    X, y, params = narrow
    p = dict(params, max_bin=max_bin)
    pm = _check_against_oracle(fb, oracle, X, y, p, 3)
    assert pm.stats["n_tiles"] >= 2
    # the product's cuts are the oracle's (the sketch of every feature)
    vals, offs = oracle.sketch_cuts(X, max_bin)
    pv, po = pm.cuts()
    assert np.array_equal(po, offs) and np.array_equal(pv.view(np.uint32), vals.view(np.uint32))


@pytest.mark.parametrize("gpu_math", ["exact", "fast"])
def test_c2_narrow_500_rounds_are_repeatable(fb, narrow, gpu_math):
    X, y, params = narrow
    p = dict(params, max_bin=255, gpu_math=gpu_math)
    cuts = fb.sketch(X, 255)
    _say("sketched")
    a = fb.train(p, X, y, num_boost_round=500, cuts=cuts)
    _say(f"500 rounds in {a.stats['train_seconds']:.2f}s")
    b = fb.train(p, X, y, num_boost_round=500, cuts=cuts)
    assert a.num_trees == 500 and a.stats["device_trees"] == 500
    assert_same_models(a, b)
    _same_margins(a, b, y.size)


def test_c3_wide_first_rounds_match_oracle(fb, oracle):
    from ferrisboost_amd import datasets

    X, y, params, _ = datasets.wide_binary(400_000, 2000)
    try:
        pm = _check_against_oracle(fb, oracle, X, y, params, 2)
        used = {int(f) for t in pm.trees() for f in t["feat"][t["is_leaf"] == 0]}
        assert len(used) > 1
    finally:
        del X, y
        gc.collect()


def test_c4_widebin_lossguide_first_rounds_match_oracle(fb, oracle):
    from ferrisboost_amd import datasets

    X, y, params, _ = datasets.widebin_cat(2_000_000)
    try:
        pm = _check_against_oracle(fb, oracle, X, y, params, 2)
        t = pm.tree_nodes(0)
        # max_leaves 255 and the default max_depth 6 allow 64 leaves
        assert (t["is_leaf"] == 1).sum() == 64
        assert pm.cat_words().size > 0  # categorical splits were taken
    finally:
        del X, y
        gc.collect()


@pytest.fixture(scope="module")
def c5():
    from ferrisboost_amd import datasets

    _say("generating 50M x 200")
    X, y, params, _ = datasets.streaming(50_000_000, 200)
    _say("50M x 200 generated")
    yield X, y, params, {}
    del X, y
    gc.collect()


def _c5_cuts(fb, c5, max_bin):
    X, _, _, cache = c5
    if max_bin not in cache:
        cache[max_bin] = fb.sketch(X, max_bin)
        _say(f"sketched max_bin {max_bin}")
    return cache[max_bin]


@pytest.mark.parametrize("max_bin", [256, 255])
def test_c5_streamed_under_4gib_equals_resident(fb, c5, max_bin):
    """gpu_memory_budget = 4 GiB: most tiles stream from pinned host memory
    and the model is byte-identical to the all-resident run."""
    X, y, params, _ = c5
    p = dict(params, max_bin=max_bin)
    cuts = _c5_cuts(fb, c5, max_bin)
    res = fb.train(p, X, y, num_boost_round=3, cuts=cuts)
    _say(f"resident: setup {res.stats['setup_seconds']:.1f}s, 3 rounds {res.stats['train_seconds']:.2f}s")
    assert res.stats["resident_tiles"] == res.stats["n_tiles"]
    st = fb.train(dict(p, gpu_memory_budget=4 << 30), X, y, num_boost_round=3, cuts=cuts)
    _say(f"streamed: setup {st.stats['setup_seconds']:.1f}s, 3 rounds {st.stats['train_seconds']:.2f}s")
    assert st.stats["budget_bytes"] == 4 << 30 and st.stats["device_bytes"] <= 4 << 30
    assert st.stats["resident_tiles"] < st.stats["n_tiles"] and st.stats["streamed_bytes"] > 0
    assert_same_models(res, st)
    _same_margins(res, st, y.size)


@pytest.fixture(scope="module")
def c5_resident(fb, c5):
    """The configured C5 job, resident: 100 rounds at max_bin 256."""
    X, y, params, _ = c5
    assert params["max_bin"] == 256
    pm = fb.train(params, X, y, num_boost_round=100, cuts=_c5_cuts(fb, c5, params["max_bin"]))
    _say(f"resident: 100 trees in {pm.stats['train_seconds']:.2f}s")
    assert pm.stats["resident_tiles"] == pm.stats["n_tiles"]
    return pm


def test_c5_streamed_100_rounds_equal_resident(fb, c5, c5_resident, monkeypatch):
    """The whole C5 job as configured (100 rounds, max_bin 256: no value is
    missing, so 8-bit cells) under a 4 GiB budget: most tiles stream from
    pinned host memory at every level of every tree, and all 100 trees and
    the training margins equal the resident run's byte for byte."""
    X, y, params, _ = c5
    monkeypatch.setenv("FB_LOG_ROUNDS", "10")  # the library's progress line every 10 rounds
    _say("streamed: 100 rounds")
    with uncaptured():
        st = fb.train(dict(params, gpu_memory_budget=4 << 30), X, y, num_boost_round=100,
                      cuts=_c5_cuts(fb, c5, params["max_bin"]))
    _say(f"streamed: 100 rounds in {st.stats['train_seconds']:.1f}s, "
         f"{st.stats['resident_tiles']}/{st.stats['n_tiles']} tiles resident, "
         f"{st.stats['streamed_bytes'] / 1e9:.0f} GB streamed")
    assert st.stats["device_bytes"] <= 4 << 30
    assert st.stats["resident_tiles"] < st.stats["n_tiles"] and st.stats["streamed_bytes"] > 0
    assert_same_models(c5_resident, st)
    _same_margins(c5_resident, st, y.size)


def test_c5_shap_of_the_100_tree_ensemble(fb, oracle, c5, c5_resident):
    """TreeSHAP of the 100-tree depth-8 ensemble on 1M rows: the first 20k
    against the oracle (<= 1e-5), every row additive against the margin."""
    X, y, params, _ = c5
    pm = c5_resident
    assert pm.num_trees == 100
    rows = X[:1_000_000]
    phi = pm.predict(rows, pred_contribs=True)
    margin = pm.predict(rows, output_margin=True)
    assert np.max(np.abs(phi.astype(np.float64).sum(axis=1) - margin)) <= 1e-4
    trees = pm.trees()
    om = oracle.model_from_nodes(trees, pm.cat_words(), "binary:logistic", float(pm.base_score))
    sub = rows[:20_000]
    parts = np.array_split(np.arange(sub.shape[0]), 16)
    _say("device SHAP done")
    with ThreadPoolExecutor(16) as ex:
        want = np.concatenate(list(ex.map(lambda ix: om.shap(sub[ix]), parts)))
    _say("oracle SHAP done")
    assert np.max(np.abs(phi[:20_000] - want)) <= 1e-5
