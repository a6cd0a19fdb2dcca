"""CPU pins of the oracle's column samplers beyond colsample_bytree and of
its starting margins:

* the nested bylevel / bynode sets and the weighted sampler, restated from
  the reference's own unit tests (src/data/colsample.rs:313-465) and its
  end-to-end nested test (src/training/mod.rs:7379-7429);
* what the mathematics fixes about them: exponential clocks draw feature i
  first with probability w_i / sum(w) and pairs with the successive-draw
  probabilities; the uniform subsets are equally likely; every split of a
  trained tree uses a feature of its node's set;
* base_margin (src/training/mod.rs:7802-7975): a start equal to the
  intercept changes nothing, a start replaces the intercept but not the
  stored estimate (a closed-form leaf), class-major multiclass starts, and
  the input checks.
"""

from __future__ import annotations

import itertools

import numpy as np
import pytest

from helpers import node_depths, wiggly


# ------------------------------------------------ reference unit tests

def test_weighted_stages_exclude_zero_only_when_sampling(oracle):
    w = [0.0, 2.0, 0.0, 1.0]
    for seed in range(32):
        assert oracle.sample_features_weighted(4, 0.75, seed, 0, w).tolist() == [1, 3]
        assert oracle.sample_features_weighted(4, 1.0, seed, 0, w).tolist() == [0, 1, 2, 3]
    assert oracle.nested_set([0, 2], 0.5, 0.5, 7, 0, 1, 0, w).size == 0
    assert oracle.nested_set([], 0.5, 0.5, 7, 0, 2, 1, w).size == 0
    assert oracle.nested_set([1], 0.5, 0.5, 7, 0, 2, 1, w).tolist() == [1]


def test_weighted_draws_favor_larger_weights_without_duplicates(oracle):
    heavy = sum(oracle.sample_features_weighted(2, 0.5, s, 0, [1.0, 9.0]).tolist() == [1]
                for s in range(4096))
    assert 3500 <= heavy < 3900, heavy
    extremes = np.array([np.float32(1e-45), np.finfo(np.float32).max, 1.0, 0.0], np.float32)
    for s in range(32):
        picked = oracle.sample_features_weighted(4, 0.5, s, 0, extremes).tolist()
        assert len(picked) == 2 and picked[0] < picked[1]
        assert 3 not in picked and 1 in picked


def test_equal_weights_preserve_uniform_sampler_exactly(oracle):
    assert oracle.validated_weights([3.0] * 12, 12) == 0
    for r in range(20):
        assert np.array_equal(oracle.sample_features_weighted(12, 0.4, 7, r, None),
                              oracle.sample_features(12, 0.4, 7, r))


def test_invalid_weights_are_rejected(oracle):
    for bad, what in (([1.0, -1.0], "nonnegative"), ([1.0, np.nan], "finite"),
                      ([0.0, 0.0], "positive")):
        with pytest.raises(ValueError, match=what):
            oracle.validated_weights(bad, 2)
    assert oracle.validated_weights([1.0, 2.0], 2) == 1


def test_nested_sets_are_nested_sized_sorted_and_deterministic(oracle):
    tree = oracle.sample_features(100, 0.8, 7, 3)
    assert tree.size == 80
    for depth in range(4):
        level = oracle.nested_set(tree, 0.5, 0.5, 7, 3, 1, depth)
        assert level.size == 40 and np.all(np.diff(level) > 0)
        assert np.isin(level, tree).all()
        assert np.array_equal(level, oracle.nested_set(tree, 0.5, 0.5, 7, 3, 1, depth))
        for node in range(6):
            s = oracle.nested_set(level, 0.5, 0.5, 7, 3, 2, node)
            assert s.size == 20 and np.all(np.diff(s) > 0) and np.isin(s, level).all()
            assert np.array_equal(s, oracle.nested_set(level, 0.5, 0.5, 7, 3, 2, node))
    lv = lambda seed, t, d: oracle.nested_set(tree, 0.5, 0.5, seed, t, 1, d)  # noqa: E731
    assert not np.array_equal(lv(7, 3, 0), lv(7, 3, 1))
    level = lv(7, 3, 0)
    assert not np.array_equal(oracle.nested_set(level, 0.5, 0.5, 7, 3, 2, 0),
                              oracle.nested_set(level, 0.5, 0.5, 7, 3, 2, 1))
    assert not np.array_equal(lv(7, 3, 0), lv(7, 4, 0))
    assert not np.array_equal(lv(7, 3, 0), lv(8, 3, 0))


def test_nested_rate_one_is_identity(oracle):
    tree = np.arange(10, dtype=np.uint32)
    assert np.array_equal(oracle.nested_set(tree, 1.0, 0.5, 0, 0, 1, 3), tree)
    assert np.array_equal(oracle.nested_set(tree, 0.5, 1.0, 0, 0, 2, 9), tree)


# ------------------------------------------------ what the mathematics fixes

def _chi2_ok(counts, probs, n):
    """Pearson's statistic below a bound well above its 0.999 quantile for
    these few degrees of freedom (a wrong law fails by orders of magnitude)."""
    exp = np.asarray(probs) * n
    stat = float(((np.asarray(counts) - exp) ** 2 / exp).sum())
    return stat < 25.0, stat


def test_exponential_clocks_draw_in_proportion_to_weight(oracle):
    # One draw of five (rate 0.2): P(i) = w_i / sum(w), zero never drawn.
    # A key of -ln(U) * w, ln(U) / w or U / w breaks this law.
    w = np.array([1.0, 2.0, 3.0, 0.0, 4.0], np.float32)
    n = 20000
    counts = np.zeros(5)
    for s in range(n):
        picked = oracle.sample_features_weighted(5, 0.2, s, 11, w)
        assert picked.size == 1
        counts[picked[0]] += 1
    assert counts[3] == 0
    ok, stat = _chi2_ok(counts[[0, 1, 2, 4]], w[[0, 1, 2, 4]] / w.sum(), n)
    assert ok, (counts, stat)


def test_exponential_clocks_draw_pairs_successively(oracle):
    # Two of three with weights 1, 1, 2: successive proportional draws give
    # P{0,1} = 1/6 and P{0,2} = P{1,2} = 5/12.
    w = [1.0, 1.0, 2.0]
    n = 12000
    counts = {(0, 1): 0, (0, 2): 0, (1, 2): 0}
    for s in range(n):
        counts[tuple(oracle.sample_features_weighted(3, 0.7, s, 5, w).tolist())] += 1
    ok, stat = _chi2_ok(list(counts.values()), [1 / 6, 5 / 12, 5 / 12], n)
    assert ok, (counts, stat)


def test_uniform_subsets_are_equally_likely(oracle):
    # bylevel 0.5 of six features: each of the 20 three-sets with chance 1/20,
    # over the subset keys of many depths and trees.
    base = np.arange(6, dtype=np.uint32)
    subsets = {c: 0 for c in itertools.combinations(range(6), 3)}
    n = 0
    for tree in range(200):
        for depth in range(30):
            subsets[tuple(oracle.nested_set(base, 0.5, 1.0, 3, tree, 1, depth).tolist())] += 1
            n += 1
    ok, stat = _chi2_ok(list(subsets.values()), [1 / 20] * 20, n)
    assert ok, stat


# ------------------------------------------------ end to end

def _train(oracle, x, y, **kw):
    p = dict(n_rounds=5, max_depth=6, max_bin=64, eta=0.3, objective="reg:squarederror",
             cols_per_block=1, nthread=1, seed=9)
    p.update(kw)
    return oracle.train(x, y, oracle.make_params(**p))


def _bits(m):
    return b"".join(t.tobytes() for t in m.trees())


@pytest.mark.parametrize("bylevel, bynode", [(0.6, 1.0), (1.0, 0.6), (0.8, 0.5)])
def test_nested_sampling_is_thread_and_blocking_invariant(oracle, bylevel, bynode):
    """src/training/mod.rs:7379-7412 on its wiggly_data(1500, 6)."""
    x, y = wiggly(1500, 6)
    full = _bits(_train(oracle, x, y))
    ref = _bits(_train(oracle, x, y, colsample_bylevel=bylevel, colsample_bynode=bynode))
    assert ref != full
    for threads, cols in ((4, 2), (2, 1), (3, 5)):
        got = _train(oracle, x, y, colsample_bylevel=bylevel, colsample_bynode=bynode,
                     nthread=threads, cols_per_block=cols)
        assert _bits(got) == ref, (threads, cols)


@pytest.mark.parametrize("kw", [
    dict(colsample_bylevel=0.5, colsample_bynode=0.5),
    dict(colsample_bytree=0.8, colsample_bynode=0.5, grow_policy="lossguide", max_leaves=12),
    dict(colsample_bytree=0.7, colsample_bylevel=0.5,
         feature_weights=[1, 0, 2, 3, 1, 0.5, 4, 1, 2, 1]),
    dict(colsample_bynode=0.4, feature_weights=[1, 0, 2, 3, 1, 0.5, 4, 1, 2, 1]),
])
def test_every_split_uses_a_feature_of_its_node_set(oracle, kw):
    rng = np.random.default_rng(4)
    x = rng.normal(size=(3000, 10)).astype(np.float32)
    y = (x @ rng.normal(size=10) + 0.3 * rng.normal(size=3000)).astype(np.float32)
    m = _train(oracle, x, y, n_rounds=4, **kw)
    assert _bits(m) != _bits(_train(oracle, x, y, n_rounds=4))
    fw = kw.get("feature_weights")
    weighted = fw is not None and oracle.validated_weights(fw, 10) == 1
    by = kw.get("colsample_bytree", 1.0)
    bl, bn = kw.get("colsample_bylevel", 1.0), kw.get("colsample_bynode", 1.0)
    checked = 0
    for t, tree in enumerate(m.trees()):
        tree_set = (oracle.sample_features_weighted(10, by, 9, t, fw if weighted else None)
                    if by < 1 else np.arange(10, dtype=np.uint32))
        depth = node_depths(tree)
        for i in np.flatnonzero(tree["is_leaf"] == 0):
            level = oracle.nested_set(tree_set, bl, bn, 9, t, 1, int(depth[i]),
                                      fw if weighted else None)
            s = oracle.nested_set(level, bl, bn, 9, t, 2, int(i), fw if weighted else None)
            assert tree["feat"][i] in s, (t, i)
            if weighted:
                assert all(fw[f] > 0 for f in s)
            checked += 1
    assert checked > 10


def test_invalid_nested_rates_are_rejected(oracle):
    x, y = wiggly(100, 1)
    for bylevel, bynode in ((-0.5, 1.0), (1.0, 1.5), (1.0, float("nan"))):
        with pytest.raises(RuntimeError, match="colsample_by"):
            _train(oracle, x, y, colsample_bylevel=bylevel, colsample_bynode=bynode)


# ------------------------------------------------ base_margin

def test_base_margin_equal_to_the_intercept_changes_nothing(oracle):
    x, y = wiggly(400, 3)
    yb = (y > 0).astype(np.float32)
    for obj, labels in (("reg:squarederror", y), ("binary:logistic", yb)):
        plain = _train(oracle, x, labels, objective=obj)
        start = np.full(400, plain.base_margin, np.float32)
        withm = _train(oracle, x, labels, objective=obj, base_margin=start)
        assert _bits(plain) == _bits(withm)
        assert plain.base_score == withm.base_score


def test_base_margin_replaces_the_start_but_not_the_estimated_intercept(oracle):
    n = 16
    x = np.zeros((n, 1), np.float32)
    margin = (np.arange(n) * 0.5).astype(np.float32)
    y = (margin + 1.0).astype(np.float32)
    m = _train(oracle, x, y, n_rounds=1, max_depth=1, eta=1.0, base_margin=margin,
               **{"lambda": 0.0})
    assert abs(m.base_score - y.mean()) < 1e-5
    # gradient pred - y = -1 on every row, Hessian 1: the leaf is +1
    assert m.trees()[0]["leaf_value"][0] == 1.0
    assert np.array_equal(m.train_margins(n), margin + np.float32(1.0))


def test_multiclass_base_margin_is_class_major(oracle):
    n = 30
    x = (np.arange(n) % 5).astype(np.float32).reshape(n, 1)
    y = (np.arange(n) % 3).astype(np.float32)
    kw = dict(objective="multi:softprob", num_class=3, n_rounds=2, max_depth=3)
    plain = _train(oracle, x, y, **kw)
    cm = plain.class_margins()
    start = np.concatenate([np.full(n, cm[k], np.float32) for k in range(3)])
    assert _bits(_train(oracle, x, y, base_margin=start, **kw)) == _bits(plain)
    skew = np.where(np.arange(3 * n) < n, 2.0, 0.0).astype(np.float32)
    skewed = _train(oracle, x, y, base_margin=skew, **kw)
    assert _bits(skewed) != _bits(plain)
    assert np.array_equal(skewed.class_margins(), cm)


def test_base_margin_must_be_finite(oracle):
    x, y = wiggly(20, 2)
    bad = np.zeros(20, np.float32)
    bad[3] = np.nan
    with pytest.raises(RuntimeError, match="finite"):
        _train(oracle, x, y, base_margin=bad)
