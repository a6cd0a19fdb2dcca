"""CPU pins of the oracle's reg:quantileerror, against what the reference's own
tests and the mathematics fix:

* the intercepts are the labels' alpha quantiles: the reference's known
  answers (quantile_intercept_matches_xgboost_rules,
  src/training/objective.rs:1386-1401) and numpy's linear-interpolation
  quantile at alpha (n + 1) - 1;
* the round's scale is (sum w sqrt|p - y| / sum w)^2: the reference's hand
  value (7/6)^2 (tests/robust_objectives_009.rs:51-58) and the zero cases
  (objective.rs:1452-1462);
* the pair is the derivative of the smoothed pinball loss
  L(r) = S/2 (0.04 S log cosh(r / (0.04 S)) + (1 - 2 alpha) r), checked by
  central differences, and tends to S (1 - alpha) and -S alpha for large
  residuals; the Hessian is the majorising curvature 12.5 tanh(x)/x, floored
  at 12.5 * 3e-4, never below the loss's own 12.5 sech^2(x);
* with max_depth 0 every tree is -sum(g) / (sum(h) + lambda) * eta of the
  pairs under the scale of the round's starting margins (float64 recomputed);
* several alphas train one output per alpha, each output equal to the
  single-alpha model (multi_quantile_trains_one_tree_per_alpha_and_equals_
  single_alpha_models, src/training/mod.rs:7336-7377);
* a trained model covers its quantile
  (quantile_objective_trains_reproducibly_and_tracks_the_quantile,
  src/training/mod.rs:7312-7333, on its wiggly_data generator, :7431-7451).
"""

from __future__ import annotations

import numpy as np
import pytest


def _wiggly(n, seed, nf=5):
    """wiggly_data (src/training/mod.rs:7431-7451): an LCG in u64, features in
    [-2, 2), every 13th cell (by i + f) missing, a smooth signal plus noise."""
    mask = (1 << 64) - 1
    state = (seed * 0x9E3779B97F4A7C15 + 1) & mask

    def nxt():
        nonlocal state
        state = (state * 6364136223846793005 + 1442695040888963407) & mask
        return np.float32(np.float32(state >> 40) / np.float32(1 << 24))

    x = np.empty((n, nf), np.float32)
    y = np.empty(n, np.float32)
    for i in range(n):
        row = [np.float32(nxt() * np.float32(4.0) - np.float32(2.0)) for _ in range(nf)]
        sig = (np.sin(row[0] * np.float32(1.7)) + np.float32(0.8) * np.cos(row[1] * np.float32(3.0))
               - np.float32(0.5) * row[2] + np.float32(0.3) * nxt())
        for f in range(nf):
            x[i, f] = np.nan if (i + f) % 13 == 0 else row[f]
        y[i] = sig
    return x, y


def test_intercepts_known_answers(oracle):
    y = np.array([4.0, 1.0, 3.0, 2.0], np.float32)
    w = np.ones(4, np.float32)
    assert oracle.quantile_intercepts(y, [0.1]).tolist() == [1.0]
    assert oracle.quantile_intercepts(y, [0.9]).tolist() == [4.0]
    assert oracle.quantile_intercepts(y, [0.5]).tolist() == [2.5]
    assert oracle.quantile_intercepts(y, [0.5], w).tolist() == [2.0]
    assert oracle.quantile_intercepts(y, [0.1, 0.5, 0.9]).tolist() == [1.0, 2.5, 4.0]
    assert oracle.quantile_intercepts(y, [0.1, 0.5, 0.9], w).tolist() == [1.0, 2.0, 4.0]


def test_intercepts_are_numpy_quantiles(oracle):
    rng = np.random.default_rng(2)
    for n in (5, 17, 1000):
        y = rng.standard_normal(n).astype(np.float32)
        for a in (0.05, 0.3, 0.5, 0.77, 0.95):
            got = oracle.quantile_intercepts(y, [a])[0]
            # XGBoost's Quantile: the order statistic at alpha (n + 1), clamped at the ends
            pos = min(max(a * (n + 1) - 1, 0.0), n - 1)
            want = np.quantile(y.astype(np.float64), pos / (n - 1), method="linear")
            assert abs(got - want) <= 2e-7 * max(1.0, abs(want)), (n, a, got, want)
        # weighted: the first sorted label whose running weight reaches alpha * total
        w = rng.uniform(0.1, 2.0, n).astype(np.float32)
        order = np.argsort(y, kind="stable")
        cdf = np.cumsum(w[order].astype(np.float64))
        for a in (0.2, 0.5, 0.9):
            got = oracle.quantile_intercepts(y, [a], w)[0]
            idx = min(int(np.searchsorted(cdf, cdf[-1] * a, side="left")), n - 1)
            assert got == y[order][idx] or abs(cdf[idx] - cdf[-1] * a) < 1e-3


def test_scale_hand_values(oracle):
    s = oracle.quantile_scale([0.0, 2.0, 1.0], [4.0, 1.0, 1.0], [3.0, 1.0, 2.0])
    assert abs(s - (7.0 / 6.0) ** 2) < 1e-6
    assert oracle.quantile_scale([1.0, 2.0], [1.0, 2.0]) == 0.0
    assert oracle.quantile_scale([0.0, 0.0], [1.0, 4.0]) > 0.0
    assert oracle.quantile_scale([0.0, 0.0], [1.0, 4.0]) == pytest.approx(((1 + 2) / 2) ** 2)
    pairs = oracle.quantile_pairs([1.0], [2.0], 0.3, 0.0)
    assert pairs.tolist() == [[0.0, 0.0]]


def _loss(r, s, alpha):
    c = 0.04 * s
    return s / 2 * (c * np.log(np.cosh(r / c)) + (1 - 2 * alpha) * r)


@pytest.mark.parametrize("alpha", [0.1, 0.5, 0.9])
def test_pairs_are_the_smoothed_pinball_derivative(oracle, alpha):
    rng = np.random.default_rng(3)
    s = 1.7
    r = (rng.standard_normal(400) * 0.2).astype(np.float32)
    y = rng.standard_normal(400).astype(np.float32)
    p = (y + r).astype(np.float32)
    rr = p.astype(np.float64) - y.astype(np.float64)
    pairs = oracle.quantile_pairs(p, y, alpha, s).astype(np.float64)
    x = rr / (0.04 * s)
    g64 = s / 2 * (np.tanh(x) + 1 - 2 * alpha)
    h64 = 12.5 * np.maximum(np.where(x == 0, 1.0, np.tanh(x) / np.where(x == 0, 1.0, x)), 3e-4)
    assert np.allclose(pairs[:, 0], g64, rtol=2e-5, atol=2e-6)
    assert np.allclose(pairs[:, 1], h64, rtol=2e-5)
    eps = 1e-5
    fd = (_loss(rr + eps, s, alpha) - _loss(rr - eps, s, alpha)) / (2 * eps)
    assert np.allclose(pairs[:, 0], fd, rtol=1e-4, atol=1e-5)
    assert np.all(pairs[:, 1] >= 12.5 / np.cosh(x) ** 2 * (1 - 1e-5))
    far = oracle.quantile_pairs([1e4, -1e4], [0.0, 0.0], alpha, s).astype(np.float64)
    assert far[0, 0] == pytest.approx(s * (1 - alpha), rel=1e-6)
    assert far[1, 0] == pytest.approx(-s * alpha, rel=1e-6, abs=1e-6)
    assert far[0, 1] == pytest.approx(12.5 * 3e-4, rel=1e-6)
    w = rng.uniform(0.2, 3.0, 400).astype(np.float32)
    pw = oracle.quantile_pairs(p, y, alpha, s, w)
    assert np.array_equal(pw, (pairs.astype(np.float32) * w[:, None]).astype(np.float32))


def _data(n=2000, seed=0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, 4)).astype(np.float32)
    y = (x[:, 0] * 2 + rng.standard_exponential(n)).astype(np.float32)
    return x, y


@pytest.mark.parametrize("weighted", [False, True])
def test_one_leaf_trees_are_newton_steps_under_the_round_scale(oracle, weighted):
    x, y = _data(seed=4)
    w = np.random.default_rng(5).uniform(0.2, 2.0, y.size).astype(np.float32) if weighted else None
    alpha, lam, eta, rounds = 0.8, 1.0, 0.3, 4
    m = oracle.train(x, y, oracle.make_params(objective="reg:quantileerror", quantile_alpha=alpha,
                                              n_rounds=rounds, max_depth=0, eta=eta,
                                              min_child_weight=0.0, nthread=1), weights=w)
    tr = m.trees()
    assert len(tr) == rounds and all(t.size == 1 for t in tr)
    assert m.base_score == oracle.quantile_intercepts(y, [alpha], w)[0]
    margin = np.full(y.size, m.base_score, np.float64)
    ww = np.ones(y.size) if w is None else w.astype(np.float64)
    for r in range(rounds):
        s = (np.sum(ww * np.sqrt(np.abs(margin - y))) / ww.sum()) ** 2
        xx = (margin - y) / (0.04 * s)
        g = s / 2 * (np.tanh(xx) + 1 - 2 * alpha) * ww
        h = 12.5 * np.maximum(np.where(xx == 0, 1.0, np.tanh(xx) / np.where(xx == 0, 1.0, xx)),
                              3e-4) * ww
        want = -g.sum() / (h.sum() + lam) * eta
        got = float(tr[r]["leaf_value"][0])
        assert got == pytest.approx(want, rel=1e-4, abs=1e-6), (r, got, want)
        margin = margin + got
    assert np.allclose(m.train_margins(y.size), margin, atol=1e-4)


def test_several_alphas_equal_single_alpha_models(oracle):
    x, y = _wiggly(2000, 5)
    alphas = [0.1, 0.5, 0.9]
    kw = dict(n_rounds=6, max_depth=4, max_bin=16, eta=0.3, min_child_weight=0.0, nthread=1,
              cols_per_block=2)
    multi = oracle.train(x, y, oracle.make_params(objective="reg:quantileerror",
                                                  quantile_alpha=alphas, **kw))
    assert multi.num_outputs == 3 and multi.n_trees == 18
    tr = multi.trees()
    pm = multi.predict_margin(x)
    for j, a in enumerate(alphas):
        single = oracle.train(x, y, oracle.make_params(objective="reg:quantileerror",
                                                       quantile_alpha=a, **kw))
        assert multi.class_margins()[j] == single.base_score
        st = single.trees()
        for r in range(6):
            assert tr[r * 3 + j].tobytes() == st[r].tobytes(), (a, r)
        assert np.array_equal(pm[:, j].view(np.uint32), single.predict_margin(x).view(np.uint32))


@pytest.mark.parametrize("alpha", [0.1, 0.5, 0.9])
def test_trained_model_tracks_its_quantile(oracle, alpha):
    x, y = _wiggly(2000, 4)
    m = oracle.train(x, y, oracle.make_params(objective="reg:quantileerror", quantile_alpha=alpha,
                                              n_rounds=30, max_depth=4, max_bin=16, eta=0.3,
                                              min_child_weight=0.0, nthread=1, cols_per_block=2))
    frac = float(np.mean(y <= m.predict_margin(x)))
    assert abs(frac - alpha) < 0.12, (alpha, frac)


@pytest.mark.parametrize("alphas,msg", [([1.5], r"\[0, 1\]"), ([0.9, 0.1], "ascending"),
                                        ([float("nan")], r"\[0, 1\]")])
def test_invalid_alphas_are_rejected(oracle, alphas, msg):
    x, y = _data(n=100)
    with pytest.raises(RuntimeError, match=msg):
        oracle.train(x, y, oracle.make_params(objective="reg:quantileerror", quantile_alpha=alphas,
                                              n_rounds=1))
