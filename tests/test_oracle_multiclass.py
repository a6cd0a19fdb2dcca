"""CPU pins of the oracle's multiclass training (multi:softprob / multi:softmax),
against what the mathematics fixes:

* the class intercepts are the centred logs of the class frequencies
  (Objective::initial_class_margins, src/training/objective.rs:1225-1248), or
  base_score copied K times when given (src/training/mod.rs:1430-1449);
* with max_depth 0 every tree is one leaf whose value is
  -sum(g) / (sum(h) + lambda) * eta, and the pairs are the softmax gradient
  g = p - [y == k], h = max(2 p (1 - p), 1e-16) times the sample weight
  (Objective::softmax_gradients, src/training/objective.rs:1175-1219) -- the
  factor 2, the label test and the weight are each checked by a closed form
  recomputed in float64 from the margins;
* every class's pairs come from the margins at the start of the round
  (train_multiclass_rounds, src/training/mod.rs:2578-2850), and the row
  sample of class k in round r is keyed on tree index r * K + k;
* margins are class-major, prediction adds tree t to output t mod K
  (Model::predict_margins_upto, src/model/tree.rs:470-480), and labels must be
  integers in [0, num_class) (objective.rs:681-687).
"""

from __future__ import annotations

import numpy as np
import pytest

K = 3


def _data(n=2000, seed=0, k=K):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, 4)).astype(np.float32)
    y = rng.choice(k, size=n, p=np.linspace(1, 2, k) / np.linspace(1, 2, k).sum())
    return x, y.astype(np.float32)


def _train(oracle, x, y, w=None, **kw):
    params = dict(objective="multi:softprob", num_class=K, n_rounds=1, max_depth=0, eta=0.3,
                  nthread=1, min_child_weight=0.0)
    params.update(kw)
    return oracle.train(x, y, oracle.make_params(**params), weights=w)


def _softmax_pairs(m, y, w):
    """float64 softmax pairs of every class from margins m [n, K]."""
    e = np.exp(m - m.max(axis=1, keepdims=True))
    p = e / e.sum(axis=1, keepdims=True)
    onehot = (y[:, None] == np.arange(m.shape[1])[None, :]).astype(np.float64)
    ww = np.ones(len(y)) if w is None else w.astype(np.float64)
    g = (p - onehot) * ww[:, None]
    h = np.maximum(2.0 * p * (1.0 - p) * ww[:, None], 1e-16)
    return g, h


def _leaves(tr):
    return np.array([t["leaf_value"][0] for t in tr], np.float64)


def test_intercepts_are_centred_log_frequencies(oracle):
    x, y = _data()
    w = np.random.default_rng(1).uniform(0.2, 2.0, y.size).astype(np.float32)
    for weights in (None, w):
        m = _train(oracle, x, y, weights)
        ww = np.ones(y.size) if weights is None else weights.astype(np.float64)
        freq = np.array([ww[y == k].sum() for k in range(K)]) / ww.sum()
        logs = np.log(freq + 1e-6)
        assert np.allclose(m.class_margins(), logs - logs.mean(), rtol=0, atol=2e-6)
    m = _train(oracle, x, y, base_score=0.25)
    assert m.class_margins().tolist() == [0.25] * K


@pytest.mark.parametrize("weighted", [False, True])
def test_one_leaf_trees_are_the_newton_step_of_the_softmax_pairs(oracle, weighted):
    x, y = _data(seed=3)
    w = (np.random.default_rng(4).uniform(0.2, 2.0, y.size).astype(np.float32)
         if weighted else None)
    lam, eta, rounds = 1.0, 0.3, 3
    m = _train(oracle, x, y, w, n_rounds=rounds, **{"lambda": lam, "eta": eta})
    tr = m.trees()
    assert len(tr) == rounds * K and all(t.size == 1 for t in tr)
    margins = np.tile(m.class_margins().astype(np.float64), (y.size, 1))
    for r in range(rounds):
        g, h = _softmax_pairs(margins, y, w)  # the round's starting margins
        want = -g.sum(axis=0) / (h.sum(axis=0) + lam) * eta
        got = _leaves(tr[r * K:(r + 1) * K])
        assert np.allclose(got, want, rtol=1e-5, atol=1e-7), (r, got, want)
        margins = margins + got[None, :]
    assert np.allclose(m.train_margins(y.size).T, margins, atol=1e-5)


def test_a_plausible_mistake_fails_the_newton_step(oracle):
    """The closed form tells the Hessian's factor 2 apart: p (1 - p) instead
    would double every leaf."""
    x, y = _data(seed=5)
    m = _train(oracle, x, y, **{"lambda": 0.0})
    margins = np.tile(m.class_margins().astype(np.float64), (y.size, 1))
    g, h = _softmax_pairs(margins, y, None)
    got = _leaves(m.trees())
    assert np.allclose(got, -g.sum(0) / h.sum(0) * 0.3, rtol=1e-5)
    assert not np.allclose(got, -g.sum(0) / (h.sum(0) / 2) * 0.3, rtol=1e-2)


def test_row_sample_is_keyed_on_round_times_k_plus_class(oracle):
    x, y = _data(n=3000, seed=6)
    L = oracle.lib()
    th = L.orc_threshold_for(0.5)
    seed = 17
    m = _train(oracle, x, y, n_rounds=2, subsample=0.5, seed=seed, **{"lambda": 1.0})
    tr = m.trees()
    margins = np.tile(m.class_margins().astype(np.float64), (y.size, 1))
    for r in range(2):
        g, h = _softmax_pairs(margins, y, None)
        got = _leaves(tr[r * K:(r + 1) * K])
        for k in range(K):
            sel = np.array([L.orc_row_selected(i, th, seed, r * K + k) for i in range(y.size)],
                           bool)
            want = -g[sel, k].sum() / (h[sel, k].sum() + 1.0) * 0.3
            assert np.isclose(got[k], want, rtol=1e-5, atol=1e-7), (r, k)
        margins = margins + got[None, :]


def test_prediction_adds_tree_t_to_output_t_mod_k(oracle):
    x, y = _data(n=1500, seed=8)
    m = _train(oracle, x, y, n_rounds=4, max_depth=3)
    pm = m.predict_margin(x)
    assert pm.shape == (y.size, K)
    assert np.array_equal(pm.T.view(np.uint32), m.train_margins(y.size).view(np.uint32))
    one = []
    for t in m.trees():
        single = oracle.model_from_nodes([t], np.zeros(0, np.uint32), "reg:squarederror", 0.0)
        one.append(single.predict_margin(x).astype(np.float64))
    want = m.class_margins().astype(np.float64)[None, :].repeat(y.size, 0)
    for t, v in enumerate(one):
        want[:, t % K] += v
    assert np.allclose(pm, want, atol=1e-5)


def test_softmax_objective_trains_like_softprob(oracle):
    x, y = _data(n=1200, seed=9)
    a = _train(oracle, x, y, n_rounds=3, max_depth=3)
    b = _train(oracle, x, y, n_rounds=3, max_depth=3, objective="multi:softmax")
    for ta, tb in zip(a.trees(), b.trees()):
        assert ta.tobytes() == tb.tobytes()


@pytest.mark.parametrize("bad", [-1.0, 3.0, 1.5, np.nan])
def test_labels_must_be_class_indices(oracle, bad):
    x, y = _data(n=100)
    y[7] = bad
    with pytest.raises(RuntimeError, match="integers in"):
        _train(oracle, x, y)
