"""CPU pins of the quantile sketch (FeatureSketch, src/data/sketch.rs:28-435)
that the oracle and the product's host sketch share, beyond the reference's
property tests:

(a) The exact-summary regime. With D distinct values per feature and
    max_bin < D <= 16 * max_bin (the summary limit), no summary ever holds
    more than the limit, so compress never drops an entry and the final
    summary is every distinct value with its exact rank interval, whatever
    the batch order; with integer weights and fewer than 2^23 rows every
    rank sum is exact in f32. The cuts are then the first values whose
    exact midrank reaches each target total * k / max_bin: computed here
    from numpy's unique counts, independently of the sketch, over many
    batches (every merge level runs) in sorted, reversed and shuffled order.
(b) The lossy regime (C2's 28 columns at 10.5M rows, C4's 80 numeric
    columns at 2M rows): estimated ranks never exceed true ranks (rmin <=
    #{x < v}, rmax <= #{x <= v}, proved for build_summary, merge_entries,
    dedup and compress), so every cut's true midrank is at least its
    target; and above it by less than the bound B(N, limit) derived from the
    merge schedule (the deficiency grows by at most the compress spacing per
    level, the midrank spacing by at most one target spacing per compress).
    Both are checked against the true ranks of the sorted column.
(c) Planted mistakes in the oracle fail these (run by hand on a copy of the
    oracle; the list is in the oracle's header).
"""

from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

F32 = np.float32


def expected_cuts(values, weights, max_bin):
    """Cuts from exact ranks: the unique values, their total weights, the
    first value whose midrank reaches total * k / max_bin (targets in f32,
    as the reference computes them); a feature with at most max_bin - 1
    distinct values cuts at the midpoints of neighbours."""
    u, inv = np.unique(values, return_inverse=True)
    w = np.ones(values.size) if weights is None else weights.astype(np.float64)
    cnt = np.bincount(inv, weights=w)
    rmax = np.cumsum(cnt)
    rmin = rmax - cnt
    n_cuts = max_bin - 1
    if u.size <= n_cuts:
        a, b = u[:-1].astype(F32), u[1:].astype(F32)
        with np.errstate(over="ignore"):
            m = np.where(np.isfinite(b - a), a + (b - a) * F32(0.5), a * F32(0.5) + b * F32(0.5))
        return np.where(m <= a, b, m).astype(F32)
    rmid = (rmin + rmax) / 2
    total = F32(rmax[-1])
    out = []
    for k in range(1, max_bin):
        t = F32(F32(total * F32(k)) / F32(max_bin))
        idx = min(int(np.searchsorted(rmid, float(t), "left")), u.size - 1)
        v = u[idx]
        if not out or v > out[-1]:
            out.append(v)
    return np.array(out, F32)


def _distinct(rng, d):
    """d distinct nonzero float32 values (no zeros of either sign)."""
    vals = np.unique(rng.normal(0, 3, 3 * d).astype(F32))
    vals = vals[vals != 0]
    return rng.permutation(vals)[:d]


EXACT = [
    # max_bin, distinct, rows, order, weighted
    (256, 4096, 2_000_000, "shuffled", False),   # D at the summary limit
    (256, 3000, 1_200_000, "sorted", False),
    (64, 1000, 1_500_000, "reversed", False),
    (1024, 16384, 3_000_000, "shuffled", False),  # C4's max_bin, D at its limit
    (16, 200, 300_000, "shuffled", True),         # integer weights 1..3
    (255, 256, 500_000, "sorted", False),         # one more value than cuts
    (256, 200, 400_000, "shuffled", False),       # low cardinality: midpoints
]


def _exact_case(max_bin, d, n, order, weighted, seed):
    rng = np.random.default_rng(seed)
    vals = _distinct(rng, d)
    # every value appears, with skewed multiplicities
    p = rng.dirichlet(np.full(d, 0.7))
    col = np.concatenate([vals, rng.choice(vals, n - d, p=p)]).astype(F32)
    if order == "sorted":
        col = np.sort(col)
    elif order == "reversed":
        col = np.sort(col)[::-1].copy()
    else:
        col = rng.permutation(col)
    w = rng.integers(1, 4, n).astype(F32) if weighted else None
    return col, w


@pytest.mark.parametrize("case", EXACT, ids=[f"{c[0]}-{c[1]}-{c[3]}" for c in EXACT])
def test_exact_regime_cuts_equal_exact_rank_cuts(oracle, case):
    import ferrisboost_amd as fb

    max_bin, d, n, order, weighted = case
    col, w = _exact_case(*case, seed=d)
    want = expected_cuts(col, w, max_bin)
    got, offs = oracle.sketch_cuts(col.reshape(-1, 1), max_bin, weights=w)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # the product's host sketch (fbt_sketch_cuts) too
    cuts = fb.sketch(col.reshape(-1, 1), max_bin=max_bin, weight=w)
    assert np.array_equal(cuts.values.view(np.uint32), want.view(np.uint32))
    # and the final summary is every value with its exact rank interval
    if d <= 16 * max(max_bin, 2):
        s = oracle.sketch_summary(col, max_bin, w)
        u, inv = np.unique(col, return_inverse=True)
        cnt = np.bincount(inv, weights=None if w is None else w.astype(np.float64))
        assert np.array_equal(s["value"], u)
        assert np.array_equal(s["rmax"], np.cumsum(cnt).astype(F32))
        assert np.array_equal(s["rmin"], (np.cumsum(cnt) - cnt).astype(F32))


def test_exact_regime_is_order_free(oracle):
    col, _ = _exact_case(128, 2048, 1_000_000, "shuffled", False, seed=7)
    a, _ = oracle.sketch_cuts(col.reshape(-1, 1), 128)
    b, _ = oracle.sketch_cuts(np.sort(col).reshape(-1, 1), 128)
    c, _ = oracle.sketch_cuts(np.sort(col)[::-1].reshape(-1, 1).copy(), 128)
    assert np.array_equal(a, b) and np.array_equal(a, c)


# ---------------------------------------------------------------- (b)

def rank_bound(n, max_bin, s_max):
    """B(N, limit): the true midrank of a cut exceeds its target by less than
    H + C, where, for the summary limit L = 16 * max_bin (at least 32),
    level l holds W_l = 2^l L rows with target spacing
    Delta_l = W_l / (L - 1) and
      C_l <= sum_{i=1..l} 2^(l-i) (Delta_i + (s_max - 1) / 2)
        (a merge adds the two sides' coverage deficiencies, a compress at
        most one spacing),
      H_l <= s_max (1 + l / 2) + sum_{i=1..l} Delta_i
        (a merge widens the midrank spacing by at most half an entry's
        span, a compress by at most one spacing);
    the final collapse merges the occupied levels (the binary digits of the
    batch count) and compresses once more at spacing N / (L - 1). s_max
    bounds how many rows one value holds; 2 + N / 2^22 covers the f32
    rounding of midranks and targets."""
    lim = max(16 * max_bin, 32)
    nb = n // lim
    sig = (s_max - 1) / 2
    c_tot, h_max, levels = 0.0, 0.0, 0
    for lv in range(max(nb.bit_length(), 1)):
        if not (nb >> lv) & 1:
            continue
        levels += 1
        d = [(2 ** i) * lim / (lim - 1) for i in range(1, lv + 1)]
        c_tot += sum((2 ** (lv - i)) * (d[i - 1] + sig) for i in range(1, lv + 1))
        h_max = max(h_max, s_max * (1 + lv / 2) + sum(d))
    merged = nb * lim + n % lim
    d_fin = n / (lim - 1) if merged > lim else 0.0
    c_fin = c_tot + d_fin + sig
    h_fin = h_max + (levels + 1) * s_max / 2 + d_fin
    return h_fin + c_fin + 2 + n / 2 ** 22


def _lossy_check(oracle, col, max_bin):
    c = np.ascontiguousarray(col[~np.isnan(col)])
    s = np.sort(c)
    n = s.size
    summ = oracle.sketch_summary(c, max_bin)
    rm = np.searchsorted(s, summ["value"], "left")
    rp = np.searchsorted(s, summ["value"], "right")
    # estimated ranks never exceed true ranks; entries do not overlap
    assert (summ["rmin"] <= rm).all() and (summ["rmax"] <= rp).all()
    assert (summ["rmin"][1:] >= summ["rmax"][:-1]).all()
    assert summ["rmin"][0] == 0 and summ["rmax"][-1] == F32(n)
    cuts, _ = oracle.sketch_cuts(c.reshape(-1, 1), max_bin)
    assert np.all(np.diff(cuts) > 0)
    _, mult = np.unique(s, return_counts=True)
    bound = rank_bound(n, max_bin, int(mult.max()))
    rmid = (F32(0.5) * (summ["rmin"] + summ["rmax"])).astype(np.float64)
    total = F32(n)
    worst_lo, worst_hi = np.inf, -np.inf
    for k in range(1, max_bin):
        t = float(F32(F32(total * F32(k)) / F32(max_bin)))
        idx = min(int(np.searchsorted(rmid, t, "left")), summ.size - 1)
        v = summ["value"][idx]
        assert v in cuts
        mid = (np.searchsorted(s, v, "left") + np.searchsorted(s, v, "right")) / 2
        worst_lo = min(worst_lo, mid - t)
        worst_hi = max(worst_hi, mid - t)
    return worst_lo, worst_hi, bound, n / max_bin


@pytest.fixture(scope="module")
def c2_matrix():
    from ferrisboost_amd import datasets

    X, _, _, _ = datasets.narrow_binary()
    return X


@pytest.mark.parametrize("max_bin", [256, 255])
def test_c2_cuts_within_the_rank_bound(oracle, c2_matrix, max_bin):
    before = oracle.compress_clamps()
    with ThreadPoolExecutor(8) as ex:
        res = list(ex.map(lambda f: _lossy_check(oracle, c2_matrix[:, f], max_bin), range(28)))
    for f, (lo, hi, bound, width) in enumerate(res):
        assert lo >= -(2 + 10_500_000 / 2 ** 22), (f, lo)
        assert hi < bound, (f, hi, bound)
    # the derivation assumes compress's ceiling never cuts a walk short
    assert oracle.compress_clamps() == before


def test_c4_numeric_cuts_within_the_rank_bound(oracle):
    from ferrisboost_amd import datasets

    X, _, _, _ = datasets.widebin_cat()
    before = oracle.compress_clamps()
    with ThreadPoolExecutor(8) as ex:
        res = list(ex.map(lambda f: _lossy_check(oracle, X[:, f], 1024), range(80)))
    for f, (lo, hi, bound, width) in enumerate(res):
        assert lo >= -3, (f, lo)
        assert hi < bound, (f, hi, bound)
    assert oracle.compress_clamps() == before
