"""CPU pins of the oracle's growth policies, categorical enumeration and
sampling generators, restated from the reference's own tests:

* lossguide expansion order, its tie rule and the leaf cap
  (tests/lossguide.rs:89-147), the depthwise max_leaves rules
  (tests/max_leaves.rs:75-205) -- the cases live in growth_cases.py;
* categorical enumeration (src/training/split.rs:1371-1590): one-hot against
  a brute force over single categories, partition sets contiguous in weight
  order, the obvious grouping, forward-scan ties, max_cat_threshold, the
  one-hot switch; and the categorical decision (src/data/categorical.rs:
  334-350);
* SplitMix64 against its published output sequence (seed 1234567), the
  generator of colsample and, through its finaliser, of the row subsample.
"""

from __future__ import annotations

import numpy as np
import pytest

from growth_cases import cases, unlimited_equals_nonbinding

CASES = cases()


def _train(oracle, x, y, p):
    kw = dict(p)
    n = kw.pop("n_rounds")
    return oracle.train(x, y, oracle.make_params(n_rounds=n, cols_per_block=1, nthread=1, **kw))


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_growth_case(oracle, case):
    _, x, y, p, check = case
    check(_train(oracle, x, y, p).trees())


def test_zero_and_nonbinding_leaf_limits_match_bit_for_bit(oracle):
    x, y, p = unlimited_equals_nonbinding()
    a = _train(oracle, x, y, dict(p, max_leaves=0))
    b = _train(oracle, x, y, dict(p, max_leaves=64))
    for ta, tb in zip(a.trees(), b.trees()):
        assert ta.tobytes() == tb.tobytes()
    assert np.array_equal(a.predict_margin(x).view(np.uint32), b.predict_margin(x).view(np.uint32))


# ---------------------------------------------------------------- categorical

def _cat_case(seed, n_rows, n_cats, missing_pct):
    """A categorical histogram case: codes, gradient pairs, fixed-point pairs."""
    rng = np.random.default_rng(1000 + seed)
    codes = rng.integers(0, n_cats, size=n_rows).astype(np.uint8)
    codes[rng.random(n_rows) * 100 < missing_pct] = 0xFF
    g = rng.uniform(-1, 1, size=n_rows).astype(np.float32)
    h = rng.uniform(0.05, 0.25, size=n_rows).astype(np.float32)
    return codes, g, h


def _fixed(oracle, g, h):
    n = g.size
    s = oracle.quantizer_scales(float(np.abs(g).max()), float(np.abs(h).max()), n)
    gp = np.empty(2 * n, np.float32)
    gp[0::2], gp[1::2] = g, h
    fixed, total = oracle.quantize(gp, s)
    return s, fixed, total


def _best_cat(oracle, codes, fixed, total, s, n_cats, **kw):
    offsets = np.array([0, n_cats], np.uint32)
    hist = oracle.hist_build(codes.reshape(1, -1), offsets, fixed)
    p = oracle.make_params(**{"min_child_weight": 0.0, **kw})
    return oracle.best_split(hist, np.array([0], np.uint32), offsets, total, s, p,
                             given_weight=False, categorical=np.array([1], np.uint8))


def _set(sp):
    out = []
    for w in range(sp.n_cat_words):
        for b in range(64):
            if (int(sp.cats[w]) >> b) & 1:
                out.append(64 * w + b)
    return out


def _plain_gain(fixed, s, left_mask, lam, gamma=0.0):
    """G^2/(H + lambda) gain of a row partition, recomputed from the rows."""
    fg, fh = fixed[0::2], fixed[1::2]
    tg, th = int(fg.sum()), int(fh.sum())
    lg, lh = int(fg[left_mask].sum()), int(fh[left_mask].sum())
    rg, rh = tg - lg, th - lh
    inv = 1.0 / s
    f = lambda a, b: (a * inv[0]) ** 2 / (b * inv[1] + lam)  # noqa: E731
    return np.float32(f(lg, lh) + f(rg, rh) - f(tg, th) - gamma), (lg, lh), (rg, rh)


def test_one_hot_matches_brute_force_over_single_categories(oracle):
    """src/training/split.rs:1371-1428: below max_cat_to_onehot (4) the split is
    one category against the rest; gain bits, category and missing side equal
    the best of every single category on either missing side."""
    checked = 0
    for seed in range(30):
        for miss in (0, 15, 60):
            codes, g, h = _cat_case(seed, 80, 3, miss)
            s, fixed, total = _fixed(oracle, g, h)
            got = _best_cat(oracle, codes, fixed, total, s, 3)
            want = None
            for cat in range(3):
                for ml in (True, False):
                    left = np.where(codes == 0xFF, ml, codes != cat)
                    gain, _, _ = _plain_gain(fixed, s, left, 1.0)
                    if not gain > np.float32(1e-6):
                        continue
                    if want is None or gain > want[0]:
                        want = (gain, cat, ml)
            if want is None:
                assert not got.found
                continue
            assert got.found, (seed, miss)
            assert np.float32(got.gain).view(np.uint32) == want[0].view(np.uint32), (seed, miss)
            assert _set(got) == [want[1]] and bool(got.missing_left) == want[2], (seed, miss)
            checked += 1
    assert checked > 60


def test_partition_sets_are_contiguous_in_weight_order(oracle):
    """src/training/split.rs:1430-1483: the candidate's sums and gain agree with
    its own partition, and its set is a prefix or suffix of the categories
    ordered by weight -g / (h + lambda)."""
    found = 0
    for seed in range(40):
        for miss in (0, 10, 40):
            codes, g, h = _cat_case(seed, 200, 9, miss)
            s, fixed, total = _fixed(oracle, g, h)
            sp = _best_cat(oracle, codes, fixed, total, s, 9)
            if not sp.found:
                continue
            found += 1
            cats = _set(sp)
            assert 1 <= len(cats) < 9
            left = np.where(codes == 0xFF, bool(sp.missing_left), ~np.isin(codes, cats))
            gain, ls, rs = _plain_gain(fixed, s, left, 1.0)
            assert tuple(sp.left) == ls and tuple(sp.right) == rs
            assert np.float32(sp.gain).view(np.uint32) == gain.view(np.uint32)
            fg, fh = fixed[0::2].astype(np.float64), fixed[1::2].astype(np.float64)
            w = np.array([-(fg[codes == k].sum() / s[0]) / (fh[codes == k].sum() / s[1] + 1.0)
                          for k in range(9)])
            inside = w[cats]
            outside = w[[k for k in range(9) if k not in cats]]
            assert inside.min() >= outside.max() or inside.max() <= outside.min(), seed
    assert found > 60


def test_partition_finds_the_obvious_grouping(oracle):
    """src/training/split.rs:1485-1510: even categories push up, odd down."""
    codes = np.repeat(np.arange(6, dtype=np.uint8), 40)
    g = np.where(codes % 2 == 0, -1.0, 1.0).astype(np.float32)
    h = np.full(codes.size, 0.25, np.float32)
    s, fixed, total = _fixed(oracle, g, h)
    sp = _best_cat(oracle, codes, fixed, total, s, 6)
    assert sp.found and _set(sp) in ([0, 2, 4], [1, 3, 5])


def test_without_missing_rows_the_forward_scan_wins_ties(oracle):
    """src/training/split.rs:1512-1524: mirror partitions tie and the forward
    (missing-left) candidate is kept, for partition and one-hot scans."""
    for n_cats in (7, 3):
        codes, g, h = _cat_case(3 + n_cats, 120, n_cats, 0)
        s, fixed, total = _fixed(oracle, g, h)
        sp = _best_cat(oracle, codes, fixed, total, s, n_cats)
        assert sp.found and sp.missing_left, n_cats


def test_max_cat_threshold_limits_the_scan(oracle):
    """src/training/split.rs:1526-1545: threshold 3 allows prefixes of at most
    2 categories per direction; threshold 1 scans nothing."""
    codes, g, h = _cat_case(11, 400, 20, 5)
    s, fixed, total = _fixed(oracle, g, h)
    sp = _best_cat(oracle, codes, fixed, total, s, 20, max_cat_threshold=3)
    assert sp.found
    n = len(_set(sp))
    assert n <= 2 or n >= 18, n
    assert not _best_cat(oracle, codes, fixed, total, s, 20, max_cat_threshold=1).found


def test_onehot_threshold_switches_enumeration(oracle):
    """src/training/split.rs:1547-1566: 5 categories scan partitions by
    default and single categories once max_cat_to_onehot exceeds 5."""
    codes, g, h = _cat_case(5, 300, 5, 0)
    s, fixed, total = _fixed(oracle, g, h)
    part = _best_cat(oracle, codes, fixed, total, s, 5)
    onehot = _best_cat(oracle, codes, fixed, total, s, 5, max_cat_to_onehot=6)
    assert part.found and onehot.found
    assert len(_set(onehot)) == 1
    assert part.gain >= onehot.gain


def test_categorical_decision_matches_xgboost(oracle):
    """src/data/categorical.rs:334-350 through the oracle's prediction: a
    one-split tree on a categorical feature whose right-going set is
    {1, 4, 33}; members go right, other codes, truncated fractions included,
    left; negative, huge and infinite values go left."""
    t = np.zeros(3, oracle.NODE_DTYPE)
    t[0] = (0, 0.0, 1, 2, 0, 0, 0, 0.0, 1.0, 2.0, 0, 2)
    t[1] = (0, 0.0, -1, -1, 0, 1, 0, -1.0, 0.0, 1.0, 0, 0)
    t[2] = (0, 0.0, -1, -1, 0, 1, 0, 1.0, 0.0, 1.0, 0, 0)
    words = np.array([(1 << 1) | (1 << 4), 1 << 1], np.uint32)
    m = oracle.model_from_nodes([t], words, "reg:squarederror", 0.0)
    vals = [1.0, 4.0, 33.0, 0.0, 2.0, 4.9, 1000.0, -1.0, -0.5, 16_777_216.0, np.inf, -np.inf]
    right = [True, True, True, False, False, True, False, False, False, False, False, False]
    got = m.predict_margin(np.array(vals, np.float32).reshape(-1, 1))
    assert [bool(v == np.float32(1.0)) for v in got] == right


# ---------------------------------------------------------------- generators

def test_splitmix64_published_sequence(oracle):
    """SplitMix64 (Steele, Lea, Flood 2014; Vigna's splitmix64.c), the
    generator of src/data/colsample.rs:34-45: the published first outputs
    for seed 1234567."""
    out = np.zeros(5, np.uint64)
    oracle.lib().orc_splitmix64(1234567, 5, oracle._p(out))
    assert out.tolist() == [6457827717110365317, 3203168211198807973, 9817491932198370423,
                            4593380528125082431, 16408922859458223821]


def test_row_hash_is_the_splitmix_finaliser_of_the_mixed_key(oracle):
    """subsample::mix is SplitMix64's output function (src/data/subsample.rs:
    44-47): mix(state) after one increment equals the first SplitMix64 output,
    and row_hash mixes (seed, tree, row) as src/data/subsample.rs:50-55."""
    L = oracle.lib()
    out = np.zeros(1, np.uint64)
    for seed in (0, 1, 1234567, 2**63 + 11):
        L.orc_splitmix64(seed, 1, oracle._p(out))
        assert L.orc_mix64((seed + 0x9E3779B97F4A7C15) % 2**64) == int(out[0])
    M = 2**64 - 1
    rot = lambda v, r: ((v << r) | (v >> (64 - r))) & M  # noqa: E731
    for row, seed, tree in ((0, 0, 0), (5, 42, 3), (2**31, 2**40 + 7, 99)):
        key = seed ^ rot((tree * 0x9E3779B97F4A7C15) & M, 23) ^ ((row * 0xD6E8FEB86659FD93) & M)
        assert L.orc_row_hash(row, seed, tree) == L.orc_mix64(key)
