"""CPU pins of the oracle (no GPU).

The oracle is the reference of every GPU parity test, so it is itself checked
here against what fixes its behaviour independently of its own code:

* the reference's XGBoost-3.4.1 golden margins (tests/fixtures of the
  reference, copied as data under tests/golden/fixtures), bit for bit, also
  across column-block sizes and thread counts
  (tests/bit_exact_vs_xgboost.rs:94-171);
* brute-force restatements that share no intermediate with the oracle
  (row-by-row histograms, threshold enumeration by direct row partition,
  stable-partition closed form, Shapley values by subset enumeration);
* closed forms (power-of-two quantizer scales, inverse-scale exactness over
  every exponent, quadrature moments);
* the concrete expectations of the reference's unit tests (sampled feature
  counts, sketch properties).
"""

from __future__ import annotations

import ctypes as C
import math
from fractions import Fraction

import numpy as np
import pytest

from helpers import case_params, golden_cases, load_case

F32_MAX = float(np.finfo(np.float32).max)


# ---------------------------------------------------------------- golden

CASES = golden_cases()


def _train_case(O, c, **over):
    x, y, w, want = load_case(c)
    kw = case_params(c)
    kw.update(over)
    m = O.train(x, y, O.make_params(**kw), weights=w, monotone=c.get("monotone_constraints"))
    return m, x, want


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_golden_margins_bit_exact(oracle, case):
    """tests/bit_exact_vs_xgboost.rs:135-233: margins equal XGBoost's bit for bit."""
    m, x, want = _train_case(oracle, case)
    got = m.predict_margin(x)
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, f"{bad.size} rows differ, first {bad[:5]}: {got[bad[:5]]} vs {want[bad[:5]]}"
    # the margins kept during training are the same numbers
    assert np.array_equal(m.train_margins(x.shape[0]).view(np.uint32), want.view(np.uint32))


def test_golden_case_count():
    """index.json 18 + weighted 13 + monotone 13 (tests/bit_exact_vs_xgboost.rs:176)."""
    names = [c["name"] for c in CASES]
    assert len(names) == 44 and len(set(names)) == 44
    assert sum(1 for n in names if n.startswith("w_")) == 13


@pytest.mark.parametrize("cols", [1, 3, 5, 8])
def test_golden_margins_across_block_sizes(oracle, cols):
    """tests/bit_exact_vs_xgboost.rs:94-145: the column-block layout is not
    part of the algorithm (ties resolve by feature id across blocks)."""
    for c in CASES:
        if not c["name"].startswith(("a_s1", "a_s3", "deep_")):
            continue
        m, x, want = _train_case(oracle, c, cols_per_block=cols)
        assert np.array_equal(m.predict_margin(x).view(np.uint32), want.view(np.uint32)), c["name"]


@pytest.mark.parametrize("nthread", [2, 4, 8])
def test_golden_margins_across_thread_counts(oracle, nthread):
    """tests/bit_exact_vs_xgboost.rs:147-171 (cols_per_block = 1)."""
    for c in CASES:
        if not c["name"].startswith(("a_s2", "deep_logistic")):
            continue
        m, x, want = _train_case(oracle, c, cols_per_block=1, nthread=nthread)
        assert np.array_equal(m.predict_margin(x).view(np.uint32), want.view(np.uint32)), c["name"]


# ---------------------------------------------------------------- quantizer

def _pow2_scale_closed_form(bound: float, n_rows: int) -> float:
    """2^floor(log2(2^62 / n / bound)) clamped to 2^±1000 (src/types.rs:367-385),
    computed with exact rationals."""
    if not bound > 0:
        return 1.0
    n = max(n_rows, 1)
    target = Fraction(2**62, n) / Fraction(bound)
    # floor(log2(target)) exactly
    e = target.numerator.bit_length() - target.denominator.bit_length()
    if Fraction(2) ** e > target:
        e -= 1
    while Fraction(2) ** (e + 1) <= target:
        e += 1
    return math.ldexp(1.0, max(-1000, min(1000, e)))


@pytest.mark.parametrize("rows", [1, 100, 10_500_000, 2**40])
@pytest.mark.parametrize("bound", [1.0, 0.25, 3.0, 1e-3, 0.7, 12345.678, 2.0**-149, F32_MAX])
def test_quantizer_scale_closed_form(oracle, rows, bound):
    s = oracle.quantizer_scales(bound, 0.25, rows)
    assert s[0] == _pow2_scale_closed_form(bound, rows)
    assert s[1] == _pow2_scale_closed_form(0.25, rows)


def test_quantizer_scale_clamps(oracle):
    """src/types.rs:1012-1024: the exponent is clamped to +-1000."""
    assert oracle.quantizer_scales(2.0**-940, 1.0, 1)[0] == 2.0**1000
    assert oracle.quantizer_scales(2.0**1000, 1.0, 2**62)[0] == 2.0**-1000


def test_inverse_scale_exact_for_every_exponent(oracle):
    """src/types.rs:926-967: dequantising equals value / scale bit for bit for
    every exponent in -1000..=1000."""
    vals = [-(2**63), 2**63 - 1, 0, 1, -1, 2**53 - 1, 2**53 + 1, -(2**53) - 1]
    state = 37
    for _ in range(128):
        state = (state * 6364136223846793005 + 1) & (2**64 - 1)
        vals.append(state - 2**64 if state >= 2**63 else state)
    fixed = np.repeat(np.array(vals, np.int64), 2)
    L = oracle.lib()
    out = np.zeros(fixed.size, np.float64)
    for e in range(-1000, 1001):
        scales = np.array([2.0**e, 2.0**-e], np.float64)
        L.orc_to_f64(oracle._p(fixed), len(vals), oracle._p(scales), oracle._p(out))
        with np.errstate(over="ignore"):
            want_g = np.array([float(v) / scales[0] for v in vals])
            want_h = np.array([float(v) / scales[1] for v in vals])
        assert np.array_equal(out[0::2].view(np.uint64), want_g.view(np.uint64)), e
        assert np.array_equal(out[1::2].view(np.uint64), want_h.view(np.uint64)), e


def _round_half_away(q: Fraction) -> int:
    a = abs(q)
    r = math.floor(a + Fraction(1, 2))
    return r if q >= 0 else -r


def test_quantize_rounds_half_away_from_zero(oracle):
    """to_fixed = round-half-away(v * scale) (src/types.rs:320-330), checked
    with exact rationals, including exact .5 ties of both signs."""
    rng = np.random.default_rng(5)
    n = 2000
    g = rng.normal(size=n).astype(np.float32)
    h = rng.uniform(0.01, 0.25, size=n).astype(np.float32)
    scales = oracle.quantizer_scales(float(np.abs(g).max()), float(h.max()), n)
    # plant exact ties: v * scale = k + 1/2
    for i, k in enumerate([0, 1, 2, 7, -1, -2, -8]):
        g[i] = np.float32((k + 0.5) / scales[0]) if k >= 0 else np.float32((k - 0.5) / scales[0])
    gp = np.empty(2 * n, np.float32)
    gp[0::2], gp[1::2] = g, h
    fixed, total = oracle.quantize(gp, scales)
    for i in range(n):
        assert fixed[2 * i] == _round_half_away(Fraction(float(g[i])) * Fraction(scales[0])), i
        assert fixed[2 * i + 1] == _round_half_away(Fraction(float(h[i])) * Fraction(scales[1])), i
    assert total[0] == fixed[0::2].sum() and total[1] == fixed[1::2].sum()
    assert fixed[0] == 1 and fixed[2] == 2 and fixed[8] == -2 and fixed[12] == -9


def test_roundtrip_small_dyadic(oracle):
    """src/types.rs:1000-1010: -0.75 / 0.25 survive quantise + dequantise."""
    s = oracle.quantizer_scales(0.75, 0.25, 1)
    fixed, _ = oracle.quantize(np.array([-0.75, 0.25], np.float32), s)
    out = np.zeros(2)
    oracle.lib().orc_to_f64(oracle._p(fixed), 1, oracle._p(s), oracle._p(out))
    assert out.tolist() == [-0.75, 0.25]


@pytest.mark.parametrize("mult", [1e-6, 1.0, 1e6])
def test_extreme_gradient_magnitudes(oracle, mult):
    """src/training/hist.rs:760-789: no overflow and no lost signal at +-6
    orders of magnitude."""
    n = 1000
    i = np.arange(n)
    g = (((i % 17) - 8.0) * mult).astype(np.float32)
    h = (((i % 5) + 1.0) * mult).astype(np.float32)
    s = oracle.quantizer_scales(float(np.abs(g).max()), float(np.abs(h).max()), n)
    gp = np.empty(2 * n, np.float32)
    gp[0::2], gp[1::2] = g, h
    fixed, total = oracle.quantize(gp, s)
    got = np.zeros(2)
    oracle.lib().orc_to_f64(oracle._p(total), 1, oracle._p(s), oracle._p(got))
    wg, wh = float(g.astype(np.float64).sum()), float(h.astype(np.float64).sum())
    assert abs(got[0] - wg) <= max(1e-9 * abs(wh), 1e-9 * abs(wg))
    assert abs(got[1] - wh) <= 1e-9 * abs(wh)


# ---------------------------------------------------------------- histogram

def _brute_hist(bins, offsets, gpair, rows=None):
    """Row-by-row accumulation with wrapping i64 adds, skipping the sentinel
    (src/training/hist.rs:873-905)."""
    nf, n = bins.shape
    miss = 0xFF if bins.dtype == np.uint8 else 0xFFFF
    out = np.zeros((int(offsets[-1]), 2), np.int64)
    it = range(n) if rows is None else rows
    with np.errstate(over="ignore"):
        for r in it:
            for f in range(nf):
                b = int(bins[f, r])
                if b == miss:
                    continue
                out[offsets[f] + b] += gpair[2 * r: 2 * r + 2]
    return out.reshape(-1)


def _random_block(rng, n, n_bins, width, miss_rate):
    dt = np.uint8 if width == 1 else np.uint16
    miss = 0xFF if width == 1 else 0xFFFF
    bins = np.empty((len(n_bins), n), dt)
    for f, nb in enumerate(n_bins):
        bins[f] = rng.integers(0, nb, size=n)
        bins[f][rng.random(n) < miss_rate] = miss
    offsets = np.concatenate([[0], np.cumsum(n_bins)]).astype(np.uint32)
    return bins, offsets


@pytest.mark.parametrize("width", [1, 2])
def test_hist_matches_brute_force(oracle, width):
    rng = np.random.default_rng(11 + width)
    n = 300
    n_bins = [1, 2, 5, 17, 254 if width == 1 else 900]
    bins, offsets = _random_block(rng, n, n_bins, width, 0.1)
    gpair = rng.integers(-2**40, 2**40, size=2 * n, dtype=np.int64)
    assert np.array_equal(oracle.hist_build(bins, offsets, gpair), _brute_hist(bins, offsets, gpair))
    rows = np.sort(rng.choice(n, size=97, replace=False)).astype(np.uint32)
    assert np.array_equal(oracle.hist_build(bins, offsets, gpair, rows),
                          _brute_hist(bins, offsets, gpair, rows))


def test_hist_order_independent_and_wrapping(oracle):
    """tests/bit_exact_vs_xgboost.rs:292-365: shuffled row lists give the same
    histogram; sums near the i64 limit wrap instead of saturating."""
    rng = np.random.default_rng(3)
    n = 2000
    bins, offsets = _random_block(rng, n, [3, 8, 255], 1, 0.05)
    gpair = rng.integers(2**61, 2**62, size=2 * n, dtype=np.int64)  # partial sums overflow
    rows = np.arange(n, dtype=np.uint32)
    shuf = rng.permutation(rows).astype(np.uint32)
    a = oracle.hist_build(bins, offsets, gpair, rows)
    b = oracle.hist_build(bins, offsets, gpair, shuf)
    assert np.array_equal(a, b)
    assert np.array_equal(a, _brute_hist(bins, offsets, gpair))
    sums = np.zeros(2, np.int64)
    oracle.lib().orc_node_sum(oracle._p(gpair), oracle._p(shuf), n, n, oracle._p(sums))
    with np.errstate(over="ignore"):
        assert sums[0] == gpair[0::2].sum() and sums[1] == gpair[1::2].sum()


def test_hist_missing_excluded_node_sum_includes(oracle):
    """src/training/hist.rs:791-871: missing rows are in no bin but in the node sum."""
    rng = np.random.default_rng(8)
    n = 64
    bins, offsets = _random_block(rng, n, [4, 4, 4], 1, 0.0)
    bins[2, [0, 2]] = 0xFF
    gpair = rng.integers(-1000, 1000, size=2 * n, dtype=np.int64)
    h = oracle.hist_build(bins, offsets, gpair).reshape(-1, 2)
    total = gpair[0::2].sum()
    assert h[8:12, 0].sum() == total - gpair[0] - gpair[4]
    assert h[0:4, 0].sum() == total
    s = np.zeros(2, np.int64)
    oracle.lib().orc_node_sum(oracle._p(gpair), None, 0, n, oracle._p(s))
    assert s[0] - h[8:12, 0].sum() == gpair[0] + gpair[4]


def test_hist_siblings_subtract_to_parent(oracle):
    """src/training/hist.rs:909-951."""
    rng = np.random.default_rng(9)
    n = 500
    bins, offsets = _random_block(rng, n, [7, 30, 255], 1, 0.1)
    gpair = rng.integers(-2**62, 2**62, size=2 * n, dtype=np.int64)
    mask = rng.random(n) < 0.3
    left = np.nonzero(mask)[0].astype(np.uint32)
    right = np.nonzero(~mask)[0].astype(np.uint32)
    p = oracle.hist_build(bins, offsets, gpair)
    lh = oracle.hist_build(bins, offsets, gpair, left)
    rh = oracle.hist_build(bins, offsets, gpair, right)
    with np.errstate(over="ignore"):
        assert np.array_equal(p - lh, rh)


def test_hist_u16_equals_u8(oracle):
    """src/training/hist.rs:1077-1131: a 16-bit block with the same bins
    accumulates exactly like the 8-bit block."""
    rng = np.random.default_rng(10)
    n = 777
    b8, offsets = _random_block(rng, n, [5, 200, 255], 1, 0.2)
    b16 = b8.astype(np.uint16)
    b16[b8 == 0xFF] = 0xFFFF
    gpair = rng.integers(-2**50, 2**50, size=2 * n, dtype=np.int64)
    assert np.array_equal(oracle.hist_build(b8, offsets, gpair), oracle.hist_build(b16, offsets, gpair))


# ---------------------------------------------------------------- split

class _Lcg:
    """The LCG of src/training/split.rs:650-665."""

    def __init__(self, seed):
        self.s = seed & (2**64 - 1)

    def u32(self):
        self.s = (self.s * 6364136223846793005 + 1442695040888963407) & (2**64 - 1)
        return self.s >> 33

    def signed(self):
        return np.float32(np.float32(self.u32() % 20000) / np.float32(10000.0) - np.float32(1.0))


def _random_split_case(seed, n, nf, miss_pct):
    rng = _Lcg((seed * 0x9E3779B97F4A7C15 + 1) & (2**64 - 1))
    feat_ids = np.array([f * 3 + 5 for f in range(nf)], np.uint32)
    n_bins = [2 + f % 5 for f in range(nf)]
    offsets = np.concatenate([[0], np.cumsum(n_bins)]).astype(np.uint32)
    bins = np.zeros((nf, n), np.uint8)
    for f in range(nf):
        for r in range(n):
            bins[f, r] = 0xFF if rng.u32() % 100 < miss_pct else rng.u32() % n_bins[f]
    g = np.zeros(n, np.float32)
    h = np.zeros(n, np.float32)
    for r in range(n):
        g[r] = rng.signed()
        h[r] = np.float32(0.05) + np.float32(0.2) * np.float32(np.float32(rng.u32() % 1000) / np.float32(1000.0))
    return feat_ids, offsets, bins, g, h


def _brute_split(bins, offsets, feat_ids, fixed, scales, lam, gamma, mcw):
    """Enumerate every (feature, threshold, missing side) by partitioning the
    rows directly (src/training/split.rs:806-853); plain gain form."""
    nf, n = bins.shape
    inv = 1.0 / scales
    fg, fh = fixed[0::2], fixed[1::2]
    tg, th = int(fg.sum()), int(fh.sum())
    pg, ph = tg * inv[0], th * inv[1]
    parent = pg * pg / (ph + lam)
    best = None
    for f in range(nf):
        nb = int(offsets[f + 1] - offsets[f])
        col = bins[f]
        miss = col == 0xFF
        for b in range(nb + 1):
            for ml in (False, True):
                left = np.where(miss, ml, col.astype(np.int64) < b)
                lg, lh = int(fg[left].sum()), int(fh[left].sum())
                rg, rh = tg - lg, th - lh
                a, c = lg * inv[0], lh * inv[1]
                d, e = rg * inv[0], rh * inv[1]
                if c < mcw or e < mcw:
                    continue
                gain = np.float32(a * a / (c + lam) + d * d / (e + lam) - parent - gamma)
                if not gain > np.float32(1e-6):
                    continue
                if best is None or gain > best[0]:
                    best = (gain, int(feat_ids[f]), b, ml, (lg, lh), (rg, rh))
    return best


def test_split_matches_brute_force_on_random_cases(oracle):
    """src/training/split.rs:855-898: 40 seeds x 3 missing rates; gains equal
    bit for bit, and the same candidate carries the same child sums."""
    checked = 0
    for seed in range(40):
        for miss in (0, 10, 50):
            feat_ids, offsets, bins, g, h = _random_split_case(seed, 64, 4, miss)
            n = g.size
            scales = oracle.quantizer_scales(float(np.abs(g).max()), float(np.abs(h).max()), n)
            gp = np.empty(2 * n, np.float32)
            gp[0::2], gp[1::2] = g, h
            fixed, total = oracle.quantize(gp, scales)
            hist = oracle.hist_build(bins, offsets, fixed)
            lam = 1.0 + seed % 3
            mcw = (seed % 4) * 0.5
            p = oracle.make_params(**{"lambda": lam, "gamma": 0.0, "min_child_weight": mcw})
            got = oracle.best_split(hist, feat_ids, offsets, total, scales, p, given_weight=False)
            want = _brute_split(bins, offsets, feat_ids, fixed, scales, lam, 0.0, mcw)
            if want is None:
                assert not got.found, (seed, miss)
            else:
                assert got.found, (seed, miss)
                assert np.float32(got.gain).view(np.uint32) == want[0].view(np.uint32), (seed, miss)
                if (got.feat, got.bin, bool(got.missing_left)) == want[1:4]:
                    assert tuple(got.left) == want[4] and tuple(got.right) == want[5]
            checked += 1
    assert checked == 120


def test_split_tie_goes_to_lowest_feature_id(oracle):
    """Identical features: within a block the first feature (blocks hold
    ascending ids) keeps a tie (strict greater, src/training/split.rs:260-270);
    across blocks the lower id wins (:631-642), so every block layout agrees."""
    rng = np.random.default_rng(4)
    n = 200
    col = rng.integers(0, 6, size=n).astype(np.uint8)
    bins = np.stack([col, col, col])
    offsets = np.array([0, 6, 12, 18], np.uint32)
    g = rng.normal(size=n).astype(np.float32)
    h = np.full(n, 0.25, np.float32)
    s = oracle.quantizer_scales(float(np.abs(g).max()), 0.25, n)
    gp = np.empty(2 * n, np.float32)
    gp[0::2], gp[1::2] = g, h
    fixed, total = oracle.quantize(gp, s)
    hist = oracle.hist_build(bins, offsets, fixed)
    p = oracle.make_params()
    got = oracle.best_split(hist, np.array([4, 7, 9], np.uint32), offsets, total, s, p)
    assert got.found and got.feat == 4
    # one feature per block: same gain and bin in every block
    one = [oracle.best_split(hist[2 * offsets[k]: 2 * offsets[k + 1]], np.array([f], np.uint32),
                             np.array([0, 6], np.uint32), total, s, p)
           for k, f in enumerate([4, 7, 9])]
    assert len({(b.bin, np.float32(b.gain).tobytes()) for b in one}) == 1
    assert (one[0].bin, np.float32(one[0].gain)) == (got.bin, np.float32(got.gain))


def test_split_perfect_separator(oracle):
    """A feature whose bin determines the sign of the gradient is split
    exactly at the sign change."""
    n = 400
    col = (np.arange(n) % 10).astype(np.uint8)
    g = np.where(col < 7, -1.0, 1.0).astype(np.float32)
    h = np.full(n, 0.5, np.float32)
    noise = np.random.default_rng(1).integers(0, 10, size=n).astype(np.uint8)
    bins = np.stack([noise, col])
    offsets = np.array([0, 10, 20], np.uint32)
    s = oracle.quantizer_scales(1.0, 0.5, n)
    gp = np.empty(2 * n, np.float32)
    gp[0::2], gp[1::2] = g, h
    fixed, total = oracle.quantize(gp, s)
    got = oracle.best_split(oracle.hist_build(bins, offsets, fixed), np.array([0, 1], np.uint32),
                            offsets, total, s, oracle.make_params())
    assert got.found and got.feat == 1 and got.bin == 7 and not got.missing_left


# ---------------------------------------------------------------- partition

@pytest.mark.parametrize("width", [1, 2])
def test_partition_stable_closed_form(oracle, width):
    """Left rows in their order, then right rows in theirs
    (tests/gpu_histogram.rs:720-800 closed form)."""
    rng = np.random.default_rng(20 + width)
    n = 5000
    miss = 0xFF if width == 1 else 0xFFFF
    col = rng.integers(0, 40, size=n).astype(np.uint8 if width == 1 else np.uint16)
    col[rng.random(n) < 0.1] = miss
    rows = np.sort(rng.choice(n, size=3000, replace=False)).astype(np.uint32)
    rng.shuffle(rows)
    for split_bin, ml in ((17, False), (17, True), (0, False), (40, True)):
        out, nl = oracle.partition(rows, col, split_bin, ml)
        v = col[rows]
        gl = np.where(v == miss, ml, v < split_bin)
        want = np.concatenate([rows[gl], rows[~gl]])
        assert nl == int(gl.sum()) and np.array_equal(out, want)
    cats = np.zeros(1, np.uint64)
    for c in (1, 5, 33):
        cats[0] |= np.uint64(1) << np.uint64(c)
    out, nl = oracle.partition(rows, col, 0, True, cats)
    v = col[rows]
    in_set = np.isin(v, [1, 5, 33])
    gl = np.where(v == miss, True, ~in_set)
    assert nl == int(gl.sum()) and np.array_equal(out, np.concatenate([rows[gl], rows[~gl]]))


# ---------------------------------------------------------------- colsample

def test_sampled_counts(oracle):
    """src/data/colsample.rs:367-377."""
    for n, rate, k in ((300, 0.1, 30), (300, 0.3, 90), (28, 0.7, 19), (10, 0.99, 9),
                       (300, 0.0001, 1), (1, 0.5, 1), (2000, 0.5, 1000)):
        assert oracle.sample_features(n, rate, 0, 0).size == k, (n, rate)


def test_sample_properties(oracle):
    """src/data/colsample.rs:380-420: rate 1 is the identity; samples are
    sorted, unique and reproducible; seed or round changes them."""
    assert oracle.sample_features(64, 1.0, 9, 3).tolist() == list(range(64))
    s = oracle.sample_features(300, 0.1, 42, 7)
    assert s.size == 30 and np.all(np.diff(s.astype(np.int64)) > 0) and s.max() < 300
    assert np.array_equal(s, oracle.sample_features(300, 0.1, 42, 7))
    assert not np.array_equal(s, oracle.sample_features(300, 0.1, 43, 7))
    assert not np.array_equal(s, oracle.sample_features(300, 0.1, 42, 8))


# ---------------------------------------------------------------- sketch

def test_sketch_low_cardinality_exact(oracle):
    """src/data/sketch.rs:571-587: 4 unique values -> 3 cuts, one bin each."""
    x = np.tile(np.array([1.0, 2.0, 3.0, 5.0], np.float32), 1000)[:, None]
    vals, offs = oracle.sketch_cuts(x, 256)
    assert offs[-1] == 3
    L = oracle.lib()
    bins = [L.orc_find_bin(oracle._p(vals), oracle._p(offs), 0, 0, v) for v in (1.0, 2.0, 3.0, 5.0)]
    assert bins == [0, 1, 2, 3]


@pytest.mark.parametrize("shuffled", [False, True])
def test_sketch_uniform_quantiles(oracle, shuffled):
    """src/data/sketch.rs:589-616: max quantile error < 0.02 at 16 bins."""
    n, mb = 100_000, 16
    i = np.arange(n)
    v = ((i * 7919) % n if shuffled else i).astype(np.float32) / np.float32(n)
    vals, offs = oracle.sketch_cuts(v[:, None], mb)
    assert 0 < vals.size < mb
    err = max(abs(float(c) - (k + 1) / mb) for k, c in enumerate(vals))
    assert err < 0.02


def test_sketch_properties(oracle):
    """src/data/sketch.rs:659-790: weights shift quantiles; constant feature
    has no cuts; cuts strictly increase on skewed data; huge finite values
    give finite cuts; per-feature bin counts."""
    v = np.arange(1000, dtype=np.float32)[:, None]
    cu, _ = oracle.sketch_cuts(v, 8)
    cw, _ = oracle.sketch_cuts(v, 8, weights=np.where(v[:, 0] > 500, 10.0, 1.0).astype(np.float32))
    assert cw[3] > cu[3]
    c, _ = oracle.sketch_cuts(np.full((1000, 1), 42.0, np.float32), 256)
    assert c.size == 0
    i = np.arange(100_000)
    c, _ = oracle.sketch_cuts(np.where(i % 100 == 0, i, 0).astype(np.float32)[:, None], 16)
    assert np.all(np.diff(c) > 0)
    c, _ = oracle.sketch_cuts(np.array([-3.0e38, -2.0e38, 0.0, 2.0e38, F32_MAX], np.float32)[:, None], 16)
    assert c.size == 4 and np.all(np.isfinite(c)) and np.all(np.diff(c) > 0)
    x = np.stack([np.arange(1000), np.arange(1000) % 3, np.full(1000, 7)], 1).astype(np.float32)
    _, offs = oracle.sketch_cuts(x, 8)
    nb = np.diff(offs.astype(np.int64)) + 1
    assert nb[0] > 4 and nb[1] == 3 and nb[2] == 1


def test_sketch_ignores_nan(oracle):
    """src/data/sketch.rs:678-690: NaN carries no weight."""
    v = np.arange(100, dtype=np.float32)
    x = np.concatenate([v, np.full(100, np.nan, np.float32)])[:, None]
    a, _ = oracle.sketch_cuts(x, 8)
    b, _ = oracle.sketch_cuts(v[:, None], 8)
    assert np.array_equal(a, b)


# ---------------------------------------------------------------- SHAP

def test_quadrature_rule_integrates_polynomials(oracle):
    """src/model/explain.rs:989-1000."""
    nodes, w = oracle.quadrature_rule()
    for p in range(7):
        approx = sum(float(w[i]) * float(nodes[i]) ** p for i in range(8))
        assert abs(approx - 1.0 / (p + 1)) < 1e-5, p


def _tree_value(t, i, row, known, cats):
    nd = t[i]
    if nd["is_leaf"]:
        return float(nd["leaf_value"])
    f = int(nd["feat"])
    l, r = int(nd["left"]), int(nd["right"])
    if known >> f & 1:
        return _tree_value(t, l if _goes_left(nd, row[f], cats) else r, row, known, cats)
    cl, cr = float(t[l]["sum_hess"]), float(t[r]["sum_hess"])
    return (cl * _tree_value(t, l, row, known, cats) + cr * _tree_value(t, r, row, known, cats)) / (cl + cr)


def _goes_left(nd, v, cats):
    if np.isnan(v):
        return bool(nd["default_left"])
    if nd["cat_len"]:
        words = cats[int(nd["cat_begin"]): int(nd["cat_begin"]) + int(nd["cat_len"])]
        c = int(v)
        if v < 0 or c != v or c >= 32 * len(words):
            return True
        return not (int(words[c >> 5]) >> (c & 31)) & 1
    return bool(v < nd["split_cond"])


def _brute_shap(model, row, nf):
    """Shapley values by subset enumeration (src/model/explain.rs:906-963)."""
    trees = model.trees()
    cats = model.cat_words()

    def val(mask):
        return sum(_tree_value(t, 0, row, mask, cats) for t in trees)

    phi = np.zeros(nf + 1)
    for i in range(nf):
        for s in range(1 << nf):
            if s >> i & 1:
                continue
            k = bin(s).count("1")
            w = math.factorial(k) * math.factorial(nf - k - 1) / math.factorial(nf)
            phi[i] += w * (val(s | 1 << i) - val(s))
    phi[nf] = val(0) + float(model.base_margin)
    return phi


@pytest.mark.parametrize("objective", ["binary:logistic", "reg:squarederror"])
def test_shap_matches_brute_force_and_sums_to_margin(oracle, objective):
    rng = np.random.default_rng(31)
    n, nf = 600, 5
    x = rng.normal(size=(n, nf)).astype(np.float32)
    x[rng.random((n, nf)) < 0.1] = np.nan
    y = (np.nan_to_num(x[:, 0]) + 0.5 * np.nan_to_num(x[:, 1]) * np.nan_to_num(x[:, 2]) > 0)
    y = y.astype(np.float32)
    p = oracle.make_params(n_rounds=6, max_depth=4, eta=0.3, objective=objective, max_bin=32)
    m = oracle.train(x, y, p)
    rows = x[:12]
    got = m.shap(rows)
    for r in range(rows.shape[0]):
        want = _brute_shap(m, rows[r], nf)
        assert np.max(np.abs(got[r] - want)) < 2e-5, r
    margin = m.predict_margin(rows)
    assert np.max(np.abs(got.sum(axis=1) - margin)) < 1e-4


def test_shap_categorical_matches_brute_force(oracle):
    """src/model/explain.rs:1049-1094: categorical sets, invalid codes and
    missing values follow the same decisions in the explanation."""
    rng = np.random.default_rng(32)
    n, nf = 800, 4
    x = rng.normal(size=(n, nf)).astype(np.float32)
    x[:, 1] = rng.integers(0, 12, size=n)
    x[:, 3] = rng.integers(0, 3, size=n)
    y = (np.isin(x[:, 1], [2, 3, 7, 11]) ^ (x[:, 0] > 0.3)).astype(np.float32)
    cat = np.array([0, 1, 0, 1], np.uint8)
    p = oracle.make_params(n_rounds=5, max_depth=3, eta=0.5, max_bin=64)
    m = oracle.train(x, y, p, categorical=cat)
    assert any(t["cat_len"].any() for t in m.trees())
    rows = x[:10].copy()
    rows[0, 1] = np.nan
    rows[1, 1] = -1.0
    rows[2, 1] = 40.0
    got = m.shap(rows)
    for r in range(rows.shape[0]):
        assert np.max(np.abs(got[r] - _brute_shap(m, rows[r], nf))) < 2e-5, r
    assert np.max(np.abs(got.sum(axis=1) - m.predict_margin(rows))) < 1e-4


def _brute_interaction(model, row, nf, i, j):
    """Shapley interaction value of (i, j), split evenly between (i, j) and
    (j, i), by subset enumeration (src/model/explain.rs:964-980)."""
    trees = model.trees()
    cats = model.cat_words()

    def val(mask):
        return sum(_tree_value(t, 0, row, mask, cats) for t in trees)

    acc = 0.0
    for s in range(1 << nf):
        if s >> i & 1 or s >> j & 1:
            continue
        k = bin(s).count("1")
        w = math.factorial(k) * math.factorial(nf - k - 2) / (2.0 * math.factorial(nf - 1))
        acc += w * (val(s | 1 << i | 1 << j) - val(s | 1 << i) - val(s | 1 << j) + val(s))
    return acc


def _small_model(oracle, seed, nf=4, depth=3, rounds=5, categorical=False):
    rng = np.random.default_rng(seed)
    n = 700
    x = rng.normal(size=(n, nf)).astype(np.float32)
    x[rng.random((n, nf)) < 0.1] = np.nan
    cat = None
    if categorical:
        x[:, 1] = rng.integers(0, 9, size=n)
        cat = np.zeros(nf, np.uint8)
        cat[1] = 1
    y = ((np.nan_to_num(x[:, 0]) * np.nan_to_num(x[:, 2]) > 0) ^ (np.nan_to_num(x[:, 1]) > 3))
    p = oracle.make_params(n_rounds=rounds, max_depth=depth, eta=0.4, max_bin=32)
    return oracle.train(x, y.astype(np.float32), p, categorical=cat), x


@pytest.mark.parametrize("categorical", [False, True])
def test_interactions_match_brute_force_and_row_sums(oracle, categorical):
    """src/model/explain.rs:1112-1139: off-diagonal entries equal the
    brute-force Shapley interaction values, the matrix is symmetric, and
    each row sums to the row's SHAP value."""
    m, x = _small_model(oracle, 41, categorical=categorical)
    nf = x.shape[1]
    rows = x[:8]
    inter = m.explain(rows, "interactions")
    shap = m.explain(rows, "contribs")
    for r in range(rows.shape[0]):
        mat = inter[r]
        for i in range(nf):
            for j in range(nf):
                if i != j:
                    want = _brute_interaction(m, rows[r], nf, i, j)
                    assert abs(float(mat[i, j]) - want) < 5e-5, (r, i, j)
                    assert mat[i, j] == mat[j, i]
        assert np.max(np.abs(mat.sum(axis=1) - shap[r])) < 1e-4, r


def test_saabas_equals_treeshap_on_stumps_and_sums_to_margin(oracle):
    """On depth-1 trees the path attribution of Saabas is the exact Shapley
    value (one split: the only feature gets leaf - root mean); on deeper
    trees the contributions still telescope to the margin."""
    m1, x = _small_model(oracle, 43, depth=1, rounds=6)
    rows = x[:50]
    sa, sh = m1.explain(rows, "approx"), m1.explain(rows, "contribs")
    assert np.max(np.abs(sa - sh)) < 1e-6
    m3, x3 = _small_model(oracle, 44, depth=4, rounds=6)
    rows = x3[:200]
    sa = m3.explain(rows, "approx")
    assert np.max(np.abs(sa.sum(axis=1) - m3.predict_margin(rows))) < 1e-5


def test_saabas_closed_form_on_a_hand_tree(oracle):
    """The tree of src/model/tree.rs:1474-1480 (x0 < 1.5, missing left; its
    left child x1 < 0.5), worked by hand: node means are cover-weighted leaf
    means, and each path step adds the change of the mean to its split
    feature (src/model/explain.rs:730-760)."""
    nodes = np.zeros(5, oracle.NODE_DTYPE)
    # root: feat 0 < 1.5, default left; children 1 (cover 6), 2 (leaf 3.0, cover 4)
    nodes[0] = (0, 1.5, 1, 2, 1, 0, 0, 0.0, 4.0, 10.0, 0, 0)
    nodes[1] = (1, 0.5, 3, 4, 0, 0, 0, 0.0, 2.0, 6.0, 0, 0)
    nodes[2] = (0, 3.0, -1, -1, 0, 1, 0, 3.0, 0.0, 4.0, 0, 0)
    nodes[3] = (0, 1.0, -1, -1, 0, 1, 0, 1.0, 0.0, 3.0, 0, 0)
    nodes[4] = (0, 2.0, -1, -1, 0, 1, 0, 2.0, 0.0, 3.0, 0, 0)
    m = oracle.model_from_nodes([nodes], [], "reg:squarederror", 0.5)
    rows = np.array([[0.0, 0.0], [0.0, 1.0], [2.0, 0.0], [np.nan, 0.5]], np.float32)
    got = m.explain(rows, "approx")
    m1 = (1.0 * 3 + 2.0 * 3) / 6.0           # mean of node 1: 1.5
    m0 = (m1 * 6 + 3.0 * 4) / 10.0           # root mean: 2.1
    want = np.array([
        [m1 - m0, 1.0 - m1, m0 + 0.5],
        [m1 - m0, 2.0 - m1, m0 + 0.5],
        [3.0 - m0, 0.0, m0 + 0.5],
        [m1 - m0, 2.0 - m1, m0 + 0.5],
    ], np.float32)
    assert np.max(np.abs(got - want)) < 1e-6
    leaf = m.explain(rows, "leaf")
    assert leaf[:, 0].tolist() == [3.0, 4.0, 2.0, 4.0]


def test_leaf_indices_follow_the_tree(oracle):
    """src/model/explain.rs:1159-1178: one split at 0.5 (missing left) and a
    root-only tree; rows 0.2, 0.9, NaN reach leaves l, r, l and 0."""
    t0 = np.zeros(3, oracle.NODE_DTYPE)
    t0[0] = (0, 0.5, 1, 2, 1, 0, 0, 0.0, 1.0, 10.0, 0, 0)
    t0[1] = (0, 1.0, -1, -1, 0, 1, 0, 1.0, 0.0, 4.0, 0, 0)
    t0[2] = (0, 2.0, -1, -1, 0, 1, 0, 2.0, 0.0, 6.0, 0, 0)
    t1 = np.zeros(1, oracle.NODE_DTYPE)
    t1[0] = (0, 3.0, -1, -1, 0, 1, 0, 3.0, 0.0, 1.0, 0, 0)
    m = oracle.model_from_nodes([t0, t1], [], "reg:squarederror", 0.5)
    rows = np.array([[0.2], [0.9], [np.nan]], np.float32)
    assert m.explain(rows, "leaf").tolist() == [[1.0, 0.0], [2.0, 0.0], [1.0, 0.0]]


def test_leaf_ids_reproduce_the_margin(oracle):
    """Summing each tree's leaf value at the returned id, in tree order from
    the base margin, gives predict_margin bit for bit."""
    m, x = _small_model(oracle, 45, depth=5, rounds=7, categorical=True)
    rows = x[:300]
    leaf = m.explain(rows, "leaf").astype(np.int64)
    trees = m.trees()
    acc = np.full(rows.shape[0], np.float32(m.base_margin), np.float32)
    for t, tr in enumerate(trees):
        acc = (acc + tr["leaf_value"][leaf[:, t]]).astype(np.float32)
    assert np.array_equal(acc.view(np.uint32), m.predict_margin(rows).view(np.uint32))


def test_explain_base_margin_replaces_the_bias(oracle):
    """src/model/explain.rs:1216-1285: a per-row base margin replaces the
    intercept in the bias column and nothing else."""
    m, x = _small_model(oracle, 46)
    rows = x[:20]
    bm = np.linspace(-1, 1, 20).astype(np.float32)
    for kind in ("contribs", "approx"):
        a, b = m.explain(rows, kind), m.explain(rows, kind, margin=bm)
        assert np.array_equal(a[:, :-1], b[:, :-1])
        assert np.allclose(b[:, -1] - a[:, -1], bm - np.float32(m.base_margin), atol=1e-6)


# ---------------------------------------------------------------- row subsample

def _selected(oracle, n, rate, seed, tree):
    L = oracle.lib()
    th = L.orc_threshold_for(rate)
    return np.array([L.orc_row_selected(r, th, seed, tree) for r in range(n)], bool)


def test_subsample_threshold_closed_form(oracle):
    """threshold_for = floor(rate * 2^53), all rows at rate >= 1 or <= 0
    (src/data/subsample.rs:19-29)."""
    L = oracle.lib()
    for rate in (0.1, 0.25, 0.5, 0.7, 0.9, 0.999):
        assert L.orc_threshold_for(rate) == int(Fraction(float(np.float32(rate))) * 2**53)
    for rate in (1.0, 1.5, 0.0, -1.0, float("nan")):
        assert L.orc_threshold_for(rate) == 2**64 - 1


def test_subsample_properties(oracle):
    """src/data/subsample.rs:121-185: reproducible, keyed by seed and tree,
    Bernoulli per row (counts vary by tree, near the rate)."""
    a = _selected(oracle, 500, 0.5, 11, 2)
    assert np.array_equal(a, _selected(oracle, 500, 0.5, 11, 2))
    assert not np.array_equal(a, _selected(oracle, 500, 0.5, 11, 3))
    assert not np.array_equal(a, _selected(oracle, 500, 0.5, 12, 2))
    counts = [int(_selected(oracle, 10_000, 0.5, 1, t).sum()) for t in range(8)]
    assert len(set(counts)) > 1 and all(4700 <= c < 5300 for c in counts)
    for rate in (0.1, 0.25, 0.9):
        frac = _selected(oracle, 100_000, rate, 3, 0).mean()
        assert abs(frac - rate) < 0.01, rate


def test_subsample_one_is_identity_and_sampling_changes_trees(oracle):
    rng = np.random.default_rng(41)
    x = rng.normal(size=(3000, 4)).astype(np.float32)
    y = (x[:, 0] + 0.5 * rng.normal(size=3000) > 0).astype(np.float32)
    base = oracle.train(x, y, oracle.make_params(n_rounds=4, max_depth=4))
    one = oracle.train(x, y, oracle.make_params(n_rounds=4, max_depth=4, subsample=1.0))
    half = oracle.train(x, y, oracle.make_params(n_rounds=4, max_depth=4, subsample=0.5, seed=3))
    same = oracle.train(x, y, oracle.make_params(n_rounds=4, max_depth=4, subsample=0.5, seed=3))
    assert all(np.array_equal(a, b) for a, b in zip(base.trees(), one.trees()))
    assert not all(a.size == b.size and np.array_equal(a, b) for a, b in zip(base.trees(), half.trees()))
    assert all(np.array_equal(a, b) for a, b in zip(half.trees(), same.trees()))


@pytest.mark.parametrize("objective", ["binary:logistic", "reg:squarederror"])
def test_scale_pos_weight_is_folded_weight(oracle, objective):
    """gradient_weights (src/training/mod.rs:5466-5490): at a fixed base
    score, scale_pos_weight k trains the same model as sample weights
    w * k on rows labelled 1 (and w elsewhere). Sample weights also weight
    the quantile sketch, so the features have few distinct values (lossless
    cuts whatever the weights)."""
    rng = np.random.default_rng(42)
    n = 4000
    x = np.clip(np.round(rng.normal(size=(n, 5)) * 3), -8, 8).astype(np.float32)
    y = (x[:, 0] - x[:, 1] + 0.4 * rng.normal(size=n) > 0.5).astype(np.float32)
    w = rng.uniform(0.5, 2.0, size=n).astype(np.float32)
    k = np.float32(3.25)
    kw = dict(n_rounds=5, max_depth=5, objective=objective, base_score=0.3)
    a = oracle.train(x, y, oracle.make_params(scale_pos_weight=float(k), **kw), weights=w)
    b = oracle.train(x, y, oracle.make_params(**kw), weights=np.where(y == 1.0, w * k, w).astype(np.float32))
    c = oracle.train(x, y, oracle.make_params(**kw), weights=w)
    assert all(np.array_equal(s, t) for s, t in zip(a.trees(), b.trees()))
    assert not all(s.size == t.size and np.array_equal(s, t) for s, t in zip(a.trees(), c.trees()))
