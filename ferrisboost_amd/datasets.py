"""Seeded synthetic workloads of the benchmark configurations.

Each generator returns (X float32 [n, F] row-major, y float32 [n], params,
extras) at any row count, so the same definition serves small parity cases and
full-size benchmark runs. No data is downloaded.

  narrow_binary   10.5M x 28 HIGGS-like: 11 N(0,1), 10 |N(0,1)|, 7 lognormal
                  products / sums of pairs; ~53% positives from a nonlinear
                  logistic model with interaction terms; depth 8, eta 0.1.
  plumbing        100k x 28 N(0,1), y ~ Bernoulli(sigmoid(x.w)), w ~ N(0, 0.25);
                  depth 6, eta 0.1.
  wide_binary     400k x 2000 N(0,1) rows scaled to unit L2 norm, labels from the
                  sign of a 200-sparse linear model with 5% flips; depth 8,
                  colsample_bytree 0.5.
  widebin_cat     2M x (80 U[0,1) with 10% NaN + 20 Zipf(1.2) categorical codes
                  0..499), squared error on a sum of step functions + N(0, 0.1);
                  max_bin 1024, lossguide, max_leaves 255.
  streaming       50M x 200 N(0,1), logistic labels; depth 8.

Rows are generated in chunks (2^13 to 2^20 rows, fixed per workload), each
chunk from its own generator (SeedSequence(seed).spawn), on a pool of threads
(numpy releases the GIL while it fills arrays); linear scores are summed one
column at a time in float64. The data depend on the seed and the row count
only, never on the number of threads or the machine.
"""

from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

CHUNK = 1 << 20


def _sigmoid(z):
    return 1.0 / (1.0 + np.exp(-z))


def _dot(block: np.ndarray, w: np.ndarray) -> np.ndarray:
    """block @ w in float64, one column at a time in column order: the same
    sums on every machine (no BLAS partitioning)."""
    z = np.zeros(block.shape[0], np.float64)
    for f in np.nonzero(w)[0]:
        z += block[:, f].astype(np.float64) * float(w[f])
    return z


def _threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def _chunked(n_rows: int, seed: int, fn, chunk: int = CHUNK) -> None:
    """fn(rng, s, e) for every chunk [s, e) of the rows, in parallel; chunk i
    draws from the i-th child of SeedSequence(seed)."""
    starts = list(range(0, n_rows, chunk))
    kids = np.random.SeedSequence(seed).spawn(len(starts))

    def run(i):
        s = starts[i]
        fn(np.random.Generator(np.random.PCG64(kids[i])), s, min(n_rows, s + chunk))

    with ThreadPoolExecutor(_threads()) as ex:
        list(ex.map(run, range(len(starts))))


def plumbing(n_rows: int = 100_000, seed: int = 1):
    rng = np.random.default_rng(seed)
    w = rng.normal(0.0, 0.5, 28).astype(np.float32)
    X = np.empty((n_rows, 28), np.float32)
    y = np.empty(n_rows, np.float32)

    def fill(g, s, e):
        g.standard_normal((e - s, 28), dtype=np.float32, out=X[s:e])
        y[s:e] = g.random(e - s) < _sigmoid(_dot(X[s:e], w))

    _chunked(n_rows, seed + 1000, fill)
    params = {"objective": "binary:logistic", "max_depth": 6, "eta": 0.1, "max_bin": 256,
              "grow_policy": "depthwise"}
    return X, y, params, {"rounds": 100}


def narrow_binary(n_rows: int = 10_500_000, seed: int = 2, max_bin: int = 256):
    rng = np.random.default_rng(seed)
    coef = rng.normal(0.0, 0.6, 28)
    X = np.empty((n_rows, 28), np.float32)
    z = np.empty(n_rows, np.float64)
    pairs = [(0, 1), (2, 3), (4, 11), (5, 12), (6, 13), (7, 8), (9, 14)]

    def fill(g, s, e):
        m = e - s
        X[s:e, :11] = g.standard_normal((m, 11), dtype=np.float32)
        X[s:e, 11:21] = np.abs(g.standard_normal((m, 10), dtype=np.float32))
        for k, (i, j) in enumerate(pairs):
            v = X[s:e, i] * X[s:e, j] if k % 2 == 0 else X[s:e, i] + X[s:e, j]
            X[s:e, 21 + k] = np.exp(0.5 * np.clip(v, -20, 20)).astype(np.float32)
        # nonlinear logistic with three interaction terms
        Xs = X[s:e].astype(np.float64)
        z[s:e] = (_dot(Xs[:, :21], coef[:21]) + 0.8 * Xs[:, 0] * Xs[:, 3]
                  - 0.6 * Xs[:, 11] * Xs[:, 2] + 0.5 * np.tanh(Xs[:, 22] - Xs[:, 25])
                  + 0.1 * np.log1p(Xs[:, 21:28]).sum(axis=1))

    _chunked(n_rows, seed + 1000, fill, 1 << 18)
    z += 0.12 - np.median(z)  # the intercept sets ~53% positives
    y = np.empty(n_rows, np.float32)

    def label(g, s, e):
        y[s:e] = g.random(e - s) < _sigmoid(z[s:e])

    _chunked(n_rows, seed + 2000, label, 1 << 18)
    params = {"objective": "binary:logistic", "max_depth": 8, "eta": 0.1, "max_bin": max_bin,
              "grow_policy": "depthwise"}
    return X, y, params, {"rounds": 500}


def narrow_multiclass(n_rows: int = 10_500_000, n_classes: int = 4, seed: int = 2,
                      max_bin: int = 255):
    """The narrow 28-feature rows with K balanced classes: the quantile bins of a
    nonlinear score plus logistic noise (multi:softprob, depth 8, eta 0.1)."""
    X, _, _, _ = narrow_binary(n_rows, seed=seed, max_bin=max_bin)
    s = np.empty(n_rows, np.float64)

    def score(g, a, b):
        Xs = X[a:b].astype(np.float64)
        s[a:b] = (Xs[:, 0] + 0.8 * Xs[:, 3] * Xs[:, 1] - 0.5 * Xs[:, 11] + 0.3 * Xs[:, 22]
                  + g.logistic(size=b - a) * 0.5)

    _chunked(n_rows, seed + 3000, score, 1 << 18)
    edges = np.quantile(s[:: max(1, n_rows // 200_000)], np.linspace(0, 1, n_classes + 1)[1:-1])
    y = np.searchsorted(edges, s).astype(np.float32)
    params = {"objective": "multi:softprob", "num_class": n_classes, "max_depth": 8, "eta": 0.1,
              "max_bin": max_bin, "grow_policy": "depthwise"}
    return X, y, params, {"rounds": 500}


def narrow_quantile(n_rows: int = 10_500_000, alphas=(0.1, 0.5, 0.9), seed: int = 2,
                    max_bin: int = 255):
    """The narrow 28-feature rows with a heteroscedastic continuous target
    (reg:quantileerror at the given quantiles, depth 8, eta 0.1)."""
    X, _, _, _ = narrow_binary(n_rows, seed=seed, max_bin=max_bin)
    y = np.empty(n_rows, np.float32)

    def target(g, a, b):
        Xs = X[a:b].astype(np.float64)
        y[a:b] = (1.5 * Xs[:, 0] - 0.7 * Xs[:, 11] * Xs[:, 2] + 0.4 * np.log1p(Xs[:, 21])
                  + g.standard_exponential(b - a) * (1.0 + np.abs(Xs[:, 4])))

    _chunked(n_rows, seed + 4000, target, 1 << 18)
    params = {"objective": "reg:quantileerror", "quantile_alpha": list(alphas), "max_depth": 8,
              "eta": 0.1, "max_bin": max_bin, "grow_policy": "depthwise"}
    return X, y, params, {"rounds": 500}


def wide_binary(n_rows: int = 400_000, n_features: int = 2000, seed: int = 3, max_bin: int = 256):
    rng = np.random.default_rng(seed)
    w = np.zeros(n_features)
    nz = rng.choice(n_features, size=min(200, n_features), replace=False)
    w[nz] = rng.standard_normal(nz.size)
    X = np.empty((n_rows, n_features), np.float32)
    y = np.empty(n_rows, np.float32)

    def fill(g, s, e):
        blk = X[s:e]
        g.standard_normal(blk.shape, dtype=np.float32, out=blk)
        blk /= np.linalg.norm(blk, axis=1, keepdims=True).astype(np.float32)
        lab = (_dot(blk, w) > 0).astype(np.float32)
        flip = g.random(e - s) < 0.05
        lab[flip] = 1.0 - lab[flip]
        y[s:e] = lab

    _chunked(n_rows, seed + 1000, fill, 1 << 13)
    params = {"objective": "binary:logistic", "max_depth": 8, "eta": 0.1, "max_bin": max_bin,
              "colsample_bytree": 0.5, "grow_policy": "depthwise"}
    return X, y, params, {"rounds": 200}


def widebin_cat(n_rows: int = 2_000_000, seed: int = 4, n_num: int = 80, n_cat: int = 20,
                n_codes: int = 500):
    rng = np.random.default_rng(seed)
    ranks = np.arange(1, n_codes + 1, dtype=np.float64)
    p = ranks ** -1.2
    p /= p.sum()
    cdf = np.cumsum(p)
    cdf[-1] = 1.0
    steps = [(f, rng.random(), rng.normal(), rng.normal()) for f in range(0, n_num, 4)]
    effects = [rng.normal(0, 1.0, n_codes) for _ in range(n_cat)]
    X = np.empty((n_rows, n_num + n_cat), np.float32)
    y = np.empty(n_rows, np.float32)

    def fill(g, s, e):
        m = e - s
        num = g.random((m, n_num), dtype=np.float32)
        num[g.random((m, n_num)) < 0.1] = np.nan
        # Zipf(1.2) codes by inverse CDF
        cat = np.searchsorted(cdf, g.random((m, n_cat)), side="right").astype(np.float32)
        np.minimum(cat, n_codes - 1, out=cat)
        X[s:e, :n_num] = num
        X[s:e, n_num:] = cat
        t = np.zeros(m, np.float64)
        for f, thr, lo, hi in steps:
            col = np.nan_to_num(num[:, f], nan=0.5)
            t += np.where(col < thr, lo, hi)
        for k in range(n_cat):
            t += effects[k][cat[:, k].astype(np.int64)]
        y[s:e] = t + g.normal(0, 0.1, m)

    _chunked(n_rows, seed + 1000, fill, 1 << 17)
    params = {"objective": "reg:squarederror", "max_bin": 1024, "grow_policy": "lossguide",
              "max_leaves": 255, "eta": 0.1, "feature_types": ["q"] * n_num + ["c"] * n_cat}
    return X, y, params, {"rounds": 300}


def streaming(n_rows: int = 50_000_000, n_features: int = 200, seed: int = 5):
    rng = np.random.default_rng(seed)
    w = rng.normal(0.0, 0.3, n_features)
    X = np.empty((n_rows, n_features), np.float32)
    y = np.empty(n_rows, np.float32)

    def fill(g, s, e):
        g.standard_normal((e - s, n_features), dtype=np.float32, out=X[s:e])
        y[s:e] = g.random(e - s) < _sigmoid(_dot(X[s:e], w))

    _chunked(n_rows, seed + 1000, fill, 1 << 17)
    params = {"objective": "binary:logistic", "max_depth": 8, "eta": 0.1, "max_bin": 256}
    return X, y, params, {"rounds": 100}
