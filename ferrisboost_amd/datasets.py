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
"""

from __future__ import annotations

import numpy as np


def _sigmoid(z):
    return 1.0 / (1.0 + np.exp(-z))


def plumbing(n_rows: int = 100_000, seed: int = 1):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n_rows, 28), dtype=np.float32)
    w = rng.normal(0.0, 0.5, 28).astype(np.float32)
    y = (rng.random(n_rows) < _sigmoid(X.astype(np.float64) @ w)).astype(np.float32)
    params = {"objective": "binary:logistic", "max_depth": 6, "eta": 0.1, "max_bin": 256,
              "grow_policy": "depthwise"}
    return X, y, params, {"rounds": 100}


def narrow_binary(n_rows: int = 10_500_000, seed: int = 2, max_bin: int = 256):
    rng = np.random.default_rng(seed)
    X = np.empty((n_rows, 28), np.float32)
    chunk = 1 << 20
    coef = rng.normal(0.0, 0.6, 28)
    for s in range(0, n_rows, chunk):
        e = min(n_rows, s + chunk)
        m = e - s
        a = rng.standard_normal((m, 11), dtype=np.float32)
        b = np.abs(rng.standard_normal((m, 10), dtype=np.float32))
        X[s:e, :11] = a
        X[s:e, 11:21] = b
        pairs = [(0, 1), (2, 3), (4, 11), (5, 12), (6, 13), (7, 8), (9, 14)]
        for k, (i, j) in enumerate(pairs):
            z = X[s:e, i] * X[s:e, j] if k % 2 == 0 else X[s:e, i] + X[s:e, j]
            X[s:e, 21 + k] = np.exp(0.5 * np.clip(z, -20, 20)).astype(np.float32)
    # nonlinear logistic with three interaction terms; intercept sets ~53% positives
    z = np.empty(n_rows, np.float64)
    for s in range(0, n_rows, chunk):
        e = min(n_rows, s + chunk)
        Xs = X[s:e].astype(np.float64)
        z[s:e] = (Xs[:, :21] @ coef[:21] + 0.8 * Xs[:, 0] * Xs[:, 3]
                  - 0.6 * Xs[:, 11] * Xs[:, 2] + 0.5 * np.tanh(Xs[:, 22] - Xs[:, 25])
                  + 0.1 * np.log1p(Xs[:, 21:28]).sum(axis=1))
    z += 0.12 - np.median(z)
    y = (rng.random(n_rows) < _sigmoid(z)).astype(np.float32)
    params = {"objective": "binary:logistic", "max_depth": 8, "eta": 0.1, "max_bin": max_bin,
              "grow_policy": "depthwise"}
    return X, y, params, {"rounds": 500}


def wide_binary(n_rows: int = 400_000, n_features: int = 2000, seed: int = 3, max_bin: int = 256):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n_rows, n_features), dtype=np.float32)
    X /= np.linalg.norm(X, axis=1, keepdims=True).astype(np.float32)
    w = np.zeros(n_features)
    nz = rng.choice(n_features, size=min(200, n_features), replace=False)
    w[nz] = rng.standard_normal(nz.size)
    y = (X.astype(np.float64) @ w > 0).astype(np.float32)
    flip = rng.random(n_rows) < 0.05
    y[flip] = 1.0 - y[flip]
    params = {"objective": "binary:logistic", "max_depth": 8, "eta": 0.1, "max_bin": max_bin,
              "colsample_bytree": 0.5, "grow_policy": "depthwise"}
    return X, y, params, {"rounds": 200}


def widebin_cat(n_rows: int = 2_000_000, seed: int = 4, n_num: int = 80, n_cat: int = 20,
                n_codes: int = 500):
    rng = np.random.default_rng(seed)
    num = rng.random((n_rows, n_num), dtype=np.float32)
    num[rng.random((n_rows, n_num)) < 0.1] = np.nan
    ranks = np.arange(1, n_codes + 1, dtype=np.float64)
    p = ranks ** -1.2
    p /= p.sum()
    cat = rng.choice(n_codes, size=(n_rows, n_cat), p=p).astype(np.float32)
    X = np.concatenate([num, cat], axis=1)
    y = np.zeros(n_rows, np.float64)
    for f in range(0, n_num, 4):
        t = rng.random()
        col = np.nan_to_num(num[:, f], nan=0.5)
        y += np.where(col < t, rng.normal(), rng.normal())
    for f in range(n_cat):
        effect = rng.normal(0, 0.5, n_codes)
        y += effect[cat[:, f].astype(np.int64)]
    y += rng.normal(0, 0.1, n_rows)
    params = {"objective": "reg:squarederror", "max_bin": 1024, "grow_policy": "lossguide",
              "max_leaves": 255, "eta": 0.1, "feature_types": ["q"] * n_num + ["c"] * n_cat}
    return X.astype(np.float32), y.astype(np.float32), params, {"rounds": 300}


def streaming(n_rows: int = 50_000_000, n_features: int = 200, seed: int = 5):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n_rows, n_features), dtype=np.float32)
    w = rng.normal(0.0, 0.3, n_features)
    z = np.empty(n_rows)
    chunk = 1 << 20
    for s in range(0, n_rows, chunk):
        e = min(n_rows, s + chunk)
        z[s:e] = X[s:e].astype(np.float64) @ w
    y = (rng.random(n_rows) < _sigmoid(z)).astype(np.float32)
    params = {"objective": "binary:logistic", "max_depth": 8, "eta": 0.1, "max_bin": 256}
    return X, y, params, {"rounds": 100}
