"""Shared test helpers: golden fixtures and model comparison."""

from __future__ import annotations

import contextlib
import json
import os

import numpy as np

# The running pytest's config (set by conftest.py), for uncaptured().
PYTEST_CONFIG = None


@contextlib.contextmanager
def uncaptured():
    """Output written inside the block (by Python or by the native library)
    reaches the terminal at once instead of pytest's capture: long GPU steps
    print their progress as they go."""
    cm = PYTEST_CONFIG.pluginmanager.getplugin("capturemanager") if PYTEST_CONFIG else None
    if cm is None:
        yield
        return
    with cm.global_and_fixture_disabled():
        yield

FIXTURES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fixtures")
INDEXES = ("index.json", "weighted_index.json", "monotone_index.json")


def read_f32(path: str) -> np.ndarray:
    return np.fromfile(path, dtype="<f4")


def golden_cases():
    """Every XGBoost-3.4.1 golden case of the reference (tests/fixtures)."""
    out = []
    for idx in INDEXES:
        with open(os.path.join(FIXTURES, idx)) as f:
            meta = json.load(f)
        for c in meta["cases"]:
            out.append(c)
    return out


def load_case(c):
    base = os.path.join(FIXTURES, c["name"])
    x = read_f32(base + ".x").reshape(c["n_rows"], c["n_features"])
    y = read_f32(base + ".y")
    w = read_f32(base + ".w") if c.get("weights") else None
    want = read_f32(base + ".margin")
    return x, y, w, want


def case_params(c) -> dict:
    """Reference TrainParams of a fixture case (tests/bit_exact_vs_xgboost.rs:135-170)."""
    p = {
        "n_rounds": c["n_rounds"],
        "max_depth": c["max_depth"],
        "max_bin": c["max_bin"],
        "eta": c["eta"],
        "lambda": c["lambda"],
        "gamma": c["gamma"],
        "min_child_weight": c["min_child_weight"],
        "cols_per_block": c["cols_per_block"],
        "objective": c["objective"],
        "base_score": c["base_score"],
    }
    return p


def product_params(p: dict) -> dict:
    """Oracle-style keyword params -> ferrisboost_amd.train params."""
    out = dict(p)
    out.pop("n_rounds", None)
    out.pop("nthread", None)
    return out


def node_bytes(nodes: np.ndarray) -> bytes:
    """Node records without the padding field."""
    fields = [f for f in nodes.dtype.names if f != "pad"]
    return b"".join(nodes[f].tobytes() for f in fields)


def assert_same_models(oracle_model, product_model):
    """Byte-identical trees (every node field) and category sets."""
    ot, pt = oracle_model.trees(), product_model.trees()
    assert len(ot) == len(pt), f"{len(ot)} vs {len(pt)} trees"
    for t, (a, b) in enumerate(zip(ot, pt)):
        assert a.size == b.size, f"tree {t}: {a.size} vs {b.size} nodes"
        for f in a.dtype.names:
            if f == "pad":
                continue
            av, bv = a[f], b[f]
            if av.tobytes() != bv.tobytes():
                bad = np.nonzero(av.view(np.uint8).reshape(av.size, -1).any(axis=1)
                                 != bv.view(np.uint8).reshape(bv.size, -1).any(axis=1))[0]
                diff = np.nonzero(av != bv)[0]
                raise AssertionError(
                    f"tree {t} field {f} differs at nodes {diff[:8].tolist()}: "
                    f"{av[diff[:4]].tolist()} vs {bv[diff[:4]].tolist()} {bad[:0]}")
    assert np.array_equal(oracle_model.cat_words(), product_model.cat_words())


def wiggly(n, seed, nf=5):
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


def node_depths(tree) -> np.ndarray:
    """Depth of every node of a tree (structured node array)."""
    depth = np.zeros(tree.size, np.int64)
    for i in range(tree.size):
        if not tree["is_leaf"][i]:
            depth[tree["left"][i]] = depth[i] + 1
            depth[tree["right"][i]] = depth[i] + 1
    return depth
