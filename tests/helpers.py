"""Shared test helpers: golden fixtures and model comparison."""

from __future__ import annotations

import json
import os

import numpy as np

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
