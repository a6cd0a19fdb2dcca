"""ferrisboost_amd -- the MI355X (gfx950) device path of FerrisBoost.

A drop-in for the `device="cuda"` training and explanation path of
FerrisBoost (python/ferrisboost/__init__.py): the same parameter names,
defaults, aliases and error classes (ValueError for bad input, RuntimeError
for device failures), running every histogram, split scan, partition, leaf
scatter and TreeSHAP evaluation on hand-written HIP kernels through the C ABI
of include/fbhip.h, driven by the C++ round driver of include/fbtrain.h.

    import ferrisboost_amd as fb
    model = fb.train({"objective": "binary:logistic", "max_depth": 8, "eta": 0.1,
                      "device": "cuda"}, X, label=y, num_boost_round=100)
    margins = model.predict(X, output_margin=True)
    contribs = model.predict(X, pred_contribs=True)
    model.save_model("m.json")      # XGBoost schema

This package has no CPU fallback: without a gfx950 device every training or
explanation call raises RuntimeError.
"""

from __future__ import annotations

import ctypes as C
from typing import Any, Mapping

import numpy as np

from . import _native as N

__all__ = ["train", "Model", "device_available", "__version__"]
__version__ = "0.1.0"

# Canonical name -> default, as python/ferrisboost/__init__.py:_DEFAULTS.
_DEFAULTS: dict[str, Any] = {
    "objective": "binary:logistic",
    "max_depth": 6,
    "max_leaves": 0,
    "grow_policy": "depthwise",
    "max_bin": 255,
    "eta": 0.3,
    "lambda": 1.0,
    "gamma": 0.0,
    "alpha": 0.0,
    "max_delta_step": None,
    "scale_pos_weight": 1.0,
    "min_child_weight": 1.0,
    "subsample": 1.0,
    "sampling_method": "uniform",
    "colsample_bytree": 1.0,
    "colsample_bylevel": 1.0,
    "colsample_bynode": 1.0,
    "cols_per_block": None,
    "nthread": 0,
    "hist_streams": None,
    "resident_blocks": None,
    "hist_nodes_per_batch": None,
    "gpu_math": None,
    "device": None,
    "gpu_memory_budget": None,
    "device_quantize": None,
    "seed": 0,
    "base_score": None,
    "feature_weights": None,
    "monotone_constraints": None,
    "interaction_constraints": None,
    "enable_categorical": False,
    "feature_types": None,
    "missing": float("nan"),
    "max_cat_to_onehot": 4,
    "max_cat_threshold": 64,
    "eval_metric": None,
    # device-backend tuning (no reference counterpart)
    "hip_tile_bytes": 0,
    "hip_rows_per_block": 0,
    "hip_profile": False,
    "hip_host_sigmoid": False,
    "hip_host_levels": False,
    "hip_sync_round": 0,
}

_ALIASES = {
    "learning_rate": "eta",
    "reg_lambda": "lambda",
    "reg_alpha": "alpha",
    "n_jobs": "nthread",
    "random_state": "seed",
}

_OBJECTIVES = {"reg:squarederror": 0, "binary:logistic": 1}
_GROW = {"depthwise": 0, "lossguide": 1}

_UNIMPLEMENTED = {
    "tree_method": "hist is the only tree method; do not set it",
    "num_parallel_tree": "random forest mode is not supported",
}


def device_available(device: int = 0) -> bool:
    """True when a gfx950 GPU with this index is usable."""
    return N.device_available(device)


def _parse_device(value) -> int:
    if value is None:
        return 0
    if isinstance(value, str):
        v = value.strip().lower()
        if v == "cuda" or v == "gpu":
            return 0
        if v.startswith("cuda:"):
            idx = v[5:]
            if idx.isdigit():
                return int(idx)
        if v == "cpu":
            raise ValueError(
                'device="cpu" selects the reference CPU engine; this package is the device path '
                '(use device="cuda" or "cuda:N")'
            )
    raise ValueError(f'device must be "cuda" or "cuda:N", got {value!r}')


def _normalize(params: Mapping[str, Any], num_boost_round: int) -> dict[str, Any]:
    out = dict(_DEFAULTS)
    for key, value in dict(params).items():
        canon = _ALIASES.get(key, key)
        if canon in _UNIMPLEMENTED:
            raise ValueError(f"parameter {key!r}: {_UNIMPLEMENTED[canon]}")
        if canon not in _DEFAULTS:
            known = ", ".join(sorted(_DEFAULTS) + sorted(_ALIASES))
            raise ValueError(f"unknown parameter {key!r}; supported parameters: {known}")
        out[canon] = value
    if out["objective"] not in _OBJECTIVES:
        raise ValueError(
            f"objective {out['objective']!r} is not available on the ferrisboost_amd device path; "
            f"supported: {', '.join(_OBJECTIVES)}"
        )
    if out["grow_policy"] not in _GROW:
        raise ValueError(f"grow_policy must be depthwise or lossguide, got {out['grow_policy']!r}")
    if not 0 < int(out["max_bin"]) <= 65535:
        raise ValueError(f"max_bin must be in 1..=65535, got {out['max_bin']}")
    if num_boost_round < 1:
        raise ValueError(f"num_boost_round must be >= 1, got {num_boost_round}")
    gm = out["gpu_math"]
    if gm not in (None, "exact"):
        if gm == "fast":
            raise ValueError('gpu_math="fast" is not available in ferrisboost_amd; use "exact"')
        raise ValueError(f'gpu_math must be "exact" or "fast", got {gm!r}')
    if out["sampling_method"] != "uniform":
        raise ValueError("sampling_method must be uniform on the ferrisboost_amd device path")
    for k in ("colsample_bylevel", "colsample_bynode"):
        if float(out[k]) != 1.0:
            raise ValueError(f"{k} < 1 is not available on the ferrisboost_amd device path")
    if out["interaction_constraints"]:
        raise ValueError("interaction_constraints are not available on the ferrisboost_amd device path")
    if out["feature_weights"] is not None:
        raise ValueError("feature_weights are not available on the ferrisboost_amd device path")
    out["num_boost_round"] = int(num_boost_round)
    return out


def _params_struct(p: dict[str, Any], n_features: int) -> N.TrainParams:
    s = N.TrainParams()
    s.n_rounds = p["num_boost_round"]
    s.max_depth = int(p["max_depth"])
    s.max_leaves = int(p["max_leaves"])
    s.max_bin = int(p["max_bin"])
    s.learning_rate = float(p["eta"])
    s.lambda_ = float(p["lambda"])
    s.gamma = float(p["gamma"])
    s.min_child_weight = float(p["min_child_weight"])
    s.alpha = float(p["alpha"])
    s.max_delta_step = float(p["max_delta_step"] or 0.0)
    s.scale_pos_weight = float(p["scale_pos_weight"])
    s.subsample = float(p["subsample"])
    s.colsample_bytree = float(p["colsample_bytree"])
    cpb = p["cols_per_block"]
    s.cols_per_block = int(cpb) if cpb else max(n_features, 1)
    s.seed = int(p["seed"]) & 0xFFFFFFFFFFFFFFFF
    s.objective = _OBJECTIVES[p["objective"]]
    s.grow_policy = _GROW[p["grow_policy"]]
    s.max_cat_to_onehot = int(p["max_cat_to_onehot"])
    s.max_cat_threshold = int(p["max_cat_threshold"])
    if p["base_score"] is not None:
        s.base_score = float(p["base_score"])
        s.has_base_score = 1
    s.nthread = int(p["nthread"])
    s.device = _parse_device(p["device"])
    s.gpu_math = 0
    budget = p["gpu_memory_budget"]
    s.gpu_memory_budget = int(budget) if budget else 0
    s.tile_bytes = int(p["hip_tile_bytes"])
    s.rows_per_block = int(p["hip_rows_per_block"])
    s.profile = 1 if p["hip_profile"] else 0
    s.host_sigmoid = 1 if p["hip_host_sigmoid"] else 0
    s.host_levels = 1 if p["hip_host_levels"] else 0
    s.sync_round = int(p["hip_sync_round"])
    return s


class Model:
    """A trained model (Model, src/model/tree.rs:213-290)."""

    def __init__(self, handle, n_features: int, objective: str):
        self._h = handle
        self.n_features = n_features
        self.objective = objective
        self.stats: dict[str, float] = {}

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            N.train_lib().fbt_model_free(h)
            self._h = None

    @property
    def num_trees(self) -> int:
        return N.train_lib().fbt_model_n_trees(self._h)

    @property
    def base_score(self) -> float:
        return N.train_lib().fbt_model_base_score(self._h)

    @property
    def base_margin(self) -> float:
        return N.train_lib().fbt_model_base_margin(self._h)

    def tree_nodes(self, t: int) -> np.ndarray:
        L = N.train_lib()
        out = np.zeros(L.fbt_model_tree_len(self._h, t), N.NODE_DTYPE)
        L.fbt_model_tree_nodes(self._h, t, N.ptr(out))
        return out

    def trees(self) -> list[np.ndarray]:
        return [self.tree_nodes(t) for t in range(self.num_trees)]

    def cat_words(self) -> np.ndarray:
        L = N.train_lib()
        n = L.fbt_model_n_cat_words(self._h)
        out = np.zeros(n, np.uint32)
        if n:
            L.fbt_model_cat_words(self._h, N.ptr(out))
        return out

    def cuts(self) -> tuple[np.ndarray, np.ndarray]:
        L = N.train_lib()
        vals = np.zeros(L.fbt_model_n_cuts(self._h), np.float32)
        offs = np.zeros(self.n_features + 1, np.uint32)
        L.fbt_model_cuts(self._h, N.ptr(vals), N.ptr(offs))
        return vals, offs

    def train_margins(self, n_rows: int) -> np.ndarray:
        out = np.zeros(n_rows, np.float32)
        N.check_train(N.train_lib().fbt_model_train_margins(self._h, N.ptr(out), n_rows))
        return out

    def predict(self, X, output_margin: bool = False, pred_contribs: bool = False,
                device: str | None = "cuda") -> np.ndarray:
        """Margins (output_margin=True), probabilities / values, or SHAP
        contributions [n_rows, n_features + 1] with the bias last
        (pred_contribs=True, computed on the device)."""
        X = np.ascontiguousarray(X, np.float32)
        if X.ndim != 2 or X.shape[1] != self.n_features:
            raise ValueError(f"expected a 2-D array with {self.n_features} columns")
        if pred_contribs:
            out = np.zeros((X.shape[0], self.n_features + 1), np.float32)
            N.check_train(N.train_lib().fbt_shap(self._h, N.ptr(X), X.shape[0], X.shape[1],
                                                 _parse_device(device), N.ptr(out)))
            return out
        out = np.zeros(X.shape[0], np.float32)
        N.train_lib().fbt_predict_margin(self._h, N.ptr(X), X.shape[0], X.shape[1], N.ptr(out))
        if output_margin or self.objective == "reg:squarederror":
            return out
        return (1.0 / (1.0 + np.exp(-out))).astype(np.float32)

    def to_json(self) -> str:
        L = N.train_lib()
        n = L.fbt_model_to_json(self._h, None, 0)
        buf = C.create_string_buffer(n + 1)
        L.fbt_model_to_json(self._h, buf, n + 1)
        return buf.value.decode()

    def save_model(self, path: str) -> None:
        with open(path, "w") as f:
            f.write(self.to_json())


def train(params: Mapping[str, Any], X, label, weight=None, num_boost_round: int = 10) -> Model:
    """fb.train on the device path (python/ferrisboost/__init__.py:train)."""
    p = _normalize(params, num_boost_round)
    X = np.asarray(X, dtype=np.float32)
    if X.ndim != 2:
        raise ValueError("X must be a 2-D array")
    X = np.ascontiguousarray(X)
    miss = p["missing"]
    if miss is not None and not (isinstance(miss, float) and np.isnan(miss)):
        X = np.where(X == np.float32(miss), np.float32("nan"), X).astype(np.float32)
    y = np.ascontiguousarray(np.asarray(label, dtype=np.float32))
    if y.shape != (X.shape[0],):
        raise ValueError(f"label has {y.size} rows, but the training data has {X.shape[0]} rows")
    w = None if weight is None else np.ascontiguousarray(np.asarray(weight, dtype=np.float32))
    if w is not None and w.shape != (X.shape[0],):
        raise ValueError("weight must have one value per row")
    cat = None
    ft = p["feature_types"]
    if ft is not None:
        if len(ft) != X.shape[1]:
            raise ValueError("feature_types must have one entry per feature")
        cat = np.array([1 if t == "c" else 0 for t in ft], np.uint8)
    mono = None
    mc = p["monotone_constraints"]
    if mc:
        if isinstance(mc, str):
            mc = [int(v) for v in mc.strip("()").split(",") if v.strip()]
        mono = np.ascontiguousarray([int(np.sign(v)) for v in mc], np.int8)
    s = _params_struct(p, X.shape[1])
    h = C.c_void_p()
    N.check_train(N.train_lib().fbt_train(
        N.ptr(X), X.shape[0], X.shape[1], N.ptr(y), N.ptr(w), N.ptr(cat), N.ptr(mono),
        0 if mono is None else mono.size, C.byref(s), C.byref(h)))
    m = Model(h, X.shape[1], p["objective"])
    st = N.Stats()
    N.check_train(N.train_lib().fbt_last_stats(C.byref(st)))
    m.stats = {k: getattr(st, k) for k, _ in N.Stats._fields_ if k != "reserved"}
    return m
