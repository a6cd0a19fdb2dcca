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
from . import frame_rows

__all__ = ["train", "sketch", "Cuts", "Model", "device_available", "__version__"]
__version__ = "0.1.0"

# Canonical name -> default, as python/ferrisboost/__init__.py:_DEFAULTS.
_DEFAULTS: dict[str, Any] = {
    "objective": "binary:logistic",
    "num_class": None,
    "quantile_alpha": None,
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
    "hip_host_binning": False,
    "hip_host_sketch": False,
}

_ALIASES = {
    "learning_rate": "eta",
    "reg_lambda": "lambda",
    "reg_alpha": "alpha",
    "n_jobs": "nthread",
    "random_state": "seed",
}

_OBJECTIVES = {"reg:squarederror": 0, "binary:logistic": 1, "multi:softprob": 2,
               "multi:softmax": 3, "reg:quantileerror": 4}
_OBJECTIVE_NAMES = {v: k for k, v in _OBJECTIVES.items()}
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
    # num_class (python/ferrisboost/__init__.py:281-286): an integer, not negative;
    # the multiclass objectives need at least 2.
    if out["num_class"] is not None:
        if isinstance(out["num_class"], bool) or int(out["num_class"]) != out["num_class"]:
            raise ValueError(f"num_class must be an integer, got {out['num_class']!r}")
        out["num_class"] = int(out["num_class"])
        if out["num_class"] < 0:
            raise ValueError("num_class must not be negative")
    if str(out["objective"]).startswith("multi:") and (out["num_class"] or 0) < 2:
        raise ValueError(f"{out['objective']} requires num_class >= 2, got {out['num_class']}")
    out["quantile_alpha"] = _normalize_quantile_alpha(out["quantile_alpha"], out["objective"])
    if out["grow_policy"] not in _GROW:
        raise ValueError(f"grow_policy must be depthwise or lossguide, got {out['grow_policy']!r}")
    if not 0 < int(out["max_bin"]) <= 65535:
        raise ValueError(f"max_bin must be in 1..=65535, got {out['max_bin']}")
    if num_boost_round < 1:
        raise ValueError(f"num_boost_round must be >= 1, got {num_boost_round}")
    gm = out["gpu_math"]
    if gm is not None:
        gm = str(gm)
        if gm not in ("exact", "fast"):
            raise ValueError(f'gpu_math must be "exact" or "fast", got {gm!r}; fast does not '
                             "guarantee byte-identical CPU/GPU models")
        out["gpu_math"] = gm
    # GPU knobs of python/ferrisboost/__init__.py:224-280, validated as there.
    if out["hist_streams"] is not None:
        out["hist_streams"] = int(out["hist_streams"])
        if out["hist_streams"] not in (1, 2):
            raise ValueError(f"hist_streams must be 1 or 2, got {out['hist_streams']}; omit it "
                             "to let it be chosen automatically")
    if out["resident_blocks"] is not None:
        out["resident_blocks"] = int(out["resident_blocks"])
        if out["resident_blocks"] < 0:
            raise ValueError(f"resident_blocks must not be negative, got {out['resident_blocks']};"
                             " omit it to let it be chosen automatically; 0 means pure streaming")
    if out["hist_nodes_per_batch"] is not None:
        v = int(out["hist_nodes_per_batch"])
        if not 1 <= v <= 32:
            raise ValueError(f"hist_nodes_per_batch must be in 1..=32, got {v}; 1 disables "
                             "multi-node batching")
        raise ValueError("hist_nodes_per_batch is not available on the ferrisboost_amd device "
                         "path: each level's histograms are planned and built in one launch on "
                         "the device; omit it")
    if out["device_quantize"] is not None and not bool(out["device_quantize"]):
        raise ValueError("device_quantize=False is not available on the ferrisboost_amd device "
                         "path: gradient pairs are always quantized on the device; omit it")
    if out["sampling_method"] != "uniform":
        raise ValueError("sampling_method must be uniform on the ferrisboost_amd device path")
    # src/training/mod.rs:1550-1565 (the reference's message names the key).
    for k in ("subsample", "colsample_bytree", "colsample_bylevel", "colsample_bynode"):
        out[k] = float(out[k])
        if not 0.0 < out[k] <= 1.0:
            raise ValueError(f"{k} must be in (0, 1], got {out[k]}")
    if out["interaction_constraints"]:
        raise ValueError("interaction_constraints are not available on the ferrisboost_amd device path")
    if out["feature_weights"] is not None:
        out["feature_weights"] = _feature_weights_spec(out["feature_weights"])
    out["num_boost_round"] = int(num_boost_round)
    return out


def _feature_weights_spec(raw):
    """feature_weights (src/python/feature_weights.rs:14-70): a mapping of
    feature names to weights, or a one-dimensional list / tuple / numpy array
    of weights by position."""
    if isinstance(raw, Mapping):
        named = {}
        for k, v in raw.items():
            if not isinstance(k, str):
                raise ValueError("feature_weights dictionary keys must be feature-name strings")
            named[k] = _one_weight(v, f"feature_weights[{k!r}]")
        return named
    if isinstance(raw, (str, bytes)) or not isinstance(raw, (list, tuple, np.ndarray)):
        raise ValueError("feature_weights must be a mapping, list, tuple, or one-dimensional "
                         "NumPy array")
    if isinstance(raw, np.ndarray) and raw.ndim != 1:
        raise ValueError("feature_weights NumPy array must be one-dimensional")
    out = [_one_weight(v, f"feature_weights[{i}]") for i, v in enumerate(raw)]
    if not out:
        raise ValueError("feature_weights positional vector must not be empty")
    return out


def _one_weight(v, where: str) -> float:
    if isinstance(v, (bool, np.bool_)):
        raise ValueError(f"{where} must be a number, not a boolean")
    try:
        f = float(v)
    except (TypeError, ValueError):
        raise ValueError(f"{where} must be a number") from None
    if not (np.isfinite(f) and f >= 0.0):
        raise ValueError("feature_weights must be finite and nonnegative")
    return f


def _resolve_feature_weights(spec, n_features: int, names: list[str] | None):
    """The weights by feature position (FeatureWeightsSpec::resolve,
    src/python/feature_weights.rs:72-): positional lists must match the
    feature count; names need the data's feature names."""
    if spec is None:
        return None
    if isinstance(spec, dict):
        if not names:
            raise ValueError("feature_weights given by name needs data with feature names "
                             "(a pyarrow Table or a Parquet file)")
        unknown = [k for k in spec if k not in names]
        if unknown:
            raise ValueError(f"feature_weights names unknown features {unknown}")
        w = np.ones(n_features, np.float32)
        for k, v in spec.items():
            w[names.index(k)] = v
    else:
        if len(spec) != n_features:
            raise ValueError(f"feature_weights has {len(spec)} entries, expected {n_features}")
        w = np.asarray(spec, np.float32)
    if not (w > 0).any():
        raise ValueError("feature_weights must contain at least one positive weight")
    return np.ascontiguousarray(w)


def _as_base_margin(margin, n: int, k: int) -> np.ndarray:
    """base_margin (python/ferrisboost/__init__.py:966-989): (n,) or (n, 1)
    for one output, (n, k) for several; finite. Returned class-major, as
    the driver takes it ([k][n] flattened)."""
    if hasattr(margin, "to_numpy") and not isinstance(margin, np.ndarray):
        margin = margin.to_numpy()
    arr = np.asarray(margin, dtype=np.float32)
    if arr.ndim == 1 and k == 1:
        arr = arr.reshape(-1, 1)
    if arr.ndim != 2 or arr.shape[1] != k:
        want = "(n,) or (n, 1)" if k == 1 else f"(n, {k})"
        raise ValueError(f"base_margin must have shape {want}, got {tuple(arr.shape)}")
    if arr.shape[0] != n:
        raise ValueError(f"training set: base_margin has {arr.size} values, expected {n} rows "
                         f"x {k} outputs = {n * k}")
    if not np.isfinite(arr).all():
        raise ValueError("base_margin contains NaN or inf; every starting margin must be finite")
    return np.ascontiguousarray(arr.T).reshape(-1)


def _n_outputs(p: dict[str, Any]) -> int:
    if p["objective"].startswith("multi:"):
        return int(p["num_class"])
    if p["objective"] == "reg:quantileerror":
        return len(p["quantile_alpha"])
    return 1


def _normalize_quantile_alpha(value: Any, objective: str) -> list[float] | None:
    """quantile_alpha (python/ferrisboost/__init__.py:362-383): required by
    reg:quantileerror (XGBoost has no default); a scalar is a one-element
    list; several values train one output (one tree a round) per quantile;
    each in [0, 1], ascending, at most 64."""
    if value is None:
        if objective == "reg:quantileerror":
            raise ValueError(
                "reg:quantileerror needs quantile_alpha (one or more ascending quantiles in [0, 1], "
                "e.g. 0.9 or [0.1, 0.5, 0.9])"
            )
        return None
    if isinstance(value, (list, tuple, np.ndarray)):
        flat = np.asarray(value, dtype=np.float64).ravel().tolist()
    else:
        flat = [float(value)]
    if not flat:
        raise ValueError("quantile_alpha must not be an empty list")
    for alpha in flat:
        if not 0.0 <= alpha <= 1.0:
            raise ValueError(f"quantile_alpha must be in [0, 1], got {alpha}")
    if any(a > b for a, b in zip(flat, flat[1:])):
        raise ValueError(
            f"quantile_alpha must be in ascending order (as XGBoost requires), got {flat}")
    if len(flat) > 64:
        raise ValueError(f"quantile_alpha accepts at most 64 quantiles, got {len(flat)}")
    return flat


def _params_struct(p: dict[str, Any], n_features: int, names: list[str] | None = None,
                   base_margin: np.ndarray | None = None) -> N.TrainParams:
    s = N.TrainParams()
    s.colsample_bylevel = float(p["colsample_bylevel"])
    s.colsample_bynode = float(p["colsample_bynode"])
    fw = _resolve_feature_weights(p["feature_weights"], n_features, names)
    if fw is not None:
        s._fw = fw  # the struct points into it
        s.feature_weights = fw.ctypes.data_as(C.POINTER(C.c_float))
    if base_margin is not None:
        s._bm = base_margin
        s.base_margin = base_margin.ctypes.data_as(C.POINTER(C.c_float))
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
    s.num_class = int(p["num_class"] or 0) if p["objective"].startswith("multi:") else 0
    if p["objective"] == "reg:quantileerror":
        alphas = np.ascontiguousarray(p["quantile_alpha"], np.float32)
        s._alphas = alphas  # the struct points into it
        s.n_quantile_alpha = alphas.size
        s.quantile_alpha = alphas.ctypes.data_as(C.POINTER(C.c_float))
    s.grow_policy = _GROW[p["grow_policy"]]
    s.max_cat_to_onehot = int(p["max_cat_to_onehot"])
    s.max_cat_threshold = int(p["max_cat_threshold"])
    if p["base_score"] is not None:
        s.base_score = float(p["base_score"])
        s.has_base_score = 1
    s.nthread = int(p["nthread"])
    s.device = _parse_device(p["device"])
    s.gpu_math = 1 if p["gpu_math"] == "fast" else 0
    budget = p["gpu_memory_budget"]
    s.gpu_memory_budget = int(budget) if budget else 0
    s.tile_bytes = int(p["hip_tile_bytes"])
    s.rows_per_block = int(p["hip_rows_per_block"])
    s.profile = 1 if p["hip_profile"] else 0
    s.host_sigmoid = 1 if p["hip_host_sigmoid"] else 0
    s.host_levels = 1 if p["hip_host_levels"] else 0
    s.sync_round = int(p["hip_sync_round"])
    s.hist_streams = int(p["hist_streams"] or 0)
    s.resident_limit = 0 if p["resident_blocks"] is None else int(p["resident_blocks"]) + 1
    s.host_binning = 1 if p["hip_host_binning"] else 0
    s.host_sketch = 1 if p["hip_host_sketch"] else 0
    return s


_F32_MAX = float(np.finfo(np.float32).max)
_IMPORTANCE = ("weight", "gain", "cover", "total_gain", "total_cover")


def _validate_missing(value) -> float:
    """validate_missing (src/source/mod.rs): NaN or a finite float32 other
    than the reserved largest float32."""
    v = float(value)
    if np.isnan(v):
        return float("nan")
    with np.errstate(over="ignore"):
        f = np.float32(v)
    if not np.isfinite(f):
        raise ValueError(f"missing must be NaN or a finite float32, got {value!r}")
    if abs(float(f)) == _F32_MAX:
        raise ValueError("missing must not be the largest float32 (it is reserved for split boundaries)")
    return float(f)


class Model:
    """A trained or loaded model (Model, src/model/tree.rs:213-290; the
    Python class of python/ferrisboost/_core.pyi:55-265)."""

    def __init__(self, handle, n_features: int, objective: str, device: int = 0):
        self._h = handle
        self._n_features = n_features
        self._objective = objective
        self._device = device
        self.stats: dict[str, float] = {}

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            N.train_lib().fbt_model_free(h)
            self._h = None

    # ---- properties of python/ferrisboost/_core.pyi:55-80
    @property
    def n_features(self) -> int:
        return self._n_features

    @property
    def objective(self) -> str:
        return self._objective

    @property
    def num_trees(self) -> int:
        return N.train_lib().fbt_model_n_trees(self._h)

    @property
    def num_class(self) -> int:
        """Outputs per row: num_class of a multiclass model, the number of
        quantile_alpha of a reg:quantileerror model, else 1."""
        return N.train_lib().fbt_model_num_outputs(self._h)

    @property
    def quantile_alpha(self) -> list[float] | None:
        """reg:quantileerror's quantiles; None for other models
        (src/python/mod.rs:3159-3166)."""
        L = N.train_lib()
        k = L.fbt_model_quantile_alpha(self._h, None, 0)
        if k == 0:
            return None
        out = np.zeros(k, np.float32)
        L.fbt_model_quantile_alpha(self._h, N.ptr(out), k)
        return [float(v) for v in out]

    def class_margins(self) -> np.ndarray:
        """A multi-output model's per-output intercepts (empty otherwise)."""
        k = self.num_class
        out = np.zeros(k if k > 1 else 0, np.float32)
        if k > 1:
            N.train_lib().fbt_model_class_margins(self._h, N.ptr(out))
        return out

    @property
    def feature_names(self) -> list[str]:
        """The feature column names of a Parquet or Arrow training input
        (empty for arrays)."""
        return list(getattr(self, "_feature_names", []))

    @property
    def best_iteration(self):
        return None

    @property
    def best_score(self):
        return None

    def evals_result(self) -> dict:
        return {}

    @property
    def base_score(self) -> float:
        return N.train_lib().fbt_model_base_score(self._h)

    @property
    def base_margin(self) -> float:
        return N.train_lib().fbt_model_base_margin(self._h)

    @property
    def scale_pos_weight(self) -> float:
        return N.train_lib().fbt_model_scale_pos_weight(self._h)

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
        """Training margins: (n,), or class-major (num_class, n) for a
        multiclass model."""
        k = self.num_class
        out = np.zeros((k, n_rows) if k > 1 else n_rows, np.float32)
        N.check_train(N.train_lib().fbt_model_train_margins(self._h, N.ptr(out), n_rows))
        return out

    # ---- prediction and explanation
    def _tree_range(self, n_trees, iteration_range) -> tuple[int, int]:
        total = self.num_trees
        if iteration_range is not None:
            if n_trees is not None:
                raise ValueError("iteration_range and n_trees cannot both be given: the former "
                                 "counts rounds, the latter counts trees")
            # Rounds: num_class trees each (Model::slice_rounds, src/model/tree.rs:428-455).
            k = self.num_class
            rounds = total // k
            begin, end = (int(v) for v in iteration_range)
            if begin < 0 or end < 0:
                raise ValueError("iteration_range bounds must be non-negative")
            end = rounds if end == 0 else end
            if end > rounds:
                raise ValueError(f"iteration_range end = {end} exceeds the model's {rounds} rounds")
            if begin > end:
                raise ValueError(f"iteration_range begin = {begin} is greater than end = {end}")
            return begin * k, end * k
        if n_trees is None:
            return 0, total
        if int(n_trees) < 0:
            raise ValueError("n_trees must be non-negative")
        return 0, min(int(n_trees), total)

    def predict(self, data, output_margin: bool = False, n_trees: int | None = None,
                header: bool = True, *, predict_threads: int = 0, use_gpu: bool = True,
                iteration_range: tuple[int, int] | None = None, pred_contribs: bool = False,
                approx_contribs: bool = False, pred_interactions: bool = False,
                pred_leaf: bool = False, missing: float = float("nan"), base_margin=None,
                strict_shape: bool = False, device: str | None = None) -> np.ndarray:
        """Model.predict (python/ferrisboost/_core.pyi:94-197).

        Margins (output_margin=True) or probabilities / values, in float32,
        over every tree or the trees n_trees / iteration_range select.
        Explanations, at most one per call and not with output_margin:
        pred_contribs (TreeSHAP, (n, F + 1), bias last; with approx_contribs
        the Saabas attribution), pred_interactions ((n, F + 1, F + 1)) and
        pred_leaf ((n, trees) leaf ids). base_margin replaces the intercept
        per row (and the bias of explanations); missing marks values scored
        as NaN; strict_shape adds the output-group axis.

        Explanations and, with use_gpu=True (the default on this device
        path), margins and values run on the GPU (`device`, default the
        training device); use_gpu=False scores margins and values on the
        host. Every result equals the reference CPU engine's bit for bit.
        """
        del header, predict_threads  # file inputs and CPU worker counts do not apply
        if isinstance(data, (str, bytes)) or hasattr(data, "__fspath__") or (
                isinstance(data, (list, tuple)) and data and isinstance(data[0], (str, bytes))):
            raise ValueError("file inputs are not available on the ferrisboost_amd device path; "
                             "pass an array")
        kinds = [pred_contribs, pred_interactions, pred_leaf]
        if sum(bool(k) for k in kinds) > 1:
            raise ValueError("pred_contribs, pred_interactions and pred_leaf are exclusive: one "
                             "type of prediction at a time")
        if approx_contribs and pred_interactions:
            raise ValueError("approx_contribs cannot be combined with pred_interactions")
        explain = any(kinds)
        if explain and output_margin:
            raise ValueError("output_margin cannot be combined with pred_contribs / "
                             "pred_interactions / pred_leaf: one type of prediction at a time")
        if _arrow_input(data):
            from . import arrow_rows

            X = arrow_rows.table_matrix(data, getattr(self, "_feature_names", None),
                                        getattr(self, "_categories", None), self.n_features,
                                        float("nan"))
        elif frame_rows.is_frame(data):
            df = frame_rows.select_columns(data, getattr(self, "_feature_names", None))
            is_cat = N.train_lib().fbt_model_is_categorical
            flags = [bool(is_cat(self._h, f)) for f in range(self.n_features)]
            X = frame_rows.frame_matrix(df, True, getattr(self, "_categories", None),
                                        what="predict data", scoring=True, categorical=flags)[0]
        else:
            X = np.asarray(data, dtype=np.float32)
        if X.ndim != 2 or X.shape[1] != self.n_features:
            raise ValueError(f"expected a 2-D array with {self.n_features} columns, got shape "
                             f"{X.shape}")
        X = np.ascontiguousarray(X)
        miss = _validate_missing(missing)
        if not np.isnan(miss):
            X = np.where(X == np.float32(miss), np.float32("nan"), X).astype(np.float32)
        n = X.shape[0]
        k = self.num_class
        bm = None
        if base_margin is not None:
            bm = np.asarray(base_margin, dtype=np.float32)
            if k > 1:
                # (n, num_class) rows; the backend takes it class-major.
                if bm.shape != (n, k):
                    raise ValueError(f"base_margin must have shape ({n}, {k}), got {bm.shape}")
                bm = np.ascontiguousarray(bm.T)
            else:
                bm = np.ascontiguousarray(bm.reshape(-1))
                if bm.shape != (n,):
                    raise ValueError(f"base_margin has {bm.size} values, expected {n} rows x 1 "
                                     "outputs")
        b, e = self._tree_range(n_trees, iteration_range)
        dev = _parse_device(device) if device is not None else self._device
        groups = (k,) if k > 1 else ()
        if pred_leaf:
            kind, shape = N.OUT_LEAF, (n, e - b)
        elif pred_interactions:
            kind = N.OUT_INTERACTIONS
            shape = (n,) + groups + (self.n_features + 1, self.n_features + 1)
        elif pred_contribs:
            kind = N.OUT_APPROX if approx_contribs else N.OUT_CONTRIBS
            shape = (n,) + groups + (self.n_features + 1,)
        else:
            kind = N.OUT_MARGIN if output_margin else N.OUT_VALUE
            # multi:softmax's values are class indices, one per row
            shape = (n,) if (not output_margin and self.objective == "multi:softmax") else (
                (n,) + groups)
            if not use_gpu:
                dev = -1
        out = np.zeros(shape, np.float32)
        N.check_train(N.train_lib().fbt_predict(self._h, N.ptr(X), n, self.n_features, kind, b, e,
                                                N.ptr(bm), dev, N.ptr(out)))
        if strict_shape:
            if pred_leaf:
                out = out.reshape(n, (e - b) // k, k, 1)
            elif k == 1 or out.ndim == 1:
                out = out.reshape((n, 1) + out.shape[1:])
        return out

    def get_score(self, importance_type: str = "weight") -> dict[str, float]:
        """Feature importance as XGBoost's Booster.get_score (feature_scores,
        src/model/explain.rs:57-114): split counts, or the gain / cover of
        the splits, averaged per split or summed."""
        if importance_type not in _IMPORTANCE:
            raise ValueError(f"importance_type must be one of {', '.join(_IMPORTANCE)}, got "
                             f"{importance_type!r}")
        count = np.zeros(self.n_features, np.float64)
        gain = np.zeros(self.n_features, np.float64)
        cover = np.zeros(self.n_features, np.float64)
        for t in self.trees():
            for nd in t[t["is_leaf"] == 0]:
                f = int(nd["feat"])
                count[f] += 1
                gain[f] += float(nd["gain"])
                cover[f] += float(nd["sum_hess"])
        out = {}
        for f in range(self.n_features):
            if count[f] == 0:
                continue
            v = {"weight": count[f], "gain": gain[f] / count[f], "cover": cover[f] / count[f],
                 "total_gain": gain[f], "total_cover": cover[f]}[importance_type]
            out[f"f{f}"] = float(v)
        return out

    def get_categories(self):
        """Category names by feature (python/ferrisboost/_core.pyi; Model::
        categories, src/data/category_names.rs): a list of the categories in
        code order for a categorical feature trained from named categories
        (an Arrow string dictionary or string column), None for any other
        feature; None instead of a list when no feature has names. Kept on
        this object only: the model JSON does not carry them."""
        cats = getattr(self, "_categories", None)
        return None if cats is None else [None if c is None else list(c) for c in cats]

    def to_json(self) -> str:
        L = N.train_lib()
        n = L.fbt_model_to_json(self._h, None, 0)
        buf = C.create_string_buffer(n + 1)
        L.fbt_model_to_json(self._h, buf, n + 1)
        return buf.value.decode()

    def save_model(self, path: str, quiet: bool | None = None,
                   model_io_threads: int | None = None) -> None:
        """XGBoost-compatible JSON (Model::to_xgboost_json, src/model/tree.rs:600-752)."""
        del quiet, model_io_threads
        with open(path, "w") as f:
            f.write(self.to_json())

    @staticmethod
    def load_model(path: str, quiet: bool = False, model_io_threads: int = 0,
                   ingest_threads: int = 0, device: str | None = None) -> "Model":
        """XGBoost-compatible JSON (Model::from_xgboost_json,
        src/model/tree.rs:754-990): binary:logistic and reg:squarederror
        models load; anything the reader cannot represent is a ValueError."""
        del quiet, model_io_threads, ingest_threads
        with open(path, "rb") as f:
            return Model.from_json(f.read(), device=device)

    @staticmethod
    def from_json(text, device: str | None = None) -> "Model":
        raw = text.encode() if isinstance(text, str) else bytes(text)
        L = N.train_lib()
        h = C.c_void_p()
        N.check_train(L.fbt_model_from_json(raw, len(raw), C.byref(h)))
        obj = _OBJECTIVE_NAMES[L.fbt_model_objective(h)]
        return Model(h, L.fbt_model_n_features(h), obj, _parse_device(device))


class Cuts:
    """Quantile cuts of a matrix (BinCuts, src/data/columns.rs:50-360): the
    sketch of one training matrix, reusable by several train() calls on the
    same data (no reference counterpart: the reference sketches per source)."""

    def __init__(self, values: np.ndarray, offsets: np.ndarray, max_bin: int,
                 categorical: np.ndarray | None):
        self.values = np.ascontiguousarray(values, np.float32)
        self.offsets = np.ascontiguousarray(offsets, np.uint32)
        self.max_bin = int(max_bin)
        self.categorical = None if categorical is None else np.ascontiguousarray(categorical, np.uint8)


def _categorical_flags(feature_types, n_features):
    if feature_types is None:
        return None
    if len(feature_types) != n_features:
        raise ValueError("feature_types must have one entry per feature")
    return np.array([1 if t == "c" else 0 for t in feature_types], np.uint8)


def _matrix(X, missing):
    X = np.asarray(X, dtype=np.float32)
    if X.ndim != 2:
        raise ValueError("X must be a 2-D array")
    X = np.ascontiguousarray(X)
    if missing is not None and not (isinstance(missing, float) and np.isnan(missing)):
        X = np.where(X == np.float32(missing), np.float32("nan"), X).astype(np.float32)
    return X


def sketch(X, max_bin: int = 255, weight=None, feature_types=None,
           missing: float = float("nan")) -> Cuts:
    """The cuts train() would sketch for this matrix (FeatureSketch::cuts,
    src/data/sketch.rs:236-275, one sketch per feature): pass them to
    train(..., cuts=) to train several models without sketching again."""
    X = _matrix(X, missing)
    if not 0 < int(max_bin) <= 65535:
        raise ValueError(f"max_bin must be in 1..=65535, got {max_bin}")
    n, nf = X.shape
    w = None if weight is None else np.ascontiguousarray(np.asarray(weight, dtype=np.float32))
    cat = _categorical_flags(feature_types, nf)
    cap = sum(65534 if (cat is not None and cat[f]) else max(int(max_bin), 2) for f in range(nf))
    vals = np.zeros(cap + 1, np.float32)
    offs = np.zeros(nf + 1, np.uint32)
    N.check_train(N.train_lib().fbt_sketch_cuts(N.ptr(X), n, nf, int(max_bin), N.ptr(w), N.ptr(cat),
                                                N.ptr(vals), N.ptr(offs)))
    return Cuts(vals[: offs[-1]].copy(), offs, max_bin, cat)


def _monotone(mc, names: list[str] | None) -> np.ndarray | None:
    """monotone_constraints -> one int8 sign per feature (None for none): a
    "(1,0,-1)" string, a sequence, or a {column name: sign} mapping for
    inputs with column names (python/ferrisboost/__init__.py:422-426)."""
    if not mc:
        return None
    if isinstance(mc, Mapping):
        if names is None:
            raise ValueError("monotone_constraints given by column name needs column names: a "
                             "numpy array has none; use a positional tuple, or a DataFrame, a "
                             "pyarrow Table or a Parquet file")
        unknown = [k for k in mc if k not in names]
        if unknown:
            raise ValueError(f"monotone_constraints columns {unknown} are not feature columns; "
                             f"feature columns: {names}")
        mc = [mc.get(n, 0) for n in names]
    elif isinstance(mc, str):
        mc = [int(v) for v in mc.strip("()").split(",") if v.strip()]
    return np.ascontiguousarray([int(np.sign(v)) for v in mc], np.int8)


def _arrow_input(data) -> bool:
    from . import arrow_rows

    if arrow_rows.is_path(data):
        return True
    mod = type(data).__module__ or ""
    return mod.startswith("pyarrow")


def _train_arrow(p: dict[str, Any], data, label, weight, cuts, base_margin) -> Model:
    """train() on a .parquet path or a pyarrow Table / RecordBatchReader: the
    label (and weight) are column names (or arrays for a table); the feature
    rows stream through fbt_train_rows (python/ferrisboost/__init__.py:
    1090-1230)."""
    from . import arrow_rows

    if cuts is not None:
        raise ValueError("cuts= takes a numpy matrix; Parquet and Arrow inputs sketch their own")
    if arrow_rows.is_path(data):
        path = str(data).lower()
        if not (path.endswith(".parquet") or path.endswith(".pq")):
            raise ValueError(f"cannot tell the format of {str(data)!r} from its extension; "
                             "supported: .parquet / .pq")
    src = arrow_rows.ArrowRows(data, label, weight, p["enable_categorical"], p["missing"])
    types = arrow_rows.feature_types_of(src, p["feature_types"])
    cat = _categorical_flags(types, src.n_features)
    mono = _monotone(p["monotone_constraints"], list(src.features))
    bm = None if base_margin is None else _as_base_margin(base_margin, src.n_rows, _n_outputs(p))
    s = _params_struct(p, src.n_features, list(src.features), bm)
    h = C.c_void_p()
    L = N.train_lib()
    errors: list = []
    fn = src.as_callback(errors)
    rc = L.fbt_train_rows(fn, None, src.n_rows, src.n_features, N.ptr(src.labels),
                          N.ptr(src.weights), N.ptr(cat), N.ptr(mono),
                          0 if mono is None else mono.size, C.byref(s), C.byref(h))
    if errors:
        raise errors[0]
    N.check_train(rc)
    m = Model(h, src.n_features, p["objective"], s.device)
    m._feature_names = list(src.features)
    m._categories = arrow_rows.categories_of(src, types)
    st = N.Stats()
    N.check_train(L.fbt_last_stats(C.byref(st)))
    m.stats = {k: getattr(st, k) for k, _ in N.Stats._fields_}
    return m


# train() arguments of the reference that this device path leaves out:
# validation sets and what hangs off them, training continuation, ranking
# groups and survival bounds (outside the histogram / split / partition path).
_UNSUPPORTED_ARGS = {
    "evals": "validation sets (evals) are not available on the ferrisboost_amd device path",
    "early_stopping_rounds": "early stopping needs validation sets, which the ferrisboost_amd "
                             "device path does not take",
    "callbacks": "callbacks are not available on the ferrisboost_amd device path",
    "base_margin_eval_set": "validation sets (and their margins) are not available on the "
                            "ferrisboost_amd device path",
    "init_model": "training continuation (init_model) is not available on the ferrisboost_amd "
                  "device path",
    "xgb_model": "training continuation (xgb_model) is not available on the ferrisboost_amd "
                 "device path",
    "qid": "ranking objectives (qid) are not available on the ferrisboost_amd device path",
    "group": "ranking objectives (group) are not available on the ferrisboost_amd device path",
    "eval_qid": "ranking objectives are not available on the ferrisboost_amd device path",
    "eval_group": "ranking objectives are not available on the ferrisboost_amd device path",
    "label_lower_bound": "survival:aft is not available on the ferrisboost_amd device path",
    "label_upper_bound": "survival:aft is not available on the ferrisboost_amd device path",
}


def train(params: Mapping[str, Any], data, label=None, num_boost_round: int = 10,
          evals=(), early_stopping_rounds=None, evals_result: dict | None = None,
          verbose_eval=False, callbacks=None, header: bool = True, quiet: bool = False,
          weight=None, feature_types=None, base_margin=None, base_margin_eval_set=None,
          init_model=None, xgb_model=None, qid=None, group=None, eval_qid=None,
          eval_group=None, label_lower_bound=None, label_upper_bound=None, *,
          cuts: Cuts | None = None) -> Model:
    """fb.train on the device path, with the reference's signature
    (python/ferrisboost/__init__.py:1090-1114): train(params, data, label,
    num_boost_round, evals, ...).

    data is a 2-D array (label, weight and base_margin arrays), a pandas
    DataFrame (category columns need params["enable_categorical"]; the
    column names become the feature names, which predict() binds by), a
    .parquet path (label and weight name columns) or a pyarrow Table /
    RecordBatchReader (label and weight name columns or are arrays; the
    other columns are the features, streamed to the device in chunks for the
    sketch and the binning). base_margin gives every row's starting raw
    margin, (n,) or (n, num_outputs); the intercept is still estimated from
    the labels and stored. feature_types ("q" / "c" per feature) overrides
    params["feature_types"]. cuts (from sketch() on the same matrix, max_bin
    and feature_types) replaces the sketch. Validation sets, early stopping,
    callbacks, training continuation, ranking groups and survival bounds are
    not part of this path: passing them is a ValueError."""
    given = {"evals": evals, "early_stopping_rounds": early_stopping_rounds,
             "callbacks": callbacks, "base_margin_eval_set": base_margin_eval_set,
             "init_model": init_model, "xgb_model": xgb_model, "qid": qid, "group": group,
             "eval_qid": eval_qid, "eval_group": eval_group,
             "label_lower_bound": label_lower_bound, "label_upper_bound": label_upper_bound}
    for k, v in given.items():
        if v is not None and not (k == "evals" and len(v) == 0):
            raise ValueError(_UNSUPPORTED_ARGS[k])
    if isinstance(num_boost_round, bool) or not isinstance(num_boost_round, (int, np.integer)):
        raise ValueError(f"num_boost_round must be an integer, got {num_boost_round!r}")
    del verbose_eval, header, quiet  # no evaluation log; files are Parquet only
    if evals_result is not None:
        evals_result.clear()  # no validation sets, so no metric history
    if feature_types is not None:
        params = dict(params, feature_types=list(feature_types))
    p = _normalize(params, num_boost_round)
    if _arrow_input(data):
        return _train_arrow(p, data, label, weight, cuts, base_margin)
    if label is None:
        raise ValueError("label is required for array inputs")
    names = lists = None
    if frame_rows.is_frame(data):
        data, names, auto, lists = frame_rows.frame_matrix(data, p["enable_categorical"])
        if p["feature_types"] is None and any(auto):
            p["feature_types"] = ["c" if f else "q" for f in auto]
    X = _matrix(data, p["missing"])
    y = np.ascontiguousarray(np.asarray(label, dtype=np.float32))
    if y.shape != (X.shape[0],):
        raise ValueError(f"label has {y.size} rows, but the training data has {X.shape[0]} rows")
    w = None if weight is None else np.ascontiguousarray(np.asarray(weight, dtype=np.float32))
    if w is not None and w.shape != (X.shape[0],):
        raise ValueError("weight must have one value per row")
    cat = _categorical_flags(p["feature_types"], X.shape[1])
    mono = _monotone(p["monotone_constraints"], names)
    bm = None if base_margin is None else _as_base_margin(base_margin, X.shape[0], _n_outputs(p))
    s = _params_struct(p, X.shape[1], names, bm)
    h = C.c_void_p()
    L = N.train_lib()
    if cuts is None:
        N.check_train(L.fbt_train(
            N.ptr(X), X.shape[0], X.shape[1], N.ptr(y), N.ptr(w), N.ptr(cat), N.ptr(mono),
            0 if mono is None else mono.size, C.byref(s), C.byref(h)))
    else:
        if cuts.max_bin != int(p["max_bin"]) or cuts.offsets.size != X.shape[1] + 1:
            raise ValueError("cuts were sketched for another max_bin or feature count")
        N.check_train(L.fbt_train_cuts(
            N.ptr(X), X.shape[0], X.shape[1], N.ptr(y), N.ptr(w), N.ptr(cat), N.ptr(mono),
            0 if mono is None else mono.size, C.byref(s), N.ptr(cuts.values), N.ptr(cuts.offsets),
            C.byref(h)))
    m = Model(h, X.shape[1], p["objective"], s.device)
    if names is not None:
        m._feature_names = names
        kept = [c if (cat is not None and cat[j]) else None for j, c in enumerate(lists)]
        m._categories = kept if any(c is not None for c in kept) else None
    st = N.Stats()
    N.check_train(L.fbt_last_stats(C.byref(st)))
    m.stats = {k: getattr(st, k) for k, _ in N.Stats._fields_}
    return m
