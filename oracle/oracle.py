"""ctypes binding of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by the test suite, the smoke check and the
CPU-baseline leg of bench.py, only to check or time against. The shipped package
(ferrisboost_amd) never imports this module.
"""

from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")


def build(force: bool = False) -> str:
    """Compile oracle.cpp with g++ (no fast-math, no FMA contraction)."""
    src = os.path.join(HERE, "oracle.cpp")
    if force or not os.path.exists(LIB_PATH) or os.path.getmtime(LIB_PATH) < max(
        os.path.getmtime(src), os.path.getmtime(os.path.join(HERE, "oracle.h"))
    ):
        tmp = LIB_PATH + ".tmp"
        subprocess.check_call(
            ["g++", "-std=c++17", "-O2", "-ffp-contract=off", "-fPIC", "-shared", "-o", tmp, src,
             "-lpthread"]
        )
        os.replace(tmp, LIB_PATH)
    return LIB_PATH


class Params(C.Structure):
    _fields_ = [
        ("n_rounds", C.c_uint32),
        ("max_depth", C.c_uint32),
        ("max_leaves", C.c_uint32),
        ("max_bin", C.c_uint32),
        ("learning_rate", C.c_float),
        ("lambda_", C.c_float),
        ("gamma", C.c_float),
        ("min_child_weight", C.c_float),
        ("alpha", C.c_float),
        ("max_delta_step", C.c_float),
        ("scale_pos_weight", C.c_float),
        ("subsample", C.c_float),
        ("colsample_bytree", C.c_float),
        ("cols_per_block", C.c_uint32),
        ("seed", C.c_uint64),
        ("objective", C.c_uint32),
        ("grow_policy", C.c_uint32),
        ("max_cat_to_onehot", C.c_uint32),
        ("max_cat_threshold", C.c_uint32),
        ("base_score", C.c_float),
        ("has_base_score", C.c_uint32),
        ("nthread", C.c_uint32),
        ("num_class", C.c_uint32),
        ("n_quantile_alpha", C.c_uint32),
        ("quantile_alpha", C.POINTER(C.c_float)),
        ("base_margin", C.POINTER(C.c_float)),
        ("colsample_bylevel", C.c_float),
        ("colsample_bynode", C.c_float),
        ("feature_weights", C.POINTER(C.c_float)),
    ]


class Node(C.Structure):
    _fields_ = [
        ("feat", C.c_uint32),
        ("split_cond", C.c_float),
        ("left", C.c_int32),
        ("right", C.c_int32),
        ("default_left", C.c_uint8),
        ("is_leaf", C.c_uint8),
        ("pad", C.c_uint16),
        ("leaf_value", C.c_float),
        ("gain", C.c_float),
        ("sum_hess", C.c_float),
        ("cat_begin", C.c_uint32),
        ("cat_len", C.c_uint32),
    ]


NODE_DTYPE = np.dtype(
    [
        ("feat", "<u4"),
        ("split_cond", "<f4"),
        ("left", "<i4"),
        ("right", "<i4"),
        ("default_left", "u1"),
        ("is_leaf", "u1"),
        ("pad", "<u2"),
        ("leaf_value", "<f4"),
        ("gain", "<f4"),
        ("sum_hess", "<f4"),
        ("cat_begin", "<u4"),
        ("cat_len", "<u4"),
    ]
)
assert NODE_DTYPE.itemsize == C.sizeof(Node) == 40


class Split(C.Structure):
    _fields_ = [
        ("found", C.c_uint32),
        ("feat", C.c_uint32),
        ("bin", C.c_uint32),
        ("gain", C.c_float),
        ("left", C.c_int64 * 2),
        ("right", C.c_int64 * 2),
        ("missing_left", C.c_uint32),
        ("n_cat_words", C.c_uint32),
        ("cats", C.c_uint64 * 1024),
    ]


OBJECTIVES = {"reg:squarederror": 0, "binary:logistic": 1, "multi:softprob": 2,
              "multi:softmax": 3, "reg:quantileerror": 4}
GROW = {"depthwise": 0, "lossguide": 1}

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        P = C.c_void_p
        L.orc_quantizer_from_bounds.argtypes = [C.c_double, C.c_double, C.c_uint64, P]
        L.orc_quantize.argtypes = [P, C.c_uint64, P, P, P]
        L.orc_quantize.restype = None
        L.orc_to_f64.argtypes = [P, C.c_uint64, P, P]
        L.orc_to_f64.restype = None
        L.orc_sketch_cuts.argtypes = [P, C.c_uint64, C.c_uint32, C.c_uint32, P, P, P, P]
        L.orc_find_bin.argtypes = [P, P, C.c_uint32, C.c_uint8, C.c_float]
        L.orc_find_bin.restype = C.c_uint32
        L.orc_hist_build.argtypes = [P, C.c_uint32, C.c_uint64, C.c_uint32, P, P, P, C.c_uint64, P]
        L.orc_hist_build.restype = None
        L.orc_node_sum.argtypes = [P, P, C.c_uint64, C.c_uint64, P]
        L.orc_node_sum.restype = None
        L.orc_best_split.argtypes = [
            P, C.c_uint32, P, P, P, P, C.POINTER(Params), P, C.c_uint32, C.c_uint32, C.c_float,
            C.c_float, P, C.c_uint32, P, C.c_uint32, C.POINTER(Split),
        ]
        L.orc_best_split.restype = None
        L.orc_partition.argtypes = [P, C.c_uint64, P, C.c_uint32, C.c_uint32, C.c_uint32, P,
                                    C.c_uint32, P]
        L.orc_partition.restype = C.c_uint64
        L.orc_train.argtypes = [P, C.c_uint64, C.c_uint32, P, P, P, P, C.c_uint32,
                                C.POINTER(Params), C.POINTER(C.c_void_p)]
        L.orc_model_from_nodes.argtypes = [P, P, C.c_uint32, P, C.c_uint32, C.c_uint32, C.c_float,
                                           C.POINTER(C.c_void_p)]
        L.orc_model_free.argtypes = [P]
        L.orc_model_free.restype = None
        L.orc_model_n_trees.argtypes = [P]
        L.orc_model_n_trees.restype = C.c_uint32
        L.orc_model_num_outputs.argtypes = [P]
        L.orc_model_num_outputs.restype = C.c_uint32
        L.orc_model_class_margins.argtypes = [P, P]
        L.orc_model_class_margins.restype = None
        L.orc_model_tree_len.argtypes = [P, C.c_uint32]
        L.orc_model_tree_len.restype = C.c_uint32
        L.orc_model_tree_nodes.argtypes = [P, C.c_uint32, P]
        L.orc_model_tree_nodes.restype = None
        L.orc_model_n_cat_words.argtypes = [P]
        L.orc_model_n_cat_words.restype = C.c_uint32
        L.orc_model_cat_words.argtypes = [P, P]
        L.orc_model_cat_words.restype = None
        L.orc_model_base_score.argtypes = [P]
        L.orc_model_base_score.restype = C.c_float
        L.orc_model_base_margin.argtypes = [P]
        L.orc_model_base_margin.restype = C.c_float
        L.orc_model_train_seconds.argtypes = [P]
        L.orc_model_train_seconds.restype = C.c_double
        L.orc_predict_margin.argtypes = [P, P, C.c_uint64, C.c_uint32, P]
        L.orc_predict_margin.restype = None
        L.orc_model_train_margins.argtypes = [P, P]
        L.orc_model_train_margins.restype = None
        L.orc_shap.argtypes = [P, P, C.c_uint64, C.c_uint32, P]
        L.orc_explain.argtypes = [P, C.c_uint32, P, C.c_uint64, C.c_uint32, P, P]
        L.orc_quadrature_rule.argtypes = [P, P]
        L.orc_quadrature_rule.restype = None
        L.orc_sample_features.argtypes = [C.c_uint32, C.c_float, C.c_uint64, C.c_uint64, P]
        L.orc_sample_features.restype = C.c_uint32
        L.orc_sketch_summary.argtypes = [P, C.c_uint64, P, C.c_uint32, P, C.c_uint64]
        L.orc_sketch_summary.restype = C.c_uint64
        L.orc_compress_clamps.argtypes = []
        L.orc_compress_clamps.restype = C.c_uint64
        L.orc_softmax_pairs.argtypes = [P, P, P, C.c_uint64, C.c_uint32, C.c_uint32, P]
        L.orc_softmax_pairs.restype = None
        L.orc_validated_weights.argtypes = [P, C.c_uint32]
        L.orc_validated_weights.restype = C.c_int
        L.orc_sample_features_weighted.argtypes = [C.c_uint32, C.c_float, C.c_uint64,
                                                   C.c_uint64, P, P]
        L.orc_sample_features_weighted.restype = C.c_uint32
        L.orc_nested_set.argtypes = [P, C.c_uint32, C.c_float, C.c_float, C.c_uint64,
                                     C.c_uint64, C.c_uint32, C.c_uint64, P, P]
        L.orc_nested_set.restype = C.c_uint32
        L.orc_subset_key.argtypes = [C.c_uint64] * 4
        L.orc_subset_key.restype = C.c_uint64
        L.orc_sigmoid.argtypes = [P, C.c_uint64, P]
        L.orc_sigmoid.restype = None
        L.orc_sigmoid_checksum.argtypes = [C.c_uint64, C.c_uint64, C.c_uint32]
        L.orc_sigmoid_checksum.restype = C.c_uint64
        L.orc_tanh_checksum.argtypes = [C.c_uint64, C.c_uint64, C.c_uint32]
        L.orc_tanh_checksum.restype = C.c_uint64
        L.orc_splitmix64.argtypes = [C.c_uint64, C.c_uint64, P]
        L.orc_splitmix64.restype = None
        L.orc_mix64.argtypes = [C.c_uint64]
        L.orc_mix64.restype = C.c_uint64
        L.orc_row_hash.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64]
        L.orc_row_hash.restype = C.c_uint64
        L.orc_threshold_for.argtypes = [C.c_float]
        L.orc_threshold_for.restype = C.c_uint64
        L.orc_row_selected.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64]
        L.orc_row_selected.restype = C.c_int
        L.orc_gradients.argtypes = [P, P, P, C.c_uint64, C.c_uint32, P]
        L.orc_gradients.restype = None
        L.orc_base_margin.argtypes = [C.c_uint32, C.c_float]
        L.orc_base_margin.restype = C.c_float
        L.orc_estimate_base_score.argtypes = [P, P, C.c_uint64]
        L.orc_estimate_base_score.restype = C.c_float
        L.orc_quantile_scale.argtypes = [P, P, P, C.c_uint64]
        L.orc_quantile_scale.restype = C.c_float
        L.orc_quantile_pairs.argtypes = [P, P, P, C.c_uint64, C.c_float, C.c_float, P]
        L.orc_quantile_pairs.restype = None
        L.orc_quantile_intercepts.argtypes = [P, P, C.c_uint64, P, C.c_uint32, P]
        L.orc_quantile_intercepts.restype = None
        L.orc_last_error.restype = C.c_char_p
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def make_params(**kw) -> Params:
    """Params from XGBoost-style keyword names (defaults follow
    python/ferrisboost/__init__.py:_DEFAULTS)."""
    p = Params()
    p.n_rounds = kw.get("n_rounds", 10)
    p.max_depth = kw.get("max_depth", 6)
    p.max_leaves = kw.get("max_leaves", 0)
    p.max_bin = kw.get("max_bin", 255)
    p.learning_rate = kw.get("eta", 0.3)
    p.lambda_ = kw.get("lambda", 1.0)
    p.gamma = kw.get("gamma", 0.0)
    p.min_child_weight = kw.get("min_child_weight", 1.0)
    p.alpha = kw.get("alpha", 0.0)
    p.max_delta_step = kw.get("max_delta_step", 0.0)
    p.scale_pos_weight = kw.get("scale_pos_weight", 1.0)
    p.subsample = kw.get("subsample", 1.0)
    p.colsample_bytree = kw.get("colsample_bytree", 1.0)
    p.cols_per_block = kw.get("cols_per_block", 64)
    p.seed = kw.get("seed", 0)
    p.objective = OBJECTIVES[kw.get("objective", "binary:logistic")]
    p.grow_policy = GROW[kw.get("grow_policy", "depthwise")]
    p.max_cat_to_onehot = kw.get("max_cat_to_onehot", 4)
    p.max_cat_threshold = kw.get("max_cat_threshold", 64)
    if kw.get("base_score") is not None:
        p.base_score = kw["base_score"]
        p.has_base_score = 1
    p.nthread = kw.get("nthread", 1)
    p.num_class = kw.get("num_class", 0)
    qa = kw.get("quantile_alpha")
    if qa is not None:
        arr = np.ascontiguousarray(np.atleast_1d(np.asarray(qa, np.float32)))
        p._alphas = arr  # keeps the array alive with the struct
        p.n_quantile_alpha = arr.size
        p.quantile_alpha = arr.ctypes.data_as(C.POINTER(C.c_float))
    # base_margin: class-major starting margins ([outputs][n] flattened)
    bm = kw.get("base_margin")
    if bm is not None:
        arr = np.ascontiguousarray(np.asarray(bm, np.float32).ravel())
        p._base_margin = arr
        p.base_margin = arr.ctypes.data_as(C.POINTER(C.c_float))
    p.colsample_bylevel = kw.get("colsample_bylevel", 1.0)
    p.colsample_bynode = kw.get("colsample_bynode", 1.0)
    fw = kw.get("feature_weights")
    if fw is not None:
        arr = np.ascontiguousarray(np.asarray(fw, np.float32).ravel())
        p._feature_weights = arr
        p.feature_weights = arr.ctypes.data_as(C.POINTER(C.c_float))
    return p


class Model:
    def __init__(self, handle):
        self.h = handle

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_model_free(self.h)
            self.h = None

    @property
    def n_trees(self) -> int:
        return lib().orc_model_n_trees(self.h)

    def tree(self, t: int) -> np.ndarray:
        n = lib().orc_model_tree_len(self.h, t)
        out = np.zeros(n, NODE_DTYPE)
        lib().orc_model_tree_nodes(self.h, t, _p(out))
        return out

    def trees(self):
        return [self.tree(t) for t in range(self.n_trees)]

    def cat_words(self) -> np.ndarray:
        n = lib().orc_model_n_cat_words(self.h)
        out = np.zeros(n, np.uint32)
        if n:
            lib().orc_model_cat_words(self.h, _p(out))
        return out

    @property
    def num_outputs(self) -> int:
        return lib().orc_model_num_outputs(self.h)

    def class_margins(self) -> np.ndarray:
        out = np.zeros(self.num_outputs, np.float32)
        if self.num_outputs > 1:
            lib().orc_model_class_margins(self.h, _p(out))
        return out

    @property
    def base_score(self) -> float:
        return lib().orc_model_base_score(self.h)

    @property
    def base_margin(self) -> float:
        return lib().orc_model_base_margin(self.h)

    @property
    def train_seconds(self) -> float:
        return lib().orc_model_train_seconds(self.h)

    def predict_margin(self, x: np.ndarray) -> np.ndarray:
        """Margins, [n] (or [n, K] for a multiclass model)."""
        x = np.ascontiguousarray(x, np.float32)
        k = self.num_outputs
        out = np.zeros((x.shape[0], k) if k > 1 else x.shape[0], np.float32)
        lib().orc_predict_margin(self.h, _p(x), x.shape[0], x.shape[1], _p(out))
        return out

    def train_margins(self, n: int) -> np.ndarray:
        """Training margins, [n] (or class-major [K, n] for a multiclass model)."""
        k = self.num_outputs
        out = np.zeros((k, n) if k > 1 else n, np.float32)
        lib().orc_model_train_margins(self.h, _p(out))
        return out

    def shap(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros((x.shape[0], x.shape[1] + 1), np.float32)
        rc = lib().orc_shap(self.h, _p(x), x.shape[0], x.shape[1], _p(out))
        if rc:
            raise RuntimeError(lib().orc_last_error().decode())
        return out

    _EXPLAIN = {"contribs": 0, "approx": 1, "interactions": 2, "leaf": 3}

    def explain(self, x: np.ndarray, kind: str, margin=None) -> np.ndarray:
        """Explainer::compute_with_margin: kind contribs / approx / interactions / leaf."""
        x = np.ascontiguousarray(x, np.float32)
        n, nf = x.shape
        shape = {"contribs": (n, nf + 1), "approx": (n, nf + 1),
                 "interactions": (n, nf + 1, nf + 1), "leaf": (n, self.n_trees)}[kind]
        out = np.zeros(shape, np.float32)
        m = None if margin is None else np.ascontiguousarray(margin, np.float32)
        rc = lib().orc_explain(self.h, self._EXPLAIN[kind], _p(x), n, nf, _p(m), _p(out))
        if rc:
            raise RuntimeError(lib().orc_last_error().decode())
        return out


def train(x, y, params: Params, weights=None, categorical=None, monotone=None) -> Model:
    x = np.ascontiguousarray(x, np.float32)
    y = np.ascontiguousarray(y, np.float32)
    w = None if weights is None else np.ascontiguousarray(weights, np.float32)
    cat = None if categorical is None else np.ascontiguousarray(categorical, np.uint8)
    mono = None if monotone is None else np.ascontiguousarray(monotone, np.int8)
    h = C.c_void_p()
    rc = lib().orc_train(_p(x), x.shape[0], x.shape[1], _p(y), _p(w), _p(cat), _p(mono),
                         0 if mono is None else len(mono), C.byref(params), C.byref(h))
    if rc:
        raise RuntimeError(lib().orc_last_error().decode())
    return Model(h)


def model_from_nodes(trees, cat_words, objective: str, base_score: float) -> Model:
    """An oracle model holding the given node records (NODE_DTYPE arrays)."""
    nodes = np.ascontiguousarray(np.concatenate(trees)).astype(NODE_DTYPE)
    offs = np.concatenate([[0], np.cumsum([t.size for t in trees])]).astype(np.uint32)
    words = np.ascontiguousarray(cat_words, np.uint32)
    h = C.c_void_p()
    rc = lib().orc_model_from_nodes(_p(nodes), _p(offs), len(trees), _p(words), words.size,
                                    OBJECTIVES[objective], base_score, C.byref(h))
    if rc:
        raise RuntimeError(lib().orc_last_error().decode())
    return Model(h)


def quantile_scale(pred, labels, weights=None) -> float:
    pred = np.ascontiguousarray(pred, np.float32)
    y = np.ascontiguousarray(labels, np.float32)
    w = None if weights is None else np.ascontiguousarray(weights, np.float32)
    return float(lib().orc_quantile_scale(_p(pred), _p(y), _p(w), y.size))


def quantile_pairs(pred, labels, alpha, scale, weights=None) -> np.ndarray:
    """[n, 2] weighted pairs of one quantile under a given scale."""
    pred = np.ascontiguousarray(pred, np.float32)
    y = np.ascontiguousarray(labels, np.float32)
    w = None if weights is None else np.ascontiguousarray(weights, np.float32)
    out = np.empty((y.size, 2), np.float32)
    lib().orc_quantile_pairs(_p(pred), _p(y), _p(w), y.size, alpha, scale, _p(out))
    return out


def quantile_intercepts(labels, alphas, weights=None) -> np.ndarray:
    y = np.ascontiguousarray(labels, np.float32)
    w = None if weights is None else np.ascontiguousarray(weights, np.float32)
    a = np.ascontiguousarray(np.atleast_1d(alphas), np.float32)
    out = np.empty(a.size, np.float32)
    lib().orc_quantile_intercepts(_p(y), _p(w), y.size, _p(a), a.size, _p(out))
    return out


def sketch_cuts(x, max_bin, weights=None, categorical=None):
    x = np.ascontiguousarray(x, np.float32)
    n, nf = x.shape
    # numeric features emit < max_bin cuts; categorical ones one per code
    cap = sum(65534 if (categorical is not None and categorical[f]) else max(max_bin, 2)
              for f in range(nf))
    vals = np.zeros(cap + 1, np.float32)
    offs = np.zeros(nf + 1, np.uint32)
    w = None if weights is None else np.ascontiguousarray(weights, np.float32)
    cat = None if categorical is None else np.ascontiguousarray(categorical, np.uint8)
    rc = lib().orc_sketch_cuts(_p(x), n, nf, max_bin, _p(w), _p(cat), _p(vals), _p(offs))
    if rc:
        raise RuntimeError(lib().orc_last_error().decode())
    return vals[: offs[-1]].copy(), offs


def quantizer_scales(max_grad, max_hess, n_rows):
    out = np.zeros(2, np.float64)
    rc = lib().orc_quantizer_from_bounds(max_grad, max_hess, n_rows, _p(out))
    if rc:
        raise RuntimeError(lib().orc_last_error().decode())
    return out


def quantize(gpair2n: np.ndarray, scales: np.ndarray):
    gpair2n = np.ascontiguousarray(gpair2n, np.float32)
    n = gpair2n.size // 2
    out = np.zeros(2 * n, np.int64)
    s = np.zeros(2, np.int64)
    lib().orc_quantize(_p(gpair2n), n, _p(np.ascontiguousarray(scales, np.float64)), _p(out), _p(s))
    return out, s


def hist_build(bins, offsets, gpair_fixed, rows=None):
    """bins: column-major [n_feats, n_rows] uint8/uint16."""
    bins = np.ascontiguousarray(bins)
    width = bins.dtype.itemsize
    nf, n = bins.shape
    offsets = np.ascontiguousarray(offsets, np.uint32)
    out = np.zeros(2 * int(offsets[-1]), np.int64)
    r = None if rows is None else np.ascontiguousarray(rows, np.uint32)
    lib().orc_hist_build(_p(bins), width, n, nf, _p(offsets),
                         _p(np.ascontiguousarray(gpair_fixed, np.int64)), _p(r),
                         0 if r is None else r.size, _p(out))
    return out


def best_split(hist, feat_ids, offsets, node_sum, scales, params, sampled=None, given_weight=True,
               bounds=(-3.4028234663852886e38, 3.4028234663852886e38), monotone=None,
               categorical=None) -> Split:
    out = Split()
    feat_ids = np.ascontiguousarray(feat_ids, np.uint32)
    offsets = np.ascontiguousarray(offsets, np.uint32)
    smp = None if sampled is None else np.ascontiguousarray(sampled, np.uint32)
    mono = None if monotone is None else np.ascontiguousarray(monotone, np.int8)
    cat = None if categorical is None else np.ascontiguousarray(categorical, np.uint8)
    lib().orc_best_split(
        _p(np.ascontiguousarray(hist, np.int64)), feat_ids.size, _p(feat_ids), _p(offsets),
        _p(np.ascontiguousarray(node_sum, np.int64)), _p(np.ascontiguousarray(scales, np.float64)),
        C.byref(params), _p(smp), 0 if smp is None else smp.size, 1 if given_weight else 0,
        bounds[0], bounds[1], _p(mono), 0 if mono is None else mono.size, _p(cat),
        0 if cat is None else cat.size, C.byref(out))
    return out


def partition(rows, col, split_bin, missing_left, cats=None):
    rows = np.ascontiguousarray(rows, np.uint32)
    col = np.ascontiguousarray(col)
    out = np.zeros_like(rows)
    c = None if cats is None else np.ascontiguousarray(cats, np.uint64)
    nl = lib().orc_partition(_p(rows), rows.size, _p(col), col.dtype.itemsize, split_bin,
                             1 if missing_left else 0, _p(c), 0 if c is None else c.size, _p(out))
    return out, int(nl)


def quadrature_rule():
    n = np.zeros(8, np.float32)
    w = np.zeros(8, np.float32)
    lib().orc_quadrature_rule(_p(n), _p(w))
    return n, w


def sample_features(n_features, rate, seed, round_):
    out = np.zeros(max(n_features, 1), np.uint32)
    k = lib().orc_sample_features(n_features, rate, seed, round_, _p(out))
    return out[:k].copy()


def _f32_or_none(w):
    return None if w is None else np.ascontiguousarray(w, np.float32)


def validated_weights(weights, n_features) -> int:
    """0 = uniform sampling, 1 = weighted; invalid weights raise ValueError."""
    w = _f32_or_none(weights)
    rc = lib().orc_validated_weights(_p(w), n_features)
    if rc < 0:
        raise ValueError(lib().orc_last_error().decode())
    return rc


def sample_features_weighted(n_features, rate, seed, round_, weights=None):
    w = _f32_or_none(weights)
    out = np.zeros(max(n_features, 1), np.uint32)
    k = lib().orc_sample_features_weighted(n_features, rate, seed, round_, _p(w), _p(out))
    return out[:k].copy()


def nested_set(base, bylevel, bynode, seed, tree, tag, idx, weights=None):
    """NestedSampler level_set (tag 1, idx = depth) / node_set (tag 2, idx = node)."""
    b = np.ascontiguousarray(base, np.uint32)
    w = _f32_or_none(weights)
    out = np.zeros(max(b.size, 1), np.uint32)
    k = lib().orc_nested_set(_p(b), b.size, bylevel, bynode, seed, tree, tag, idx, _p(w), _p(out))
    return out[:k].copy()


def subset_key(seed, tree, tag, idx) -> int:
    return int(lib().orc_subset_key(seed, tree, tag, idx))


def sketch_summary(col, max_bin, weights=None):
    """The collapsed sketch summary of one numeric column: a structured array
    of (value, weight, rmin, rmax)."""
    c = np.ascontiguousarray(col, np.float32)
    w = _f32_or_none(weights)
    cap = 16 * max(max_bin, 2) + 64
    out = np.zeros((cap, 4), np.float32)
    k = lib().orc_sketch_summary(_p(c), c.size, _p(w), max_bin, _p(out), cap)
    if k > cap:
        out = np.zeros((k, 4), np.float32)
        lib().orc_sketch_summary(_p(c), c.size, _p(w), max_bin, _p(out), k)
    out = out[:k]
    rec = np.zeros(k, [("value", np.float32), ("weight", np.float32), ("rmin", np.float32),
                       ("rmax", np.float32)])
    for i, f in enumerate(rec.dtype.names):
        rec[f] = out[:, i]
    return rec


def compress_clamps() -> int:
    return int(lib().orc_compress_clamps())


def softmax_pairs(margins_kn, labels, weights, k):
    """Softmax pairs of class k, [n][2] f32, from class-major margins [K][n]."""
    m = np.ascontiguousarray(margins_kn, np.float32)
    y = np.ascontiguousarray(labels, np.float32)
    w = _f32_or_none(weights)
    out = np.zeros(2 * y.size, np.float32)
    lib().orc_softmax_pairs(_p(m), _p(y), _p(w), y.size, m.shape[0], k, _p(out))
    return out
