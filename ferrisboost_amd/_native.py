"""ctypes bindings of libfbhip.so (include/fbhip.h) and libfbtrain.so
(include/fbtrain.h). Loading never compiles: build with
`python -m ferrisboost_amd.build` first. A missing library is an error, never
a silent fallback."""

from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_HIP = os.path.join(HERE, "libfbhip.so")
LIB_TRAIN = os.path.join(HERE, "libfbtrain.so")

P = C.c_void_p


class Span(C.Structure):
    _fields_ = [("offset", C.c_uint32), ("len", C.c_uint32)]


class Shape(C.Structure):
    _fields_ = [("n_features", C.c_uint32), ("width", P), ("n_bins", P), ("categorical", P)]


class Plan(C.Structure):
    """fbh_plan: the memory plan of a context."""

    _fields_ = [
        ("budget", C.c_uint64),
        ("fixed_bytes", C.c_uint64),
        ("resident_record_bytes", C.c_uint64),
        ("column_bytes", C.c_uint64),
        ("staging_bytes", C.c_uint64),
        ("peak_bytes", C.c_uint64),
        ("streamed_record_bytes", C.c_uint64),
        ("n_tiles", C.c_uint32),
        ("resident_tiles", C.c_uint32),
        ("columns_resident", C.c_uint32),
        ("window_rows", C.c_uint32),
    ]


class Config(C.Structure):
    _fields_ = [
        ("memory_budget", C.c_uint64),
        ("hist_slots", C.c_uint32),
        ("tile_bytes", C.c_uint32),
        ("rows_per_block", C.c_uint32),
        ("max_cat_words", C.c_uint32),
        ("stream_windows", C.c_uint32),
        ("resident_limit", C.c_uint32),
        ("n_outputs", C.c_uint32),
        ("reserved", C.c_uint32 * 3),
    ]


class SplitParams(C.Structure):
    _fields_ = [
        ("lambda_", C.c_float),
        ("gamma", C.c_float),
        ("min_child_weight", C.c_float),
        ("alpha", C.c_float),
        ("max_delta_step", C.c_float),
        ("max_cat_to_onehot", C.c_uint32),
        ("max_cat_threshold", C.c_uint32),
        ("reserved", C.c_uint32),
    ]


class NodeReq(C.Structure):
    _fields_ = [
        ("rows", Span),
        ("sum", C.c_int64 * 2),
        ("lower", C.c_float),
        ("upper", C.c_float),
        ("slot", C.c_uint32),
        ("subtract_parent", C.c_int32),
        ("subtract_sibling", C.c_int32),
        ("reserved", C.c_uint32),
    ]


class SplitOut(C.Structure):
    _fields_ = [
        ("found", C.c_uint32),
        ("feat", C.c_uint32),
        ("bin", C.c_uint32),
        ("missing_left", C.c_uint32),
        ("gain", C.c_float),
        ("is_cat", C.c_uint32),
        ("cat_offset", C.c_uint32),
        ("n_cat_words", C.c_uint32),
        ("left", C.c_int64 * 2),
        ("right", C.c_int64 * 2),
    ]


class PartReq(C.Structure):
    _fields_ = [
        ("rows", Span),
        ("feat", C.c_uint32),
        ("bin", C.c_uint32),
        ("missing_left", C.c_uint32),
        ("cat_offset", C.c_uint32),
        ("n_cat_words", C.c_uint32),
        ("reserved", C.c_uint32),
    ]


class ChildPair(C.Structure):
    _fields_ = [
        ("parent_slot", C.c_uint32),
        ("new_slot", C.c_uint32),
        ("evaluate", C.c_uint32),
        ("reserved", C.c_uint32),
        ("lower", C.c_float * 2),
        ("upper", C.c_float * 2),
        ("left_sum", C.c_int64 * 2),
        ("right_sum", C.c_int64 * 2),
    ]


class TrainParams(C.Structure):
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
        ("device", C.c_int32),
        ("gpu_math", C.c_uint32),
        ("gpu_memory_budget", C.c_uint64),
        ("tile_bytes", C.c_uint32),
        ("rows_per_block", C.c_uint32),
        ("profile", C.c_uint32),
        ("host_sigmoid", C.c_uint32),
        ("host_levels", C.c_uint32),
        ("sync_round", C.c_uint32),
        ("hist_streams", C.c_uint32),
        ("resident_limit", C.c_uint32),
        ("host_binning", C.c_uint32),
        ("host_sketch", C.c_uint32),
        ("n_quantile_alpha", C.c_uint32),
        ("quantile_alpha", C.POINTER(C.c_float)),
        ("base_margin", C.POINTER(C.c_float)),
        ("colsample_bylevel", C.c_float),
        ("colsample_bynode", C.c_float),
        ("feature_weights", C.POINTER(C.c_float)),
    ]


# fbt_rows_fn: int (*)(void *user, uint64_t begin, uint64_t n, float *out)
ROWS_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_uint64, C.c_uint64, C.POINTER(C.c_float))


class Stats(C.Structure):
    _fields_ = [
        ("train_seconds", C.c_double),
        ("setup_seconds", C.c_double),
        ("hist_kernel_ms", C.c_double),
        ("hist_launches", C.c_uint64),
        ("hist_bytes", C.c_uint64),
        ("host_gradient_seconds", C.c_double),
        ("device_bytes", C.c_double),
        ("rounds", C.c_uint32),
        ("device_sigmoid", C.c_uint32),
        ("n_tiles", C.c_uint32),
        ("resident_tiles", C.c_uint32),
        ("streamed_bytes", C.c_uint64),
        ("planned_bytes", C.c_uint64),
        ("budget_bytes", C.c_uint64),
        ("device_trees", C.c_uint32),
        ("device_binning", C.c_uint32),
        ("sketch_seconds", C.c_double),
        ("bin_seconds", C.c_double),
        ("device_sketch", C.c_uint32),
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

# Every symbol the headers declare, per library.
HIP_SYMBOLS = [
    "fbh_last_error", "fbh_device_available", "fbh_ctx_create", "fbh_ctx_destroy",
    "fbh_plan_memory", "fbh_ctx_plan", "fbh_ctx_streamed_bytes",
    "fbh_ctx_device_bytes", "fbh_upload_block", "fbh_set_cuts", "fbh_rows_staging_bytes",
    "fbh_apply_leaf_values",
    "fbh_upload_rows", "fbh_finish_rows", "fbh_sketch_device_bytes", "fbh_sketch_fits",
    "fbh_sketch_create", "fbh_sketch_push_rows", "fbh_sketch_cuts", "fbh_sketch_missing",
    "fbh_sketch_destroy",
    "fbh_upload_quantize_gpair",
    "fbh_upload_gpair_fixed", "fbh_set_objective", "fbh_set_multiclass",
    "fbh_multiclass_begin_round", "fbh_set_output", "fbh_set_quantile",
    "fbh_quantile_last_scale", "fbh_tanh_checksum", "fbh_gradient_exchange",
    "fbh_download_margin", "fbh_set_margins", "fbh_set_gpu_math", "fbh_gradient_pairs", "fbh_sigmoid_host", "fbh_sigmoid_device", "fbh_sigmoid_checksum",
    "fbh_begin_tree", "fbh_eval_nodes", "fbh_download_histogram",
    "fbh_partition", "fbh_partition_eval", "fbh_partition_eval_masked", "fbh_grow_depthwise", "fbh_grow_depthwise_async",
    "fbh_grow_collect", "fbh_assign_leaves", "fbh_download_delta", "fbh_host_alloc",
    "fbh_host_free", "fbh_download_rows",
    "fbh_hist_timing", "fbh_set_timing", "fbh_build_histogram", "fbh_partition_rows",
    "fbh_shap_model_create", "fbh_shap_model_destroy", "fbh_shap_contribs",
    "fbh_shap_contribs_device", "fbh_shap_last_ms", "fbh_shap_interactions",
    "fbh_saabas_contribs", "fbh_predict", "fbh_predict_device", "fbh_shap_contribs_noalloc",
]
TRAIN_SYMBOLS = [
    "fbt_last_error", "fbt_train", "fbt_train_cuts", "fbt_train_rows", "fbt_last_stats",
    "fbt_last_round_stats", "fbt_last_round_launches", "fbt_model_free", "fbt_model_n_trees",
    "fbt_model_tree_len", "fbt_model_tree_nodes", "fbt_model_n_cat_words", "fbt_model_cat_words",
    "fbt_model_base_score", "fbt_model_base_margin", "fbt_model_n_features",
    "fbt_model_train_margins", "fbt_model_n_cuts", "fbt_model_cuts", "fbt_predict_margin",
    "fbt_model_to_json", "fbt_shap", "fbt_last_shap_ms", "fbt_sketch_cuts", "fbt_predict",
    "fbt_model_from_json", "fbt_model_objective", "fbt_model_scale_pos_weight",
    "fbt_model_num_outputs", "fbt_model_class_margins", "fbt_model_quantile_alpha",
    "fbt_model_is_categorical",
]

_hip = None
_train = None


class InputError(ValueError):
    """The backend's input-error class (FBH_INPUT_ERROR)."""


class BackendError(RuntimeError):
    """The backend's runtime-error class (FBH_RUNTIME_ERROR)."""


def _require(path: str) -> None:
    if not os.path.exists(path):
        raise BackendError(
            f"{os.path.basename(path)} is not built; run `python -m ferrisboost_amd.build` "
            "(the device path has no CPU fallback)"
        )


def hip() -> C.CDLL:
    global _hip
    if _hip is None:
        _require(LIB_HIP)
        L = C.CDLL(LIB_HIP)
        L.fbh_last_error.argtypes = [C.c_char_p, C.c_size_t]
        L.fbh_last_error.restype = C.c_size_t
        L.fbh_device_available.argtypes = [C.c_int]
        L.fbh_ctx_create.argtypes = [C.c_int, C.c_uint64, C.POINTER(Shape), C.POINTER(Config),
                                     C.POINTER(P)]
        L.fbh_ctx_destroy.argtypes = [P]
        L.fbh_plan_memory.argtypes = [C.c_uint64, C.POINTER(Shape), C.POINTER(Config), C.c_uint64,
                                      C.POINTER(Plan)]
        L.fbh_ctx_plan.argtypes = [P, C.POINTER(Plan)]
        L.fbh_ctx_streamed_bytes.argtypes = [P]
        L.fbh_ctx_streamed_bytes.restype = C.c_uint64
        L.fbh_ctx_device_bytes.argtypes = [P]
        L.fbh_ctx_device_bytes.restype = C.c_uint64
        L.fbh_upload_block.argtypes = [P, P, C.c_uint32, C.c_uint32, P]
        L.fbh_set_cuts.argtypes = [P, P, P, P]
        L.fbh_rows_staging_bytes.argtypes = [P]
        L.fbh_rows_staging_bytes.restype = C.c_uint64
        L.fbh_upload_rows.argtypes = [P, P, C.c_uint64, C.c_uint64]
        L.fbh_finish_rows.argtypes = [P]
        L.fbh_sketch_device_bytes.argtypes = [C.c_uint64, C.c_uint32, C.c_uint32, P]
        L.fbh_sketch_device_bytes.restype = C.c_uint64
        L.fbh_sketch_fits.argtypes = [C.c_int, C.c_uint64, C.c_uint32, C.c_uint32, P, C.c_uint64]
        L.fbh_sketch_create.argtypes = [C.c_int, C.c_uint64, C.c_uint32, C.c_uint32, P,
                                        C.c_uint64, C.POINTER(P)]
        L.fbh_sketch_push_rows.argtypes = [P, P, C.c_uint64]
        L.fbh_sketch_cuts.argtypes = [P, P, C.c_uint64, P, P]
        L.fbh_sketch_missing.argtypes = [P, P]
        L.fbh_sketch_destroy.argtypes = [P]
        L.fbh_apply_leaf_values.argtypes = [P, P, C.c_uint32]
        L.fbh_upload_quantize_gpair.argtypes = [P, P, C.c_uint64, C.c_uint64, C.c_uint64, P, P]
        L.fbh_upload_gpair_fixed.argtypes = [P, P, P]
        L.fbh_set_objective.argtypes = [P, C.c_uint32, P, P, C.c_float]
        L.fbh_set_multiclass.argtypes = [P, C.c_uint32, P, P, P]
        L.fbh_multiclass_begin_round.argtypes = [P]
        L.fbh_set_output.argtypes = [P, C.c_uint32]
        L.fbh_set_quantile.argtypes = [P, C.c_uint32, P, P, P, P]
        L.fbh_quantile_last_scale.argtypes = [P, P]
        L.fbh_tanh_checksum.argtypes = [C.c_int, C.c_uint64, C.c_uint64, P]
        L.fbh_gradient_exchange.argtypes = [P, P, P, C.c_uint64, C.c_uint64, C.c_uint64, P, P]
        L.fbh_download_margin.argtypes = [P, P]
        L.fbh_set_margins.argtypes = [P, P]
        L.fbh_set_gpu_math.argtypes = [P, C.c_uint32]
        L.fbh_gradient_pairs.argtypes = [C.c_int, C.c_uint32, C.c_uint32, P, P, P, C.c_uint64, P]
        L.fbh_sigmoid_host.argtypes = [P, C.c_uint64, P]
        L.fbh_sigmoid_device.argtypes = [C.c_int, P, C.c_uint64, P]
        L.fbh_sigmoid_checksum.argtypes = [C.c_int, C.c_uint64, C.c_uint64, P]
        L.fbh_begin_tree.argtypes = [P, P, C.c_uint32, P, C.c_uint32, C.POINTER(Span)]
        L.fbh_eval_nodes.argtypes = [P, P, C.c_uint32, C.POINTER(SplitParams), P, P, P,
                                     C.c_uint32]
        L.fbh_download_histogram.argtypes = [P, C.c_uint32, P, C.POINTER(C.c_uint64)]
        L.fbh_partition.argtypes = [P, P, C.c_uint32, P, C.c_uint32, P]
        L.fbh_partition_eval.argtypes = [P, P, C.c_uint32, P, C.c_uint32, P, P, P, P, P, P,
                                         C.c_uint32]
        L.fbh_partition_eval_masked.argtypes = [P, P, C.c_uint32, P, C.c_uint32, P, P, P, P, P,
                                                P, P, C.c_uint32]
        L.fbh_assign_leaves.argtypes = [P, P, P, C.c_uint32]
        L.fbh_download_delta.argtypes = [P, P]
        L.fbh_download_rows.argtypes = [P, P]
        L.fbh_hist_timing.argtypes = [P, C.POINTER(C.c_double), C.POINTER(C.c_uint64),
                                      C.POINTER(C.c_uint64), C.c_int]
        L.fbh_set_timing.argtypes = [P, C.c_int]
        L.fbh_build_histogram.argtypes = [C.c_int, P, C.c_uint32, C.c_uint64, C.c_uint32, P, P, P,
                                          C.c_uint64, P]
        L.fbh_partition_rows.argtypes = [C.c_int, P, C.c_uint32, C.c_uint64, P, C.c_uint64,
                                         C.c_uint32, C.c_uint32, P, C.c_uint32, P,
                                         C.POINTER(C.c_uint64)]
        L.fbh_shap_model_create.argtypes = [C.c_int, C.c_uint32, P, P, P, P, P, P, P, P, P, P, P,
                                            P, C.c_uint32, C.c_uint32, C.c_float, C.POINTER(P)]
        L.fbh_shap_model_destroy.argtypes = [P]
        L.fbh_shap_contribs.argtypes = [P, P, C.c_uint64, P, P]
        L.fbh_shap_contribs_device.argtypes = [P, P, C.c_uint64, P, P, C.c_int]
        L.fbh_shap_last_ms.argtypes = [P]
        L.fbh_shap_last_ms.restype = C.c_double
        for name in ("fbh_shap_interactions", "fbh_saabas_contribs", "fbh_shap_contribs_noalloc"):
            getattr(L, name).argtypes = [P, P, C.c_uint64, P, P]
        L.fbh_predict.argtypes = [P, P, C.c_uint64, P, C.c_uint32, P]
        L.fbh_predict_device.argtypes = [P, P, C.c_uint64, P, C.c_uint32, P, C.c_int]
        _hip = L
    return _hip


def train_lib() -> C.CDLL:
    global _train
    if _train is None:
        hip()
        _require(LIB_TRAIN)
        L = C.CDLL(LIB_TRAIN)
        L.fbt_last_error.argtypes = [C.c_char_p, C.c_size_t]
        L.fbt_last_error.restype = C.c_size_t
        L.fbt_train.argtypes = [P, C.c_uint64, C.c_uint32, P, P, P, P, C.c_uint32,
                                C.POINTER(TrainParams), C.POINTER(P)]
        L.fbt_train_cuts.argtypes = [P, C.c_uint64, C.c_uint32, P, P, P, P, C.c_uint32,
                                     C.POINTER(TrainParams), P, P, C.POINTER(P)]
        L.fbt_train_rows.argtypes = [ROWS_FN, P, C.c_uint64, C.c_uint32, P, P, P, P, C.c_uint32,
                                     C.POINTER(TrainParams), C.POINTER(P)]
        L.fbt_last_stats.argtypes = [C.POINTER(Stats)]
        L.fbt_last_round_stats.argtypes = [P, P, P, C.c_uint32]
        L.fbt_last_round_stats.restype = C.c_uint32
        L.fbt_last_round_launches.argtypes = [P, C.c_uint32]
        L.fbt_last_round_launches.restype = C.c_uint32
        L.fbt_model_free.argtypes = [P]
        L.fbt_model_free.restype = None
        for name in ("fbt_model_n_trees", "fbt_model_n_cat_words", "fbt_model_n_features",
                     "fbt_model_n_cuts"):
            getattr(L, name).argtypes = [P]
            getattr(L, name).restype = C.c_uint32
        L.fbt_model_tree_len.argtypes = [P, C.c_uint32]
        L.fbt_model_tree_len.restype = C.c_uint32
        L.fbt_model_tree_nodes.argtypes = [P, C.c_uint32, P]
        L.fbt_model_tree_nodes.restype = None
        L.fbt_model_cat_words.argtypes = [P, P]
        L.fbt_model_cat_words.restype = None
        L.fbt_model_base_score.argtypes = [P]
        L.fbt_model_base_score.restype = C.c_float
        L.fbt_model_base_margin.argtypes = [P]
        L.fbt_model_base_margin.restype = C.c_float
        L.fbt_model_train_margins.argtypes = [P, P, C.c_uint64]
        L.fbt_model_cuts.argtypes = [P, P, P]
        L.fbt_model_cuts.restype = None
        L.fbt_predict_margin.argtypes = [P, P, C.c_uint64, C.c_uint32, P]
        L.fbt_predict_margin.restype = None
        L.fbt_model_to_json.argtypes = [P, C.c_char_p, C.c_size_t]
        L.fbt_model_to_json.restype = C.c_size_t
        L.fbt_shap.argtypes = [P, P, C.c_uint64, C.c_uint32, C.c_int, P]
        L.fbt_sketch_cuts.argtypes = [P, C.c_uint64, C.c_uint32, C.c_uint32, P, P, P, P]
        L.fbt_last_shap_ms.argtypes = []
        L.fbt_last_shap_ms.restype = C.c_double
        L.fbt_predict.argtypes = [P, P, C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32,
                                  C.c_uint32, P, C.c_int, P]
        L.fbt_model_from_json.argtypes = [C.c_char_p, C.c_size_t, C.POINTER(P)]
        L.fbt_model_objective.argtypes = [P]
        L.fbt_model_objective.restype = C.c_uint32
        L.fbt_model_num_outputs.argtypes = [P]
        L.fbt_model_num_outputs.restype = C.c_uint32
        L.fbt_model_class_margins.argtypes = [P, P]
        L.fbt_model_class_margins.restype = None
        L.fbt_model_quantile_alpha.argtypes = [P, P, C.c_uint32]
        L.fbt_model_quantile_alpha.restype = C.c_uint32
        L.fbt_model_scale_pos_weight.argtypes = [P]
        L.fbt_model_scale_pos_weight.restype = C.c_float
        L.fbt_model_is_categorical.argtypes = [P, C.c_uint32]
        L.fbt_model_is_categorical.restype = C.c_uint32
        _train = L
    return _train


# fbt_predict outputs (include/fbtrain.h).
OUT_MARGIN, OUT_VALUE, OUT_LEAF, OUT_CONTRIBS, OUT_APPROX, OUT_INTERACTIONS = range(6)


def ptr(a):
    return None if a is None else a.ctypes.data_as(P)


def check_hip(rc: int) -> None:
    if rc == 0:
        return
    buf = C.create_string_buffer(4096)
    hip().fbh_last_error(buf, len(buf))
    msg = buf.value.decode(errors="replace")
    raise (InputError if rc == 1 else BackendError)(msg)


def check_train(rc: int) -> None:
    if rc == 0:
        return
    buf = C.create_string_buffer(4096)
    train_lib().fbt_last_error(buf, len(buf))
    msg = buf.value.decode(errors="replace")
    raise (InputError if rc == 1 else BackendError)(msg)


def device_available(device: int = 0) -> bool:
    return bool(hip().fbh_device_available(device))
