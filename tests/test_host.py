"""CPU tests of the boundary and the host logic (no GPU needed).

* both C-ABI libraries load and export every function include/*.h declares;
* the Python package mirrors the reference's parameter surface and error
  classes (python/ferrisboost/__init__.py, src/error.rs:1-68): bad input is a
  ValueError before any device work, and with no device every training call
  is a RuntimeError -- the package has no CPU fallback;
* the product's quantile sketch (the setup step that feeds both engines)
  produces the oracle's cuts bit for bit;
* bench.py refuses more than one GPU;
* the histograms' shift quantizer of f32 pairs equals the gradient pass's
  double formula.
"""

from __future__ import annotations

import ctypes as C
import os
import re
import subprocess
import sys

import numpy as np
import pytest

from conftest import ROOT, gpu_ready

HEADERS = [os.path.join(ROOT, "include", h) for h in ("fbhip.h", "fbtrain.h")]


def _declared(path: str, prefix: str) -> list[str]:
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(" + prefix + r"_\w+)\s*\(", text)))


def test_headers_declare_the_boundary():
    hip = _declared(HEADERS[0], "fbh")
    train = _declared(HEADERS[1], "fbt")
    assert {"fbh_ctx_create", "fbh_eval_nodes", "fbh_partition", "fbh_build_histogram",
            "fbh_shap_contribs", "fbh_last_error"} <= set(hip)
    assert {"fbt_train", "fbt_shap", "fbt_model_to_json"} <= set(train)


def test_integration_ffi_block_matches_the_header():
    """INTEGRATION.md's Rust FFI block declares every function of
    include/fbhip.h with the same parameter and return types, in order, and
    every #[repr(C)] struct with the header's fields (names and types)."""
    import ffi_check as F

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    hdr = open(os.path.join(root, "include", "fbhip.h")).read()
    block = F.rust_block(open(os.path.join(root, "INTEGRATION.md")).read())
    hf, rf = F.header_functions(hdr), F.rust_functions(block)
    assert set(hf) == set(rf), (sorted(set(hf) - set(rf)), sorted(set(rf) - set(hf)))
    for name, (ret, args) in hf.items():
        rret, rargs = rf[name]
        assert (rret if rret != "()" else "c_void") == ret, name
        assert [t for _, t in rargs] == [t for _, t in args], name
    hs, rs = F.header_structs(hdr), F.rust_structs(block)
    assert len(hs) >= 10
    for name, fields in hs.items():
        assert rs.get(name) == fields, name


def test_libraries_export_every_declared_symbol():
    from ferrisboost_amd import _native as N

    L = N.hip()
    T = N.train_lib()
    for name in _declared(HEADERS[0], "fbh"):
        assert hasattr(L, name), f"libfbhip.so does not export {name}"
    for name in _declared(HEADERS[1], "fbt"):
        assert hasattr(T, name), f"libfbtrain.so does not export {name}"
    # the Python binding knows every symbol, too
    assert set(_declared(HEADERS[0], "fbh")) == set(N.HIP_SYMBOLS)
    assert set(_declared(HEADERS[1], "fbt")) == set(N.TRAIN_SYMBOLS)


def test_libraries_are_gfx950_code_objects():
    """The HIP library carries a gfx950 code object (and no other target)."""
    from ferrisboost_amd import _native as N

    data = open(N.LIB_HIP, "rb").read()
    assert b"gfx950" in data
    assert b"sm_" + b"80" not in data


def test_oracle_is_not_linked_by_the_product():
    """The shipped libraries and package never reference the oracle."""
    from ferrisboost_amd import _native as N

    for lib in (N.LIB_HIP, N.LIB_TRAIN):
        out = subprocess.run(["ldd", lib], capture_output=True, text=True).stdout
        assert "oracle" not in out
        assert b"orc_" not in open(lib, "rb").read()
    pkg = os.path.join(ROOT, "ferrisboost_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".h")):
                src = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in src.lower(), f


def test_error_classes_map_to_python():
    from ferrisboost_amd import _native as N

    assert issubclass(N.InputError, ValueError)
    assert issubclass(N.BackendError, RuntimeError)


def _tiny():
    rng = np.random.default_rng(0)
    x = rng.normal(size=(64, 3)).astype(np.float32)
    y = (x[:, 0] > 0).astype(np.float32)
    return x, y


@pytest.mark.parametrize("params, msg", [
    ({"device": "cpu"}, "device"),
    ({"device": "tpu"}, "device"),
    ({"objective": "reg:pseudohubererror"}, "objective"),
    ({"objective": "reg:quantileerror"}, "needs quantile_alpha"),
    ({"objective": "reg:quantileerror", "quantile_alpha": 1.5}, r"must be in \[0, 1\]"),
    ({"objective": "reg:quantileerror", "quantile_alpha": [0.9, 0.1]}, "ascending"),
    ({"objective": "reg:quantileerror", "quantile_alpha": []}, "must not be an empty list"),
    ({"objective": "reg:quantileerror", "quantile_alpha": [0.5] * 65}, "at most 64"),
    ({"objective": "multi:softprob"}, "num_class >= 2"),
    ({"objective": "multi:softmax", "num_class": 1}, "num_class >= 2"),
    ({"objective": "multi:softprob", "num_class": 2.5}, "num_class must be an integer"),
    ({"objective": "multi:softprob", "num_class": -3}, "num_class must not be negative"),
    ({"grow_policy": "levelwise"}, "grow_policy"),
    ({"max_bin": 0}, "max_bin"),
    ({"max_bin": 70000}, "max_bin"),
    ({"gpu_math": "sloppy"}, "gpu_math"),
    ({"hist_streams": 3}, "hist_streams"),
    ({"resident_blocks": -1}, "resident_blocks"),
    ({"hist_nodes_per_batch": 40}, "hist_nodes_per_batch"),
    ({"hist_nodes_per_batch": 8}, "hist_nodes_per_batch is not available"),
    ({"device_quantize": False}, "device_quantize"),
    ({"colsample_bylevel": 0.0}, r"colsample_bylevel must be in \(0, 1\]"),
    ({"colsample_bynode": 1.5}, r"colsample_bynode must be in \(0, 1\]"),
    ({"colsample_bynode": float("nan")}, "colsample_bynode"),
    ({"feature_weights": [1.0, -1.0, 1.0]}, "nonnegative"),
    ({"feature_weights": [0.0, 0.0, 0.0]}, "at least one positive"),
    ({"feature_weights": [1.0, 2.0]}, "has 2 entries, expected 3"),
    ({"feature_weights": "abc"}, "must be a mapping"),
    ({"feature_weights": np.ones((2, 2))}, "one-dimensional"),
    ({"feature_weights": [True, 1.0, 1.0]}, "boolean"),
    ({"feature_weights": {"f0": 1.0}}, "needs data with feature names"),
    ({"tree_method": "exact"}, "tree_method"),
    ({"no_such_param": 1}, "unknown parameter"),
    ({"interaction_constraints": [[0, 1]]}, "interaction"),
])
def test_bad_params_are_value_errors(params, msg):
    import ferrisboost_amd as fb

    x, y = _tiny()
    with pytest.raises(ValueError, match=msg):
        fb.train(params, x, label=y, num_boost_round=2)


def test_train_takes_the_reference_argument_order():
    """python/ferrisboost/__init__.py:1090-1114: train(params, data, label,
    num_boost_round, evals, ...); what this path leaves out is refused by
    name before any device work."""
    import ferrisboost_amd as fb

    x, y = _tiny()
    with pytest.raises(ValueError, match="num_boost_round must be >= 1"):
        fb.train({}, x, y, 0)  # the fourth positional argument is num_boost_round
    with pytest.raises(ValueError, match="num_boost_round must be an integer"):
        fb.train({}, x, y, np.ones(x.shape[0], np.float32))
    with pytest.raises(ValueError, match="validation sets"):
        fb.train({}, x, y, 2, [(x, y, "valid")])
    for kw, what in (({"early_stopping_rounds": 3}, "early stopping"),
                     ({"init_model": "m.json"}, "continuation"),
                     ({"xgb_model": "m.json"}, "continuation"),
                     ({"qid": np.zeros(x.shape[0])}, "ranking"),
                     ({"label_lower_bound": y}, "survival")):
        with pytest.raises(ValueError, match=what):
            fb.train({}, x, y, 2, **kw)
    with pytest.raises(ValueError, match="label is required"):
        fb.train({}, x)
    results = {"stale": 1}
    with pytest.raises((RuntimeError, ValueError)):
        fb.train({"max_depth": 15}, x, y, 2, evals_result=results)
    assert results == {}


@pytest.mark.parametrize("params, margin, msg", [
    ({}, np.zeros(7, np.float32), "base_margin has 7 values, expected"),
    ({}, np.zeros((64, 2), np.float32), r"must have shape \(n,\) or \(n, 1\)"),
    ({"objective": "multi:softprob", "num_class": 3}, np.zeros(64, np.float32),
     r"must have shape \(n, 3\)"),
    ({}, np.full(64, np.inf, np.float32), "finite"),
])
def test_base_margin_shapes_are_checked(params, margin, msg):
    import ferrisboost_amd as fb

    x, y = _tiny()
    y = np.floor(y * 2.999).astype(np.float32) if params else y
    with pytest.raises(ValueError, match=msg):
        fb.train(params, x, y, 2, base_margin=margin)


def test_bad_shapes_are_value_errors():
    import ferrisboost_amd as fb

    x, y = _tiny()
    with pytest.raises(ValueError):
        fb.train({}, x, label=y[:10], num_boost_round=2)
    with pytest.raises(ValueError):
        fb.train({}, x[:, 0], label=y, num_boost_round=2)
    with pytest.raises(ValueError):
        fb.train({}, x, label=y, weight=np.ones(3, np.float32), num_boost_round=2)
    with pytest.raises(ValueError):
        fb.train({}, x, label=y, num_boost_round=0)


@pytest.mark.parametrize("params, msg", [
    ({"max_depth": 15}, "max_depth"),
    ({"eta": -1.0}, "learning_rate"),
    ({"subsample": 0.0}, "subsample"),
    ({"colsample_bytree": 1.5}, "colsample_bytree"),
    ({"gpu_math": "fast", "hip_host_sigmoid": True}, "gpu_math"),
])
def test_driver_validation_is_input_error(params, msg):
    """The C++ driver validates before any device call (src/types.rs:432-660,
    src/training/mod.rs:1487-1493): FBH_INPUT_ERROR -> ValueError."""
    import ferrisboost_amd as fb

    x, y = _tiny()
    with pytest.raises(ValueError, match=msg):
        fb.train(params, x, label=y, num_boost_round=2)


@pytest.mark.skipif(gpu_ready(), reason="checks the no-device error path")
def test_no_device_is_a_runtime_error_not_a_fallback():
    import ferrisboost_amd as fb

    x, y = _tiny()
    assert not fb.device_available(0)
    with pytest.raises(RuntimeError):
        fb.train({"max_depth": 3}, x, label=y, num_boost_round=2)


def _product_cuts(x, max_bin, weights=None, categorical=None):
    from ferrisboost_amd import _native as N

    x = np.ascontiguousarray(x, np.float32)
    n, nf = x.shape
    cap = sum(65534 if (categorical is not None and categorical[f]) else max(max_bin, 2)
              for f in range(nf))
    vals = np.zeros(cap + 1, np.float32)
    offs = np.zeros(nf + 1, np.uint32)
    w = None if weights is None else np.ascontiguousarray(weights, np.float32)
    cat = None if categorical is None else np.ascontiguousarray(categorical, np.uint8)
    N.check_train(N.train_lib().fbt_sketch_cuts(N.ptr(x), n, nf, max_bin, N.ptr(w), N.ptr(cat),
                                                N.ptr(vals), N.ptr(offs)))
    return vals[: offs[-1]].copy(), offs


@pytest.mark.parametrize("max_bin", [16, 255, 256, 1024])
def test_product_sketch_equals_oracle(oracle, max_bin):
    rng = np.random.default_rng(max_bin)
    n = 60_000
    x = np.stack([
        rng.normal(size=n),
        np.abs(rng.normal(size=n)),
        np.exp(rng.normal(size=n)),
        rng.integers(0, 7, size=n),
        rng.uniform(size=n),
        np.full(n, 3.0),
        rng.integers(0, 300, size=n),
    ], 1).astype(np.float32)
    x[rng.random(x.shape) < 0.07] = np.nan
    w = rng.uniform(0.5, 2.0, size=n).astype(np.float32)
    cat = np.array([0, 0, 0, 0, 0, 0, 1], np.uint8)
    for weights in (None, w):
        a = _product_cuts(x, max_bin, weights, cat)
        b = oracle.sketch_cuts(x, max_bin, weights, cat)
        assert np.array_equal(a[1], b[1])
        assert np.array_equal(a[0].view(np.uint32), b[0].view(np.uint32))


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)


def test_host_sigmoid_restatement_equals_libm(oracle):
    """The restated expf (glibc's table-driven method) gives the host libm's
    logistic sigmoid bit for bit: every 251st float bit pattern (17.1M
    inputs, all exponents) plus a dense sweep of the margins training meets.
    The device compile of the same code is checked on all 2^32 inputs by the
    GPU suite."""
    from ferrisboost_amd import _native as N

    u = np.arange(0, 2**32, 251, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([u.view(np.float32),
                        np.arange(-105.0, 105.0, 2.0**-10, dtype=np.float64).astype(np.float32)])
    got = np.empty_like(x)
    want = np.empty_like(x)
    N.check_hip(N.hip().fbh_sigmoid_host(N.ptr(x), x.size, N.ptr(got)))
    oracle.lib().orc_sigmoid(oracle._p(x), x.size, oracle._p(want))
    gb, wb = got.view(np.uint32).copy(), want.view(np.uint32).copy()
    gb[np.isnan(got)] = 0x7FC00000
    wb[np.isnan(want)] = 0x7FC00000
    bad = np.nonzero(gb != wb)[0]
    assert bad.size == 0, [(hex(int(x.view(np.uint32)[i])), got[i], want[i]) for i in bad[:5]]
    # denormal outputs are produced and kept
    assert np.any((want > 0) & (want < np.finfo(np.float32).tiny))


# ---------------------------------------------------------------- memory plan

def _plan(n_rows, n_features, n_bins=256, width=1, budget=0, free=0, slots=128,
          categorical=None, windows=0, resident_limit=0):
    from ferrisboost_amd import _native as N

    w = np.full(n_features, width, np.uint8)
    nb = np.full(n_features, n_bins - 1 if width == 1 and n_bins > 255 else n_bins, np.uint32)
    cat = None if categorical is None else np.ascontiguousarray(categorical, np.uint8)
    shape = N.Shape(n_features, N.ptr(w), N.ptr(nb), N.ptr(cat))
    cfg = N.Config()
    cfg.memory_budget = budget
    cfg.hist_slots = slots
    cfg.stream_windows = windows
    cfg.resident_limit = resident_limit
    out = N.Plan()
    N.check_hip(N.hip().fbh_plan_memory(n_rows, C.byref(shape), C.byref(cfg), free, C.byref(out)))
    return out


def test_plan_everything_resident_when_it_fits():
    """288 GB of HBM: the narrow and wide configs are fully resident."""
    for n, f in ((10_500_000, 28), (400_000, 2000)):
        p = _plan(n, f, free=280 << 30)
        assert p.resident_tiles == p.n_tiles and p.columns_resident == 1
        assert p.staging_bytes == 0 and p.streamed_record_bytes == 0
        assert p.peak_bytes == p.fixed_bytes + p.resident_record_bytes + p.column_bytes
        assert p.peak_bytes <= p.budget
        # the record tiles and the columns each hold every cell once (u8)
        assert p.column_bytes == n * f and p.resident_record_bytes >= n * f


def test_plan_streams_under_a_forced_budget():
    """50M x 200 u8 under 4 GiB: columns leave HBM, the windows are reserved,
    some tiles stay resident and the rest stream; the plan fits the budget."""
    p = _plan(50_000_000, 200, budget=4 << 30)
    assert p.budget == 4 << 30 and p.peak_bytes <= p.budget
    assert p.columns_resident == 0 and p.column_bytes == 0
    assert 0 < p.resident_tiles < p.n_tiles
    assert p.staging_bytes > 0 and p.window_rows >= 65536
    assert p.streamed_record_bytes > 0


def test_plan_residency_grows_with_the_budget():
    prev = -1
    for gib in (3, 4, 6, 8, 12, 16, 24):
        p = _plan(50_000_000, 200, budget=gib << 30)
        assert p.peak_bytes <= p.budget
        assert p.resident_tiles >= prev
        prev = p.resident_tiles
    assert prev == _plan(50_000_000, 200, budget=24 << 30).n_tiles


def test_plan_resident_blocks_caps_resident_tiles():
    """resident_blocks (python/ferrisboost/__init__.py:233-239): at most that
    many tiles stay resident even when all would fit; 0 is pure streaming."""
    full = _plan(2_000_000, 120, free=280 << 30)
    assert full.resident_tiles == full.n_tiles >= 4
    for k in (0, 1, 3):
        p = _plan(2_000_000, 120, free=280 << 30, resident_limit=k + 1)
        assert p.resident_tiles == k and p.columns_resident == 0
        assert p.staging_bytes > 0 and p.streamed_record_bytes > 0
    big = _plan(2_000_000, 120, free=280 << 30, resident_limit=full.n_tiles + 5)
    assert big.resident_tiles == big.n_tiles and big.columns_resident == 1


def test_plan_hist_streams_sets_the_streaming_windows():
    """hist_streams 1 keeps one window of each kind instead of two: half the
    staging bytes (src/python/mod.rs:224-231 validates 1 or 2)."""
    two = _plan(50_000_000, 200, budget=6 << 30)
    one = _plan(50_000_000, 200, budget=6 << 30, windows=1)
    assert two.staging_bytes == 2 * one.staging_bytes
    assert one.window_rows == two.window_rows and one.peak_bytes <= one.budget
    with pytest.raises(ValueError, match="stream_windows"):
        _plan(50_000_000, 200, budget=6 << 30, windows=3)


def test_plan_rejects_a_budget_below_the_per_row_arrays():
    """Planning failure is an error, never a silent fallback
    (src/training/gpu_mem_plan.rs:764-800)."""
    with pytest.raises(ValueError, match="gpu_memory_budget"):
        _plan(50_000_000, 200, budget=1 << 30)


def test_plan_default_reserve():
    """Without a budget: free memory minus max(15 %, 512 MiB)
    (default_safety_reserve, src/training/gpu_mem_plan.rs:957-959)."""
    p = _plan(100_000, 28, free=100 << 30)
    assert p.budget == (100 << 30) - (100 << 30) // 100 * 15
    p = _plan(100_000, 28, free=2 << 30)
    assert p.budget == (2 << 30) - (512 << 20)


_QUANT_CHECK = r"""
#include "fbhip_quant.h"
#include <cmath>
#include <cstdio>
#include <cstring>
// The gradient pass's formula: round half away from zero of v * 2^l in
// double, saturated to int64, NaN to 0.
static int64_t by_double(float v, int l) {
    double x = std::round(std::ldexp((double)v, l));
    if (std::isnan(x)) return 0;
    if (x >= 9223372036854775808.0) return INT64_MAX;
    if (x < -9223372036854775808.0) return INT64_MIN;
    return (int64_t)x;
}
int main() {
    const int ls[] = {0, 1, 14, 23, 24, 38, 39, 40, 41, 62, 63, 64, 212, 1000,
                      -1, -24, -25, -149, -1000};
    long bad = 0, n = 0;
    for (int l : ls) {
        if (fbh::pow2_exponent(std::ldexp(1.0, l)) != l) bad++;
        // every 251st bit pattern, plus the neighbourhood of every power of two
        for (uint64_t u = 0; u <= 0xFFFFFFFFull; u += 251) {
            for (uint32_t d = 0; d < 2; d++) {
                uint32_t b = (uint32_t)u ^ (d ? 0x80000000u : 0u);
                float v;
                memcpy(&v, &b, 4);
                n++;
                if (fbh::quantize_pow2(v, l) != by_double(v, l)) bad++;
            }
        }
        for (uint32_t e = 0; e < 256; e++)
            for (int k = -3; k <= 3; k++)
                for (uint32_t sgn = 0; sgn < 2; sgn++) {
                    uint32_t b = ((e << 23) + (uint32_t)k) ^ (sgn << 31);
                    float v;
                    memcpy(&v, &b, 4);
                    n++;
                    if (fbh::quantize_pow2(v, l) != by_double(v, l)) bad++;
                }
    }
    printf("%ld %ld\n", n, bad);
    return bad != 0;
}
"""


def test_shift_quantizer_equals_the_double_formula(tmp_path):
    """The histograms' integer quantisation of f32 pairs (fbhip_quant.h) gives
    sat_i64(round((double)v * 2^l)), the gradient pass's value
    (GradQuantizer::to_fixed, src/types.rs:367-385), for the scales 2^l the
    quantizer makes: sampled bit patterns of both signs and every exponent's
    neighbourhood (zeros, subnormals, infinities, NaNs, the 2^63 saturation
    edge) at shifts from -1000 to 1000. Built from the product header with
    the host compiler."""
    src = tmp_path / "quant_check.cpp"
    src.write_text(_QUANT_CHECK)
    exe = tmp_path / "quant_check"
    inc = os.path.join(ROOT, "ferrisboost_amd", "csrc")
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", inc, str(src), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    n, bad = map(int, r.stdout.split())
    assert n > 600_000_000 // 2 and bad == 0, r.stdout
