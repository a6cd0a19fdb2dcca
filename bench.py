#!/usr/bin/env python3
"""Benchmark of the device training path on one MI355X.

Default workload (the headline): 10.5M x 28 HIGGS-like binary classification,
max_bin=255 (u8 bins), depth 8, eta 0.1, gpu_math="exact" (byte-identical
trees). One step = one boosting round with everything resident in HBM; W
warmup rounds, then K timed rounds; the round timer runs between blocking
device syncs. Other workloads (--workload):

  wide      400k x 2000 L2-normalised rows, colsample_bytree 0.5, depth 8
  widebin   2M x (80 numeric with 10% NaN + 20 categorical x 500 codes),
            max_bin 1024 (u16), reg:squarederror, lossguide, 255 leaves
  streaming 50M x 200 N(0,1) binary, max_bin 256 (8-bit cells: no missing
            value; about 10 GB of bins),
            depth 8, with the device budget forced to 4 GiB: most tiles
            stream from pinned host memory
  multiclass  the narrow rows with 4 classes, multi:softprob (4 trees a round)
  quantile  the narrow rows with a continuous target, reg:quantileerror at
            quantile_alpha 0.1 / 0.5 / 0.9 (3 trees a round)
  shap      GPU TreeSHAP of 1M rows x 200 features against a 100-tree,
            depth-8 ensemble (trained first, untimed); one step = one pass
  predict   GPU margins of the same rows and ensemble; one step = one pass

Prints one JSON line:
  value         boosting rounds per second (shap: rows per second)
  roofline      the dominant kernel: histogram algorithmic bytes (cells +
                16 B gradient pair + 4 B row id per accumulated row, + 32 B
                per written histogram bin; the pair counts 16 B also where the
                kernel reads 8 B of f32 and quantizes it) over their HIP-event
                time, against 8 TB/s HBM; traffic: HBM bytes per launch in the
                same rounds, from the committed rocprofv3 counter summary
                (`--traffic-summary` writes it from the counter runs)
  cpu_baseline  the CPU oracle (C++ restatement of the reference CPU engine)
                on a bounded sample of the same workload, threads stated
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
# VALU issue peak: 256 CUs x 64 lanes x 2.4 GHz, one fp32 operation a lane a cycle (the
# kernels are built without FMA contraction and without packed fp32).
VALU_PEAK_TOPS = 39.3
# TreeSHAP of the 100-tree depth-8 ensemble: VALU lane-operations a row, counted by
# SQ_INSTS_VALU x 64 / rows for shap_rec_kernel on the shap workload.
SHAP_VALU_OPS_PER_ROW = 11.23e6
# Prediction of the same ensemble: VALU lane-operations a row (SQ_INSTS_VALU x 64 / rows
# for predict_lds4_kernel on the predict workload).
PREDICT_VALU_OPS_PER_ROW = 11934
# MI355X fp32 vector peak (FMA counted as two operations).
FP32_PEAK_TFLOPS = 157.3
# QuadratureTreeSHAP's arithmetic (8 quadrature points): for each child edge of an
# internal node the extend (3 operations a point) and the unwind of that edge's
# contribution (5 a point), plus the sum of the two subtrees' returns (1 a point); for a
# leaf the scaled return (2 a point, and the path weight). The unwinds of a feature met
# twice on a path are data-dependent and not counted: a lower bound.
SHAP_QP = 8
SHAP_FLOPS_INTERNAL = 2 * (3 + 5) * SHAP_QP + SHAP_QP
SHAP_FLOPS_LEAF = 2 * SHAP_QP + 1


def shap_flops_per_row(model) -> int:
    """Algorithmic floating-point operations of one row's TreeSHAP over the
    model (the same for every row: every row visits every node)."""
    total = 0
    for t in model.trees():
        leaves = int((t["is_leaf"] == 1).sum())
        total += SHAP_FLOPS_INTERNAL * (t.size - leaves) + SHAP_FLOPS_LEAF * leaves
    return total


def node_visits_per_row(model, X) -> float:
    """Nodes a prediction walk visits per row (root to leaf, every tree),
    averaged over the first 100k rows from their leaf ids."""
    leaf = model.predict(X[:100_000], pred_leaf=True).astype(np.int64)
    visits = 0.0
    for k, t in enumerate(model.trees()):
        depth = np.zeros(t.size, np.int64)
        for i in range(t.size):  # parents come before children in node-id order
            if t["is_leaf"][i] != 1:
                depth[t["left"][i]] = depth[i] + 1
                depth[t["right"][i]] = depth[i] + 1
        visits += float((depth[leaf[:, k]] + 1).mean())
    return visits
METRIC = "histogram build GB/s (% HBM peak) + boosting rounds/sec, 10.5M×28 u8 bins depth 8"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def load_traffic(path: str):
    """A committed counter summary of the histogram kernel: `key = value`
    lines, and one `round R LAUNCHES FETCH_KIB WRITE_KIB` line per round of
    the profiled job's first training run (FETCH_SIZE and WRITE_SIZE summed
    over that round's histogram dispatches)."""
    meta, rounds = {}, {}
    try:
        with open(path) as f:
            for line in f:
                s = line.strip()
                if not s or s.startswith("#"):
                    continue
                if s.startswith("round "):
                    _, r, n, fk, wk = s.split()
                    rounds[int(r)] = (int(n), float(fk), float(wk))
                elif "=" in s:
                    k, v = s.split("=", 1)
                    meta[k.strip()] = v.strip()
    except OSError:
        return None, None
    return meta, rounds


def window_traffic(path: str, workload: str, lo: int, hi: int):
    """HBM bytes per histogram launch over rounds [lo, hi) of `workload`, from
    the committed summary (None and the reason where it does not cover them:
    another workload, or rounds it did not profile)."""
    meta, rounds = load_traffic(path)
    if meta is None:
        return None, f"no counter summary {os.path.relpath(path, ROOT)}"
    if meta.get("workload") != workload:
        return None, f"{os.path.relpath(path, ROOT)} profiles another workload"
    if any(r not in rounds for r in range(lo, hi)):
        return None, f"{os.path.relpath(path, ROOT)} does not cover rounds {lo}..{hi - 1}"
    ff, wf = float(meta["fetch_factor"]), float(meta["write_factor"])
    n = sum(rounds[r][0] for r in range(lo, hi))
    fetch = sum(rounds[r][1] for r in range(lo, hi)) * 1024.0 * ff
    write = sum(rounds[r][2] for r in range(lo, hi)) * 1024.0 * wf
    if n == 0:
        return None, f"no histogram launch in rounds {lo}..{hi - 1}"
    return {"bytes": (fetch + write) / n, "fetch": fetch / n, "write": write / n,
            "launches": n}, None


def copy_probe(mib: int) -> int:
    """Run a plain device copy of known size (the calibration kernel of the
    FETCH_SIZE / WRITE_SIZE counters)."""
    import torch

    n = mib << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": n, "launches": 3}), flush=True)
    return 0


def cpu_threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), for the baseline's record."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def base_line(args, value, unit, ms_per_step, config, dtype="int64"):
    return {
        "metric": METRIC,
        "value": value,
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic",
        "config": config,
    }


def train_workload(args, X, y, params, desc: str, traffic_tag: str):
    import ferrisboost_amd as fb
    from ferrisboost_amd import _native as N

    rounds = args.warmup + args.steps
    timed = slice(args.warmup, rounds)

    def run(profile: bool):
        # The round loop collects each tree a round late; hip_sync_round makes
        # it wait for the device before the first timed round, so the timed
        # rounds are bracketed by device synchronisation on both sides.
        gparams = dict(params, device="cuda:0", hip_profile=profile, hip_sync_round=args.warmup)
        t0 = time.time()
        model = fb.train(gparams, X, y, num_boost_round=rounds)
        log(f"trained {rounds} rounds in {time.time() - t0:.1f}s "
            f"(profile {profile}, setup {model.stats['setup_seconds']:.1f}s, device sigmoid "
            f"{model.stats['device_sigmoid']})")
        wall = np.zeros(rounds)
        hms = np.zeros(rounds)
        hbytes = np.zeros(rounds, np.uint64)
        hlaunch = np.zeros(rounds, np.uint64)
        n = N.train_lib().fbt_last_round_stats(N.ptr(wall), N.ptr(hms), N.ptr(hbytes), rounds)
        assert n == rounds
        assert N.train_lib().fbt_last_round_launches(N.ptr(hlaunch), rounds) == rounds
        return model, wall, hms, hbytes, hlaunch

    # The throughput comes from a run without event timing; the histogram
    # kernels are timed (HIP events on their dispatches) in a second run.
    model, wall, _, _, _ = run(False)
    t_wall = float(wall[timed].sum())
    pmodel, _, hms, hbytes, hlaunch = run(True)
    # Both runs grow the same trees (the device path is deterministic).
    same_runs = all(np.array_equal(model.tree_nodes(t), pmodel.tree_nodes(t))
                    for t in range(rounds))
    t_hist_ms = float(hms[timed].sum())
    b_hist = float(hbytes[timed].astype(np.float64).sum())
    hist_gbps = b_hist / (t_hist_ms * 1e-3) / 1e9 if t_hist_ms > 0 else 0.0
    launches = int(hlaunch[timed].sum())
    bytes_per_launch = b_hist / launches if launches else 0.0
    roofline = {
        "bound": "hbm",
        "achieved": round(hist_gbps, 1),
        "peak": HBM_PEAK_GBPS,
        "unit": "GB/s",
        "frac": round(hist_gbps / HBM_PEAK_GBPS, 4),
        "traffic": None,
        "algorithmic_bytes_per_launch": round(bytes_per_launch),
    }
    # HBM traffic of the same rounds' histogram launches (the trees are the
    # same in every run of this workload), from the committed counter summary.
    if traffic_tag:
        tr, why = window_traffic(os.path.join(ROOT, "profiles", f"hist_traffic_{traffic_tag}.txt"),
                                 desc, args.warmup, rounds)
        if tr and tr["launches"] != launches:
            tr, why = None, (f"the summary counts {tr['launches']} launches in rounds "
                             f"{args.warmup}..{rounds - 1}, this run {launches}")
        if tr:
            roofline["traffic"] = round(tr["bytes"])
            roofline["traffic_rounds"] = [args.warmup, rounds - 1]
            roofline["traffic_over_algorithmic"] = round(tr["bytes"] / bytes_per_launch, 3)
        else:
            roofline["traffic_note"] = why

    cpu = None
    parity = None
    if not args.no_cpu:
        from oracle import oracle as O

        threads = cpu_threads()
        cols = max(1, -(-X.shape[1] // threads))
        op = {k: v for k, v in params.items() if k not in ("device", "feature_types", "gpu_math")}
        op.update(n_rounds=args.cpu_rounds, cols_per_block=cols, nthread=threads)
        cat = None
        if "feature_types" in params:
            cat = np.array([1 if t == "c" else 0 for t in params["feature_types"]], np.uint8)
        t0 = time.time()
        om = O.train(X, y, O.make_params(**op), categorical=cat)
        cpu_s = om.train_seconds
        log(f"cpu oracle {args.cpu_rounds} rounds: {cpu_s:.1f}s train, {time.time() - t0:.1f}s total")
        blocks = -(-X.shape[1] // cols)
        cpu = {
            "value": round(args.cpu_rounds / cpu_s, 4),
            "unit": "rounds/s",
            "cores": min(threads, blocks),
            "kind": "port",
            "sample": f"first {args.cpu_rounds} rounds of the same {X.shape[0]}x{X.shape[1]} "
                      f"workload (histograms threaded over {blocks} column blocks; "
                      "gradient, split and partition single-threaded, so this understates "
                      "a fully threaded CPU engine)",
            "cpu_model": cpu_model(),
            "host_cpus": os.cpu_count(),
        }
        # gpu_math="fast" is deterministic but not byte-equal to the CPU
        # engine (the device exponential), so no tree comparison is made.
        if params.get("gpu_math") != "fast":
            parity = all(
                np.array_equal(om.tree(t)[f], model.tree_nodes(t)[f])
                for t in range(om.n_trees) for f in om.tree(t).dtype.names if f != "pad")

    config = {"workload": desc, "rows": int(X.shape[0]), "features": int(X.shape[1]),
              "rounds": rounds}
    config.update({k: params[k] for k in ("max_bin", "max_depth", "max_leaves", "grow_policy",
                                          "colsample_bytree", "objective", "num_class",
                                          "quantile_alpha", "gpu_math")
                   if k in params})
    out = base_line(args, round(args.steps / t_wall, 3), "rounds/s",
                    round(1e3 * t_wall / args.steps, 3), config)
    out.update({
        "hist_gbps": round(hist_gbps, 1),
        "hist_ms_per_round": round(t_hist_ms / args.steps, 3),
        "hist_launches_per_round": round(launches / args.steps, 2),
        # the whole job: setup (sketch and binning) plus every round, warmup included
        "job_seconds": round(model.stats["setup_seconds"] + float(wall.sum()), 3),
        "gradient_ms_per_round": round(1e3 * model.stats["host_gradient_seconds"] / rounds, 3),
        # setup (outside the timed rounds): the quantile sketch, then binning
        # (each on the device when it fits, the host's cuts and bins either way)
        "setup": {"seconds": round(model.stats["setup_seconds"], 3),
                  "sketch_seconds": round(model.stats["sketch_seconds"], 3),
                  "binning_seconds": round(model.stats["bin_seconds"], 3),
                  "device_sketch": bool(model.stats["device_sketch"]),
                  "device_binning": bool(model.stats["device_binning"])},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "parity_first_rounds_vs_cpu": parity,
        "repeat_runs_identical": same_runs,
    })
    return out


def streaming_workload(args):
    import ferrisboost_amd as fb
    from ferrisboost_amd import _native as N
    from ferrisboost_amd import datasets

    n_rows = args.rows or 50_000_000
    t0 = time.time()
    X, y, params, _ = datasets.streaming(n_rows=n_rows, n_features=200)
    # The configured max_bin 256 (no missing value: 8-bit cells), or 255
    max_bin = args.max_bin or params["max_bin"]
    params = dict(params, max_bin=max_bin)
    log(f"data {X.shape} generated in {time.time() - t0:.1f}s")
    budget = 4 << 30
    rounds = args.warmup + args.steps
    t0 = time.time()
    model = fb.train(dict(params, device="cuda:0", gpu_memory_budget=budget, hip_profile=True,
                          hip_sync_round=args.warmup),
                     X, y, num_boost_round=rounds)
    st = model.stats
    log(f"trained {rounds} rounds in {time.time() - t0:.1f}s (setup {st['setup_seconds']:.1f}s); "
        f"{st['resident_tiles']}/{st['n_tiles']} tiles resident, plan {st['planned_bytes']} "
        f"of {st['budget_bytes']} bytes")
    wall = np.zeros(rounds)
    hms = np.zeros(rounds)
    hbytes = np.zeros(rounds, np.uint64)
    N.train_lib().fbt_last_round_stats(N.ptr(wall), N.ptr(hms), N.ptr(hbytes), rounds)
    t_wall = float(wall[args.warmup:].sum())
    config = {"workload": f"streaming {n_rows}x200 N(0,1) binary, max_bin={max_bin} (8-bit "
                          "cells), depth 8, gpu_memory_budget=4 GiB", "rows": n_rows,
              "features": 200, "max_bin": max_bin, "max_depth": 8, "gpu_memory_budget": budget}
    out = base_line(args, round(args.steps / t_wall, 4), "rounds/s",
                    round(1e3 * t_wall / args.steps, 1), config)
    streamed = float(st["streamed_bytes"])
    train_s = float(st["train_seconds"])
    out.update({
        "resident_tiles": int(st["resident_tiles"]),
        "n_tiles": int(st["n_tiles"]),
        "planned_bytes": int(st["planned_bytes"]),
        "device_bytes": int(st["device_bytes"]),
        "streamed_gb_per_round": round(streamed / rounds / 1e9, 2),
        "h2d_gbps": round(streamed / train_s / 1e9, 1),
        "setup": {"seconds": round(st["setup_seconds"], 3),
                  "sketch_seconds": round(st["sketch_seconds"], 3),
                  "binning_seconds": round(st["bin_seconds"], 3),
                  "device_sketch": bool(st["device_sketch"]),
                  "device_binning": bool(st["device_binning"])},
        "roofline": {"bound": "hbm", "achieved": round(float(hbytes[args.warmup:].sum()) /
                                                         (float(hms[args.warmup:].sum()) * 1e-3) / 1e9, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": None, "traffic": None,
                     "note": "histogram time includes waiting for PCIe windows"},
        "cpu_baseline": None,
    })
    out["roofline"]["frac"] = round(out["roofline"]["achieved"] / HBM_PEAK_GBPS, 4)
    return out


def explained_model(args):
    """The 100-tree depth-8 ensemble of the streaming data's first rows (1M x
    200 by default), trained untimed, and those rows."""
    import ferrisboost_amd as fb
    from ferrisboost_amd import datasets

    n_rows = args.rows or 1_000_000
    X, y, params, _ = datasets.streaming(n_rows=n_rows, n_features=200)
    t0 = time.time()
    model = fb.train(dict(params, device="cuda:0"), X, y, num_boost_round=100)
    log(f"trained 100 trees on {X.shape} in {time.time() - t0:.1f}s")
    return model, X


def predict_workload(args):
    from ferrisboost_amd import _native as N

    model, X = explained_model(args)
    n_rows = X.shape[0]
    L = N.train_lib()
    model.predict(X[:4096], output_margin=True)  # load the kernels
    for _ in range(args.warmup):
        model.predict(X, output_margin=True)
    kernel_ms = 0.0
    t0 = time.time()
    for _ in range(args.steps):
        margin = model.predict(X, output_margin=True)
        kernel_ms += L.fbt_last_shap_ms()
    wall = time.time() - t0
    rows_per_s = args.steps * n_rows / (kernel_ms * 1e-3)
    # bytes the kernel must move: the row in, its margin out
    per_row = 4 * X.shape[1] + 4
    gbps = args.steps * n_rows * per_row / (kernel_ms * 1e-3) / 1e9
    visits = node_visits_per_row(model, X)
    cpu = None
    parity = None
    if not args.no_cpu:
        from oracle import oracle as O

        k = 20_000
        om = O.model_from_nodes(model.trees(), model.cat_words(), model.objective,
                                model.base_score)
        t0 = time.time()
        ref = om.predict_margin(X[:k])
        cpu_s = time.time() - t0
        parity = bool(np.array_equal(ref.view(np.uint32), margin[:k].view(np.uint32)))
        cpu = {"value": round(k / cpu_s, 1), "unit": "rows/s", "cores": 1, "kind": "port",
               "sample": f"margins of the first {k} rows (same trees), one thread",
               "cpu_model": cpu_model(), "host_cpus": os.cpu_count()}
    config = {"workload": f"GPU prediction (margins), {n_rows} rows x {X.shape[1]} features, "
                          "100 trees depth 8", "rows": n_rows, "features": int(X.shape[1]),
              "trees": 100, "max_depth": 8}
    out = base_line(args, round(rows_per_s, 1), "rows/s", round(kernel_ms / args.steps, 3),
                    config, dtype="f32")
    # The walk is a chain of dependent loads (node, then the row's cell, then
    # the child), so its bound is memory latency, not bandwidth or VALU
    # issue: the VALU and HBM figures beside it are far from their peaks.
    valu = rows_per_s * PREDICT_VALU_OPS_PER_ROW / 1e12
    out.update({
        "roofline": {"bound": "latency", "achieved": round(rows_per_s * visits / 1e9, 2),
                     "peak": None, "unit": "G node visits/s", "frac": None, "traffic": None,
                     "node_visits_per_row": round(visits, 1),
                     "valu_tops": round(valu, 3), "valu_frac": round(valu / VALU_PEAK_TOPS, 4),
                     "hbm_gbps": round(gbps, 1), "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4)},
        "pcie_inclusive_rows_per_s": round(args.steps * n_rows / wall, 1),
        "cpu_baseline": cpu,
        "margins_bit_identical_to_cpu": parity,
    })
    return out


def shap_workload(args):
    from ferrisboost_amd import _native as N

    model, X = explained_model(args)
    n_rows = X.shape[0]
    L = N.train_lib()
    model.predict(X[:4096], pred_contribs=True)  # load the kernels
    for _ in range(args.warmup):
        model.predict(X, pred_contribs=True)
    kernel_ms = 0.0
    t0 = time.time()
    for _ in range(args.steps):
        phi = model.predict(X, pred_contribs=True)
        kernel_ms += L.fbt_last_shap_ms()
    wall = time.time() - t0
    rows_per_s = args.steps * n_rows / (kernel_ms * 1e-3)
    # bytes the kernel must move: the row in, its contributions out
    per_row = 4 * X.shape[1] + 4 * (X.shape[1] + 1)
    gbps = args.steps * n_rows * per_row / (kernel_ms * 1e-3) / 1e9
    tops = rows_per_s * SHAP_VALU_OPS_PER_ROW / 1e12
    alg = shap_flops_per_row(model)
    margin = model.predict(X[:20000], output_margin=True)
    additivity = float(np.max(np.abs(phi[:20000].sum(axis=1) - margin)))

    cpu = None
    parity = None
    if not args.no_cpu:
        from oracle import oracle as O

        k = 2000
        om = O.model_from_nodes(model.trees(), model.cat_words(), model.objective,
                                model.base_score)
        t0 = time.time()
        ref = om.shap(X[:k])
        cpu_s = time.time() - t0
        parity = float(np.max(np.abs(ref - phi[:k])))
        cpu = {"value": round(k / cpu_s, 1), "unit": "rows/s", "cores": 1, "kind": "port",
               "sample": f"the first {k} rows of the same explanation (same trees), one thread"}
    config = {"workload": f"GPU TreeSHAP, {n_rows} rows x {X.shape[1]} features, "
                          "100 trees depth 8 (QuadratureTreeSHAP)",
              "rows": n_rows, "features": int(X.shape[1]), "trees": 100, "max_depth": 8}
    out = base_line(args, round(rows_per_s, 1), "rows/s", round(kernel_ms / args.steps, 3),
                    config, dtype="f32")
    out.update({
        "roofline": {"bound": "valu", "achieved": round(tops, 2), "peak": VALU_PEAK_TOPS,
                     "unit": "T lane-ops/s", "frac": round(tops / VALU_PEAK_TOPS, 4),
                     "traffic": None, "ops_per_row": SHAP_VALU_OPS_PER_ROW,
                     "algorithmic_flops_per_row": alg,
                     "algorithmic_tflops": round(rows_per_s * alg / 1e12, 2),
                     "algorithmic_frac_fp32_peak": round(rows_per_s * alg / 1e12 / FP32_PEAK_TFLOPS, 4),
                     "hbm_gbps": round(gbps, 2)},
        "pcie_inclusive_rows_per_s": round(args.steps * n_rows / wall, 1),
        "additivity_max_abs": additivity,
        "cpu_baseline": cpu,
        "max_abs_vs_cpu": parity,
    })
    return out


# Boosting rounds of the full training jobs the bench workloads stand for.
FULL_ROUNDS = {"narrow": 500, "wide": 200, "widebin": 300}


def workload_desc(args):
    """The training workload's description (the line's config.workload) and
    the tag of its histogram counter summary (None: no summary kept)."""
    w = args.workload
    if w == "narrow":
        rows = args.rows or 10_500_000
        cells = ("u8 bins" if args.max_bin <= 255 else
                 "256 bins a feature in 8-bit cells: no missing values" if args.max_bin == 256
                 else "u16 bins")
        return (f"narrow {rows}x28 HIGGS-like binary, max_bin={args.max_bin} ({cells}), depth 8, "
                f"eta 0.1, gpu_math={args.gpu_math}, depthwise",
                f"narrow_{args.max_bin}" if args.gpu_math == "exact" else None)
    if w in ("multiclass", "quantile"):
        rows = args.rows or 10_500_000
        what = ("4 classes, multi:softprob (4 trees a round)" if w == "multiclass" else
                "reg:quantileerror at quantile_alpha 0.1/0.5/0.9 (3 trees a round)")
        return (f"narrow {rows}x28 rows, {what}, max_bin=255 (u8 bins), depth 8, "
                f"eta 0.1, gpu_math={args.gpu_math}, depthwise", None)
    if w == "wide":
        rows = args.rows or 400_000
        return (f"wide {rows}x2000 L2-normalised binary, max_bin=256, depth 8, "
                f"colsample_bytree 0.5, gpu_math={args.gpu_math}",
                "wide" if args.gpu_math == "exact" else None)
    rows = args.rows or 2_000_000
    return (f"wide-bin {rows}x100 (80 numeric 10% NaN + 20 categorical x 500 "
            "Zipf codes), max_bin=1024 (u16), reg:squarederror, lossguide 255 leaves", "widebin")


def workload_data(args):
    from ferrisboost_amd import datasets

    w = args.workload
    if w == "narrow":
        X, y, params, _ = datasets.narrow_binary(args.rows or 10_500_000, max_bin=args.max_bin)
    elif w == "multiclass":
        X, y, params, _ = datasets.narrow_multiclass(args.rows or 10_500_000)
    elif w == "quantile":
        X, y, params, _ = datasets.narrow_quantile(args.rows or 10_500_000)
    elif w == "wide":
        X, y, params, _ = datasets.wide_binary(args.rows or 400_000, n_features=2000)
    else:
        X, y, params, _ = datasets.widebin_cat(args.rows or 2_000_000)
    return X, y, params


def _counter_rows(d: str, counter: str):
    """(dispatch id, kernel name, value) of every dispatch in a rocprofv3
    --pmc CSV under directory d, in dispatch order."""
    import csv
    import glob

    files = sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True))
    if not files:
        raise SystemExit(f"no counter_collection.csv under {d}")
    out = []
    for fn in files:
        with open(fn, newline="") as f:
            for row in csv.DictReader(f):
                if row["Counter_Name"] == counter:
                    out.append((int(row["Dispatch_Id"]), row["Kernel_Name"],
                                float(row["Counter_Value"])))
    out.sort()
    return out


def traffic_summary(args, d: str) -> int:
    """Write profiles/hist_traffic_<tag>.txt from the counter runs under d:
    <tag>_FETCH_SIZE/ and <tag>_WRITE_SIZE/ (the bench command with
    hist_kernel and gradient_kernel dispatches counted), copy_FETCH_SIZE/ and
    copy_WRITE_SIZE/ (--copy-probe 1024). The histogram dispatches of round r
    are those between the r-th and the (r+1)-th gradient dispatch of the
    first training run."""
    desc, tag = workload_desc(args)
    if tag is None:
        raise SystemExit(f"no counter summary is kept for {desc}")
    rounds = args.warmup + args.steps
    copy_bytes = 1024 << 20
    factor = {}
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        v = [x for _, k, x in _counter_rows(os.path.join(d, f"copy_{c}"), c) if "copy" in k.lower()]
        factor[c] = copy_bytes / (1024.0 * sum(v) / len(v))
    per = {}
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        rows = _counter_rows(os.path.join(d, f"{tag}_{c}"), c)
        grads = [i for i, k, _ in rows if "gradient_kernel<" in k]
        if len(grads) != 2 * rounds:
            raise SystemExit(f"{c}: {len(grads)} gradient dispatches, expected 2 x {rounds}")
        table = [[] for _ in range(rounds)]
        r = -1
        for i, k, x in rows:
            if "gradient_kernel<" in k:
                r += 1
            elif "hist_kernel" in k and 0 <= r < rounds:
                table[r].append(x)
        per[c] = table
    if [len(t) for t in per["FETCH_SIZE"]] != [len(t) for t in per["WRITE_SIZE"]]:
        raise SystemExit("the FETCH_SIZE and WRITE_SIZE runs launched different histograms")
    extra = "" if args.workload != "narrow" else (
        f" --max-bin {args.max_bin}" if args.max_bin != 255 else "")
    cmd = f"python3 bench.py --workload {args.workload}{extra} --steps {args.steps} " \
          f"--warmup {args.warmup} --no-cpu"
    ff, wf = factor["FETCH_SIZE"], factor["WRITE_SIZE"]
    lines = [
        f"# HBM traffic of the histogram kernel: {desc}, {rounds} rounds",
        "# Commands (repository root on the MI355X box; one counter a pass):",
    ]
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        lines.append(f'#   rocprofv3 --pmc {c} -f csv --kernel-include-regex "hist_kernel|gradient_kernel" '
                     f"-d gpurun_out/pmct/{tag}_{c} -o c -- {cmd}")
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        lines.append(f"#   rocprofv3 --pmc {c} -f csv -d gpurun_out/pmct/copy_{c} -o c -- "
                     "python3 bench.py --copy-probe 1024")
    lines += [
        f"#   python3 bench.py --workload {args.workload}{extra} --steps {args.steps} "
        f"--warmup {args.warmup} --traffic-summary gpurun_out/pmct",
        "# Calibration: a 1 GiB device copy reads FETCH_SIZE "
        f"{copy_bytes / 1024 / ff:.0f} KiB and WRITE_SIZE {copy_bytes / 1024 / wf:.0f} KiB a "
        "dispatch, so bytes = KiB x 1024 x factor. FETCH_SIZE counts L2 misses to the fabric,",
        "# some of which the 256 MB Infinity Cache serves, so it bounds HBM reads from above.",
        "# The bench line of a run of this workload averages the rounds it times; the rows",
        "# below are the first training run of the command (the second grows the same trees).",
        f"workload = {desc}",
        f"fetch_factor = {ff:.4f}",
        f"write_factor = {wf:.4f}",
        f"rounds = {rounds}",
    ]
    # per launch position within a round (the tree level for depthwise
    # trees), over the rounds a default bench window times and over all
    def by_pos(lo, hi):
        acc = {}
        for r in range(lo, min(hi, rounds)):
            for j, (fk, wk) in enumerate(zip(per["FETCH_SIZE"][r], per["WRITE_SIZE"][r])):
                a = acc.setdefault(j, [0, 0.0, 0.0])
                a[0] += 1
                a[1] += fk
                a[2] += wk
        return acc
    for lo, hi in ((5, 25), (0, rounds)):
        lines.append(f"# launch j of a round, rounds {lo}..{min(hi, rounds) - 1}: launches, "
                     "fetch MB, write MB a launch")
        for j, (n, fk, wk) in sorted(by_pos(lo, hi).items()):
            lines.append(f"#   {j:3d} {n:6d} {fk * 1024 * ff / n / 1e6:10.1f} "
                         f"{wk * 1024 * wf / n / 1e6:8.1f}")
    lines.append("# round, histogram launches, FETCH_SIZE KiB, WRITE_SIZE KiB (sums over the round)")
    for r in range(rounds):
        lines.append(f"round {r} {len(per['FETCH_SIZE'][r])} {sum(per['FETCH_SIZE'][r]):.0f} "
                     f"{sum(per['WRITE_SIZE'][r]):.0f}")
    path = os.path.join(ROOT, "profiles", f"hist_traffic_{tag}.txt")
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")
    print(path)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default: the rest of the workload's full round count "
                         "for narrow, wide and widebin, else 20)")
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="narrow",
                    choices=["narrow", "multiclass", "quantile", "wide", "widebin", "streaming",
                             "shap", "predict"])
    ap.add_argument("--rows", type=int, default=0, help="rows (0: the workload's own size)")
    ap.add_argument("--max-bin", type=int, default=0,
                    help="narrow and streaming workloads: 255 or 256 (8-bit cells; 256 bins fill "
                         "a byte where no value is missing) or more (u16); default 255 for "
                         "narrow, the configured 256 for streaming")
    ap.add_argument("--gpu-math", default="exact", choices=["exact", "fast"],
                    help="narrow, multiclass, quantile and wide workloads: exact (byte-identical "
                         "trees) or fast (hardware exp on the device)")
    ap.add_argument("--cpu-rounds", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run a device copy of MIB MiB (counter calibration) and exit")
    ap.add_argument("--traffic-summary", metavar="DIR", default=None,
                    help="write the workload's histogram counter summary under profiles/ from "
                         "the rocprofv3 --pmc runs under DIR (no GPU needed) and exit")
    args = ap.parse_args()
    if args.steps is None:
        # A training workload's default run is the whole job: warmup plus
        # timed rounds add up to its round count (500, 200 and 300 rounds).
        full = FULL_ROUNDS.get(args.workload)
        args.steps = max(1, full - args.warmup) if full else 20
    if args.max_bin == 0 and args.workload != "streaming":
        args.max_bin = 255
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only; --gpus {args.gpus} is not supported "
              "(the training path is single-device)", file=sys.stderr)
        return 2
    if args.copy_probe:
        return copy_probe(args.copy_probe)
    if args.traffic_summary:
        return traffic_summary(args, args.traffic_summary)

    import ferrisboost_amd as fb

    if not fb.device_available(0):
        print("no gfx950 device at cuda:0", file=sys.stderr)
        return 1

    t0 = time.time()
    if args.workload == "shap":
        out = shap_workload(args)
    elif args.workload == "predict":
        out = predict_workload(args)
    elif args.workload == "streaming":
        out = streaming_workload(args)
    else:
        X, y, params = workload_data(args)
        log(f"data {X.shape} generated in {time.time() - t0:.1f}s")
        desc, tag = workload_desc(args)
        if args.workload != "widebin":
            params = dict(params, gpu_math=args.gpu_math)
        out = train_workload(args, X, y, params, desc, tag)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
