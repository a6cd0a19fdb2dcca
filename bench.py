#!/usr/bin/env python3
"""Benchmark of the device training path on one MI355X.

Workload (default): 10.5M x 28 HIGGS-like binary classification, max_bin=255
(u8 bins), depth 8, eta 0.1, gpu_math="exact" (host gradients, byte-identical
trees). One step = one boosting round. W warmup rounds, then K timed rounds,
all resident in HBM; the round timer runs between blocking device syncs.

Prints one JSON line:
  value      boosting rounds per second over the K timed rounds
  roofline   histogram kernels: algorithmic bytes (cells + 16 B gradient pair
             + 4 B row id per accumulated row, + 32 B per written histogram
             bin) over their HIP-event time, against 8 TB/s HBM
  cpu_baseline  the CPU oracle (C++ restatement of the reference CPU engine)
             on the same data, first R rounds, host threads stated
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
METRIC = "histogram build GB/s (% HBM peak) + boosting rounds/sec, 10.5M×28 u8 bins depth 8"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def load_traffic(path: str):
    """`key = value` lines of a committed rocprofv3 counter summary."""
    out = {}
    try:
        with open(path) as f:
            for line in f:
                if "=" in line and not line.lstrip().startswith("#"):
                    k, v = line.split("=", 1)
                    try:
                        out[k.strip()] = float(v.split()[0])
                    except (ValueError, IndexError):
                        pass
    except OSError:
        return None
    return out or None


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


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--rows", type=int, default=10_500_000)
    ap.add_argument("--max-bin", type=int, default=255)
    ap.add_argument("--cpu-rounds", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run a device copy of MIB MiB (counter calibration) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only; --gpus {args.gpus} is not supported "
              "(the training path is single-device)", file=sys.stderr)
        return 2
    if args.copy_probe:
        return copy_probe(args.copy_probe)

    import ferrisboost_amd as fb
    from ferrisboost_amd import _native as N
    from ferrisboost_amd import datasets

    if not fb.device_available(0):
        print("no gfx950 device at cuda:0", file=sys.stderr)
        return 1

    t0 = time.time()
    X, y, params, _ = datasets.narrow_binary(args.rows, max_bin=args.max_bin)
    log(f"data {X.shape} generated in {time.time() - t0:.1f}s")
    rounds = args.warmup + args.steps
    gparams = dict(params, device="cuda:0", hip_profile=True)
    t0 = time.time()
    model = fb.train(gparams, X, y, num_boost_round=rounds)
    log(f"trained {rounds} rounds in {time.time() - t0:.1f}s "
        f"(setup {model.stats['setup_seconds']:.1f}s)")
    wall = np.zeros(rounds)
    hms = np.zeros(rounds)
    hbytes = np.zeros(rounds, np.uint64)
    n = N.train_lib().fbt_last_round_stats(N.ptr(wall), N.ptr(hms), N.ptr(hbytes), rounds)
    assert n == rounds
    timed = slice(args.warmup, rounds)
    t_wall = float(wall[timed].sum())
    t_hist_ms = float(hms[timed].sum())
    b_hist = float(hbytes[timed].astype(np.float64).sum())
    rounds_per_sec = args.steps / t_wall
    hist_gbps = b_hist / (t_hist_ms * 1e-3) / 1e9 if t_hist_ms > 0 else 0.0
    launches = int(model.stats["hist_launches"])
    bytes_per_launch = float(model.stats["hist_bytes"]) / launches if launches else 0.0
    traffic = load_traffic(os.path.join(ROOT, "profiles",
                                        f"hist_traffic_narrow_{'u8' if args.max_bin <= 255 else 'u16'}.txt"))
    roofline = {
        "bound": "hbm",
        "achieved": round(hist_gbps, 1),
        "peak": HBM_PEAK_GBPS,
        "unit": "GB/s",
        "frac": round(hist_gbps / HBM_PEAK_GBPS, 4),
        "traffic": traffic.get("hbm_bytes_per_launch") if traffic else None,
        "algorithmic_bytes_per_launch": round(bytes_per_launch),
    }

    cpu = None
    parity = None
    if not args.no_cpu:
        from oracle import oracle as O

        threads = min(16, os.cpu_count() or 1)
        cols = max(1, -(-X.shape[1] // threads))
        op = {k: v for k, v in params.items() if k != "device"}
        op.update(n_rounds=args.cpu_rounds, cols_per_block=cols, nthread=threads)
        t0 = time.time()
        om = O.train(X, y, O.make_params(**op))
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
                      "gradient, split and partition single-threaded)",
        }
        parity = all(
            np.array_equal(om.tree(t)[f], model.tree_nodes(t)[f])
            for t in range(args.cpu_rounds) for f in om.tree(t).dtype.names if f != "pad")

    out = {
        "metric": METRIC,
        "value": round(rounds_per_sec, 3),
        "unit": "rounds/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * t_wall / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int64",
        "data": "synthetic",
        "config": {
            "workload": f"narrow {X.shape[0]}x{X.shape[1]} HIGGS-like binary, max_bin={args.max_bin} "
                        f"({'u8' if args.max_bin <= 255 else 'u16'} bins), depth 8, eta 0.1, "
                        "gpu_math=exact, depthwise",
            "rows": int(X.shape[0]),
            "features": int(X.shape[1]),
            "max_bin": args.max_bin,
            "max_depth": 8,
        },
        "hist_gbps": round(hist_gbps, 1),
        "hist_ms_per_round": round(t_hist_ms / args.steps, 3),
        "hist_launches_per_round": round(launches / rounds, 2),
        "host_gradient_ms_per_round": round(1e3 * model.stats["host_gradient_seconds"] / rounds, 3),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "parity_first_rounds_vs_cpu": parity,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
