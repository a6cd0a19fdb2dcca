"""Build recipe of the native libraries (hipcc, gfx950 code objects).

libfbhip.so   the device backend behind include/fbhip.h (HIP kernels + C ABI)
libfbtrain.so the host round driver behind include/fbtrain.h (C++), linked
              against libfbhip.so

Run `python -m ferrisboost_amd.build` (or call build()) after changing a
source; loading never compiles.
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
ROOT = os.path.dirname(HERE)
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -ffp-contract=off: no FMA contraction, every float op rounds like the host
# engine. Correctly rounded f32 divide/sqrt for TreeSHAP. Packed fp32 ops are
# disabled (a known-unreliable instruction family on this hardware).
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-result",
]

BACKEND_SRCS = ["fbhip_kernels.hip", "fbhip_ctx.hip", "fbhip_shap.hip", "fbhip_sketch.hip"]
DRIVER_SRCS = ["fbt_data.cpp", "fbt_train.cpp", "fbt_model.cpp", "fbt_json.cpp", "fbt_api.cpp"]

LIB_HIP = os.path.join(HERE, "libfbhip.so")
LIB_TRAIN = os.path.join(HERE, "libfbtrain.so")


def _run(cmd):
    print(" ".join(cmd), flush=True)
    subprocess.check_call(cmd)


def build(jobs: int = 4) -> None:
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    objs = []
    procs = []
    for s in BACKEND_SRCS:
        o = os.path.join(objdir, s + ".o")
        objs.append(o)
        procs.append(subprocess.Popen([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, s), "-o", o]))
    for p in procs:
        if p.wait() != 0:
            raise RuntimeError("hipcc failed")
    tmp = LIB_HIP + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB_HIP)
    drv = [os.path.join(CSRC, s) for s in DRIVER_SRCS if os.path.exists(os.path.join(CSRC, s))]
    if drv:
        tmp = LIB_TRAIN + ".tmp"
        _run(["g++", "-std=c++17", "-O2", "-fPIC", "-shared", "-ffp-contract=off", "-pthread",
              "-I", os.path.join(ROOT, "include"), "-o", tmp, *drv, "-L", HERE, "-lfbhip",
              "-Wl,-rpath,$ORIGIN"])
        os.replace(tmp, LIB_TRAIN)


if __name__ == "__main__":
    build()
    sys.exit(0)
