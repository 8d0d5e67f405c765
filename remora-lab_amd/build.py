"""Build librkv.so (the C-ABI library of include/rkv.h) for gfx950 with hipcc.

Run as a script or call build().  Objects compile in parallel, then link in
place next to this file so the library travels with the source tree.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "librkv.so")
OBJDIR = os.path.join(HERE, "_build")

SOURCES = ["rkv_append.hip", "rkv_decode.hip", "rkv_decode_rows32.hip", "rkv_prefill.hip",
           "rkv_r4kv.hip", "rkv_stream.hip", "rkv_scratch.hip", "rkv_runtime.cpp", "rkv_serve.cpp"]

# Per-file extra flags.  rkv_decode.hip: MFMA destinations and accumulators
# in VGPRs (no AGPR<->VGPR copies around the VALU work on them).  The
# two-wave 32-row variant (rkv_decode_rows32.hip) is bounded to 256 registers
# per wave by its launch bounds and allocates no AGPRs either way.
EXTRA = {"rkv_decode.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}

# -packed-fp32-ops off: no v_pk_*_f32 are generated (unreliable on this pool).
# f32 division and sqrt stay correctly rounded and f32 denormals are kept, so
# the quantizer is bit-exact with the IEEE CPU reference.
HIPFLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-gpu-flush-denormals-to-zero",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-I" + os.path.join(HERE, "..", "include"),
]


def _hipcc() -> str:
    for c in ("/opt/rocm/bin/hipcc", "hipcc"):
        if os.path.sep not in c or os.path.exists(c):
            return c
    return "hipcc"


def _compile(src: str) -> str:
    obj = os.path.join(OBJDIR, os.path.splitext(src)[0] + ".o")
    cmd = [_hipcc(), *HIPFLAGS, *EXTRA.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".hip"):
        cmd[1:1] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = OUT + ".tmp"
    cmd = [_hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc link failed:\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
