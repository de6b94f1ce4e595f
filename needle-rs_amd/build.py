"""Build libneedle_hip.so (gfx950) in-tree with hipcc.

Usage: python needle-rs_amd/build.py   (or __graft_entry__.build()).

Flags that matter for parity: -ffp-contract=off (the reference never fuses
a*b+c; every fma in the kernels is an explicit __builtin_fmaf), correctly
rounded f32 division and sqrt (HIP's default; no fast-math), packed FP32
instructions disabled.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "needle_hip")
LIB = os.path.join(OUT_DIR, "libneedle_hip.so")
OBJ_DIR = os.path.join(HERE, "_build")

SOURCES = ["nh_api.hip", "nh_act.hip", "nh_gemv.hip", "nh_gemv_res.hip", "nh_gemm.hip", "nh_misc.hip", "nh_forward.hip",
           "nh_archive.cpp", "nh_model.cpp"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in ordinary VGPRs: the epilogue reads every one of them.
    "-mllvm", "--amdgpu-mfma-vgpr-form",
    "-Wall",
    "-Wno-unused-result",
]


# Per-file flags.  The forward's kernels run one to a few dozen workgroups
# each and wait on their arguments first: their first 16 argument dwords
# are preloaded into SGPRs at wave launch (the Needle-3 decode token 537.5 ->
# 526 us).  So are the resident matrices' GEMVs, the decode step's products
# (520.7 -> 510.8 us).  The streamed GEMV measured slower with it (the
# 512-workgroup K = 2048 product 3.63 -> 3.68 us) and the GEMMs the same, so
# they keep the plain argument loads.
PRELOAD = ["-mllvm", "-amdgpu-kernarg-preload-count=16"]
FILE_FLAGS = {"nh_forward.hip": PRELOAD, "nh_gemv_res.hip": PRELOAD}


def _compile(src: str) -> str:
    obj = os.path.join(OBJ_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, *FILE_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ_DIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
