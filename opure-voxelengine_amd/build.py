"""Builds libopure_hip.so (gfx950 HIP kernels + the C-ABI of include/opure_hip.h)
and the C++20 engine library, in-tree, with hipcc.

    python opure-voxelengine_amd/build.py [--jobs N]

Objects go to opure-voxelengine_amd/_build/, libraries to opure-voxelengine_amd/lib/.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
ENGINE = os.path.join(HERE, "engine")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "lib")
HIP_LIB = os.path.join(LIB, "libopure_hip.so")
ENGINE_LIB = os.path.join(LIB, "libopure_engine.so")

ARCH = "gfx950"
HIP_SOURCES = ["runtime.hip", "gemv.hip", "gemv_f32.hip", "gemv_i8.hip", "gemv_i4h.hip", "gemv_i4b.hip",
               "attention.hip", "accept.hip", "verify.hip"]
# -ffp-contract=off: every float expression rounds as written (fmas are
# explicit __fmaf_rn), like the CPU oracle.  Packed-fp32 instructions stay
# off: they are emitted only from plain float
# code by the compiler, and are kept out of every kernel in this library.
HIP_FLAGS = ["-O3", "-std=c++20", "-fPIC", f"--offload-arch={ARCH}", "-Wall", "-Wno-unused-function", "-ffp-contract=off",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-I", os.path.join(ROOT, "include")]


def hipcc() -> str:
    for cand in ("/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _compile(src: str, obj: str) -> str:
    cmd = [hipcc(), *HIP_FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def _stale(src: str, obj: str, headers_mtime: float) -> bool:
    return not os.path.exists(obj) or os.path.getmtime(obj) < max(os.path.getmtime(src), headers_mtime)


def build(jobs: int = 8, verbose: bool = False, incremental: bool = False) -> str:
    """Compiles every HIP source (incremental: only those older than their
    object or than any header) and links both libraries."""
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIB, exist_ok=True)
    headers = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")]
    headers += [os.path.join(ROOT, "include", f) for f in os.listdir(os.path.join(ROOT, "include"))]
    hm = max(os.path.getmtime(h) for h in headers)
    objs = []
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        futs = []
        for s in HIP_SOURCES:
            obj = os.path.join(BUILD, s.replace(".hip", ".o"))
            src = os.path.join(CSRC, s)
            if incremental and not _stale(src, obj, hm):
                objs.append(obj)
                continue
            futs.append(ex.submit(_compile, src, obj))
        for f in futs:
            objs.append(f.result())
    tmp = HIP_LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, HIP_LIB)
    if verbose:
        print("built", HIP_LIB)
    if os.path.isdir(ENGINE) and any(f.endswith(".cpp") for f in os.listdir(ENGINE)):
        srcs = sorted(os.path.join(ENGINE, f) for f in os.listdir(ENGINE) if f.endswith(".cpp"))
        tmp = ENGINE_LIB + ".tmp"
        cmd = ["g++", "-O2", "-std=c++20", "-fPIC", "-shared", "-Wall", "-Wextra",
               "-I", os.path.join(ROOT, "include"), "-I", ENGINE, "-o", tmp, *srcs,
               f"-L{LIB}", "-lopure_hip", "-Wl,-rpath,$ORIGIN"]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"engine build failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
        os.replace(tmp, ENGINE_LIB)
        if verbose:
            print("built", ENGINE_LIB)
    return HIP_LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=8)
    ap.add_argument("--incremental", action="store_true", help="recompile only sources older than a header or object")
    args = ap.parse_args()
    build(args.jobs, verbose=True, incremental=args.incremental)
    sys.exit(0)
