"""Builds libnest_splat.so for gfx950 from csrc/ with hipcc (no GPU needed).

    python nest-splatting_amd/build.py [--jobs N]

Objects go to nest-splatting_amd/_build/, the shared library to
nest-splatting_amd/nest_splat/libnest_splat.so (in-tree, so that it travels
with the source tree).  Every translation unit is compiled with
-ffp-contract=off (the kernels' float evaluation order is part of their
contract) and with packed FP32 instructions disabled.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "nest_splat", "libnest_splat.so")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")

SOURCES = ["abi.cpp", "preprocess.hip", "binning.hip", "render.hip", "backward.hip", "grid_encode.hip", "mlp.hip",
           "rvq.hip"]

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
ARCH = os.environ.get("NEST_OFFLOAD_ARCH", "gfx950")
CFLAGS = [f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-Wall", "-Wno-unused-function", "-Wno-unused-variable", f"-I{INCLUDE}"]


def _headers_mtime() -> float:
    hs = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")]
    hs += [os.path.join(INCLUDE, f) for f in os.listdir(INCLUDE) if f.endswith(".h")]
    return max(os.path.getmtime(h) for h in hs)


def _compile(src: str, incremental: bool = False) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    if incremental and os.path.exists(obj):
        newest = max(os.path.getmtime(os.path.join(CSRC, src)), _headers_mtime())
        if os.path.getmtime(obj) > newest:
            return obj
    cmd = [HIPCC, *CFLAGS]
    if src.endswith(".cpp"):
        cmd += ["-x", "hip"]
    cmd += ["-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr[-6000:]}")
    return obj


def build(jobs: int = 4, verbose: bool = True, incremental: bool = False) -> str:
    """Compiles every source (incremental: only those older than their
    object file or any header) and links the library."""
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(lambda src: _compile(src, incremental), SOURCES))
    tmp = OUT + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-6000:]}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 4))
    ap.add_argument("--incremental", action="store_true", help="recompile only sources newer than their objects")
    a = ap.parse_args()
    try:
        build(a.jobs, incremental=a.incremental)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
