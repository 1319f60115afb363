"""Build the gfx950 attention library in-tree.

``python -m toyinfer_amd.build`` (or ``__graft_entry__.build()``) compiles
every HIP and host C++ source under ``toyinfer_amd/csrc`` with hipcc (one
object per source, compiled in parallel under ``toyinfer_amd/lib/obj``) and
links them into ``toyinfer_amd/lib/libtoyinfer_attn.so``.  Packed-FP32 VALU forms are
disabled on purpose: some of their encodings have produced silently wrong
results on the target machines, and the kernels do not depend on them.
"""
from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB_DIR = os.path.join(HERE, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libtoyinfer_attn.so")
SYNTH_PATH = os.path.join(LIB_DIR, "libtoyinfer_synth.so")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build")
    return path


def sources() -> list:
    """HIP kernels and launchers (*.hip) plus host-only C++ (*.cpp)."""
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))


def build_synth(verbose: bool = False) -> str:
    """Host-only synthetic-input generator (same bits as synth.py's numpy code)."""
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = SYNTH_PATH + ".tmp"
    cmd = ["gcc", "-O3", "-march=x86-64-v3", "-ffp-contract=off", "-fno-fast-math", "-fopenmp",
           "-fPIC", "-shared", "-std=c11", "-Wall", "-o", tmp,
           os.path.join(CSRC, "synth.c"), "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, SYNTH_PATH)
    return SYNTH_PATH


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed building libtoyinfer_attn.so")


def build_library(verbose: bool = False) -> str:
    """One object per source (in parallel), then one shared library."""
    from concurrent.futures import ThreadPoolExecutor

    os.makedirs(LIB_DIR, exist_ok=True)
    obj_dir = os.path.join(LIB_DIR, "obj")
    os.makedirs(obj_dir, exist_ok=True)
    srcs = sources()
    objs = [os.path.join(obj_dir, os.path.basename(src) + ".o") for src in srcs]
    cmds = [[hipcc(), *HIP_FLAGS, "-c", "-o", obj, src] for src, obj in zip(srcs, objs)]
    workers = min(len(cmds), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        list(pool.map(lambda c: _run(c, verbose), cmds))
    tmp = LIB_PATH + ".tmp"
    _run([hipcc(), *HIP_FLAGS, "-shared", "-o", tmp, *objs], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def build_all(verbose: bool = False) -> None:
    build_library(verbose)
    build_synth(verbose)


if __name__ == "__main__":
    build_all(verbose=True)
