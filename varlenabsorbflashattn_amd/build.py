"""Build the HIP C-ABI library ``libvafa.so`` in-tree for gfx950.

Every translation unit is compiled by ``hipcc --offload-arch=gfx950`` in
parallel, then linked into one shared object next to this file.  The library
exports only the ``extern "C"`` functions declared in ``include/vafa.h``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
ROOT = os.path.dirname(HERE)
LIB_NAME = "libvafa.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
SOURCES = ["plan.cpp", "capi.cpp", "simt.hip", "reduce.hip", "varlen_mfma.hip", "varlen_bwd_mfma.hip",
           "varlen_f32.hip",
           "absorb_mfma.hip", "absorb_bwd_mfma.hip", "absorb_f32.hip",
           "absorb_project.hip"]
ARCH = os.environ.get("VAFA_OFFLOAD_ARCH", "gfx950")


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libvafa.so)")


def _flags():
    return [
        "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
        f"--offload-arch={ARCH}",
        # packed fp32 ops are disabled for all device code on this target
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-fvisibility=hidden",
        "-I", os.path.join(ROOT, "include"),
    ]


def _compile(src: str, obj_dir: str) -> str:
    obj = os.path.join(obj_dir, os.path.splitext(src)[0] + ".o")
    cmd = [_hipcc(), *_flags(), "-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src}\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = True) -> str:
    obj_dir = os.path.join(HERE, "_build")
    os.makedirs(obj_dir, exist_ok=True)
    jobs = min(len(SOURCES), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, obj_dir), SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build()
    sys.exit(0)
