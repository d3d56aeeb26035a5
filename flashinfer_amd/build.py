"""Builds libmi_moe.so (all HIP kernels + the C ABI) for gfx950 with hipcc.

Usage: python -m flashinfer_amd.build [--jobs N] [--save-temps]
The shared library lands next to this file so it travels with the tree.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmi_moe.so")
SOURCES = ["route.hip", "sort.hip", "gemm1.hip", "gemm2.hip", "gemm1_tile.hip", "gemm2_tile.hip",
           "gemm2_combine.hip", "combine.hip", "capi.hip"]
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall",
    # code object v5 loads in every ROCm 6.x/7.x runtime, including the one
    # bundled with the PyTorch wheel
    "-mcode-object-version=5",
    "-Wno-unused-command-line-argument",
    # packed fp32 VALU ops stay off: the compiler must not form v_pk_*_f32
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build libmi_moe.so")
    return path


def _compile(src: str, extra) -> str:
    obj = os.path.join(BUILD, src.replace(".hip", ".o"))
    cmd = [hipcc(), *HIPCC_FLAGS, *extra, "-I", os.path.join(HERE, "..", "include"),
           "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    warn = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if warn.strip():
        print(warn, file=sys.stderr)
    return obj


def build(jobs: int = 8, extra=()) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, list(extra)), SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-mcode-object-version=5", "-shared", "-fPIC",
           *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("--save-temps", action="store_true", help="keep ISA dumps in _build/")
    a = ap.parse_args()
    extra = ["-save-temps=obj"] if a.save_temps else []
    print(build(a.jobs, extra))


if __name__ == "__main__":
    main()
