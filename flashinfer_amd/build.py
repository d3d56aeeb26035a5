"""Builds libmi_moe.so (all HIP kernels + the C ABI, for the default
definition: H=7168, I=2048, 32 of 256 experts, 8 groups, top-4 groups,
top-8), one libmi_moe_<tag>.so per further definition in
shapes.DEFINITIONS, and libmi_peaks.so (achievable-peak probes used by
bench.py), for gfx950 with hipcc; and _mi_moe_host, the native host path of
kernel.run (host C++ against torch's headers, built with g++).

Usage: python -m flashinfer_amd.build [--jobs N] [--save-temps]
The shared libraries land next to this file so they travel with the tree.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

from .shapes import DEFINITIONS, definition_supported, lib_name_of

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmi_moe.so")
SOURCES = ["route.hip", "sort.hip", "gemm1.hip", "gemm2.hip", "gemm1_tile.hip", "gemm2_tile.hip",
           "gemm1_wide.hip", "gemm2_wide.hip", "gemm2_combine.hip", "combine.hip", "quant.hip", "capi.hip"]
PEAKS_LIB = os.path.join(HERE, "libmi_peaks.so")
PEAKS_SOURCES = ["peaks.hip"]
# Per-source flags: MFMA results in VGPRs rather than AGPRs.
# * peaks.hip: in the default AGPR form the compiler gives the bf16 MFMA
#   loop partially overlapping srcC / vdst registers and shuffles every
#   chain through VGPRs each round.
# * gemm1.hip: each MFMA result is scaled in VALU; the VGPR form drops a
#   v_accvgpr_read per result register (GEMM1 stream 1% faster at T=64).
SOURCE_FLAGS = {"peaks.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
                "gemm1.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
                "gemm1_wide.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
                "gemm2_wide.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}
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


def _compile(src: str, extra, defn=None) -> str:
    sub = os.path.join(BUILD, defn.tag if defn else "common")
    os.makedirs(sub, exist_ok=True)
    obj = os.path.join(sub, src.replace(".hip", ".o"))
    defs = defn.defines() if defn else []
    cmd = [hipcc(), *HIPCC_FLAGS, *SOURCE_FLAGS.get(src, []), *defs, *extra,
           "-I", os.path.join(HERE, "..", "include"),
           "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    warn = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if warn.strip():
        print(warn, file=sys.stderr)
    return obj


def _link(objs, out):
    tmp = out + ".tmp"
    # -Bsymbolic: each shape's library binds its own kernels and helpers even
    # when several (same C++ names, other shape constants) share a process
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-mcode-object-version=5", "-shared", "-fPIC",
           "-Wl,-Bsymbolic", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link of {os.path.basename(out)} failed:\n{r.stderr}")
    os.replace(tmp, out)


HOST_SRC = os.path.join(CSRC, "host_bind.cpp")
HOST_LIB = os.path.join(HERE, "_mi_moe_host" + sysconfig.get_config_var("EXT_SUFFIX"))


def build_host() -> str:
    """The torch extension _mi_moe_host: host code only, so g++ builds it
    (against torch's headers and its bundled pybind11) without hipcc."""
    import torch
    tdir = os.path.dirname(torch.__file__)
    tlib = os.path.join(tdir, "lib")
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = HOST_LIB + ".tmp"
    cmd = [shutil.which("g++") or "g++", "-O2", "-shared", "-fPIC", "-std=c++17", "-Wall",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DUSE_ROCM", "-D__HIP_PLATFORM_AMD__=1",
           "-I", os.path.join(tdir, "include"),
           "-I", os.path.join(tdir, "include", "torch", "csrc", "api", "include"),
           "-I", sysconfig.get_paths()["include"], "-I", os.path.join(rocm, "include"),
           HOST_SRC, "-o", tmp, "-L", tlib, "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
           "-ltorch_python", "-L", os.path.join(rocm, "lib"), "-lamdhip64",
           f"-Wl,-rpath,{tlib}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"g++ failed on host_bind.cpp:\n{r.stderr}")
    os.replace(tmp, HOST_LIB)
    return HOST_LIB


def build(jobs: int = 8, extra=()) -> str:
    bad = [d for d in DEFINITIONS if not definition_supported(d)]
    if bad:
        raise ValueError(f"unsupported definitions (see shapes.py): {bad}")
    os.makedirs(BUILD, exist_ok=True)
    jobs_list = [(s, d) for d in DEFINITIONS for s in SOURCES] + [(s, None) for s in PEAKS_SOURCES]
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda j: _compile(j[0], list(extra), j[1]), jobs_list))
    n = len(SOURCES)
    for k, d in enumerate(DEFINITIONS):
        _link(objs[k * n:(k + 1) * n], os.path.join(HERE, lib_name_of(d)))
    _link(objs[len(DEFINITIONS) * n:], PEAKS_LIB)
    build_host()
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
