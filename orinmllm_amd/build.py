"""Build liborin_attn.so (gfx950) in-tree with hipcc.

Usage: python -m orinmllm_amd.build [--jobs N]

The library has no PyTorch dependency: it exports the C ABI of include/orin_attn.h.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_PATH = os.path.join(PKG_DIR, "liborin_attn.so")
SOURCES = ["decode.hip", "decode_mfma.hip", "fwd.hip", "fwd_pp.hip", "producers.hip", "outproj.hip", "capi.hip"]
# C++ host mirror of kuiper's kernel:: functions and op:: layers over the C ABI.
HOST_DIR = os.path.join(PKG_DIR, "cpp")
HOST_SOURCES = ["base.cpp", "kernels.cpp", "layers.cpp"]
HOST_LIB_PATH = os.path.join(PKG_DIR, "liborin_attn_host.so")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # packed fp32 VALU ops are disabled for every kernel in this library
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(REPO, "include"),
    "-I", CSRC,
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: a ROCm toolchain is required to build liborin_attn.so")
    return path


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{res.stderr}")
    return obj


def build_host(verbose: bool = False) -> str:
    """Compile the C++ host mirror into liborin_attn_host.so, linked to liborin_attn.so."""
    objs = []
    for src in HOST_SOURCES:
        obj = os.path.join(BUILD_DIR, "host_" + os.path.splitext(src)[0] + ".o")
        cmd = [hipcc(), "-std=c++17", "-O2", "-fPIC", "-Wall", "-I", os.path.join(HOST_DIR, "include"),
               "-I", os.path.join(REPO, "include"), "-c", os.path.join(HOST_DIR, "src", src), "-o", obj]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{res.stderr}")
        objs.append(obj)
    tmp = HOST_LIB_PATH + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", "-o", tmp, *objs, "-L", PKG_DIR, "-lorin_attn",
           "-Wl,-rpath,$ORIGIN"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"host link failed:\n{res.stderr}")
    os.replace(tmp, HOST_LIB_PATH)
    if verbose:
        print(f"built {HOST_LIB_PATH}")
    return HOST_LIB_PATH


def build(jobs: int | None = None, verbose: bool = False) -> str:
    """Compile every HIP source for gfx950 and link liborin_attn.so, then the C++ host
    mirror liborin_attn_host.so. Always recompiles."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB_PATH + ".tmp"
    # rocBLAS serves the output projection (a plain GEMM); everything else is this library's.
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, "-lrocblas"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    build_host(verbose)
    return LIB_PATH


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args(argv)
    build(args.jobs, verbose=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
