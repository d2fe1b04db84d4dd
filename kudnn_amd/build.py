"""Builds the native libraries of the package in-tree.

- ``kudnn_amd/lib/libkudnn_hip.so``: the HIP kernels for gfx950 and the C ABI (``include/kudnn_hip.h``),
  compiled with hipcc.
- ``kudnn_amd/lib/libkudnn.so``: the KuDNN-compatible C++ API (``include/kudnn.hpp``), host-only, compiled
  with g++ and linked against libkudnn_hip.so (rpath $ORIGIN).

Run ``python -m kudnn_amd.build`` or call :func:`build_all`.
"""
from __future__ import annotations

import concurrent.futures
import hashlib
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
HOST = PKG / "host"
LIB = PKG / "lib"
BUILD = PKG / "_build"
INCLUDE = ROOT / "include"

ARCH = os.environ.get("KUDNN_OFFLOAD_ARCH", "gfx950")
HIP_SOURCES = ["gemm_mfma.hip", "gemm_pingpong.hip", "gemm_kslice.hip", "skinny_bf16.hip", "pack.hip", "capi.cpp"]
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    # Packed-FP32 instructions are kept out of every kernel (the compiler would form them from
    # scalar float code); this is a device-only feature flag, the host pass ignores it with a warning.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Wall", "-Wextra"]


# The ping-pong kernel's translation unit and the headers it compiles from: their digest is compiled into the library
# (kudnn_pingpong_source_digest) and recorded with the C3 traffic counters, which bench.py reports only for a library
# built from the same sources.
PINGPONG_SOURCES = ["gemm_pingpong.hip", "device_common.h", "kmajor_copy.h", "kernels.h", "plan_types.h"]


def pingpong_digest() -> str:
    """SHA-256 (first 16 hex digits) over the names and bytes of PINGPONG_SOURCES."""
    h = hashlib.sha256()
    for name in PINGPONG_SOURCES:
        h.update(name.encode() + b"\0" + (CSRC / name).read_bytes() + b"\0")
    return h.hexdigest()[:16]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libkudnn_hip.so)")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out)


def build_hip(verbose: bool = False) -> Path:
    """Compiles every HIP translation unit for gfx950 and links libkudnn_hip.so."""
    hipcc = _hipcc()
    BUILD.mkdir(exist_ok=True)
    LIB.mkdir(exist_ok=True)
    objs = []
    jobs = []
    for src in HIP_SOURCES:
        obj = BUILD / (Path(src).stem + ".o")
        objs.append(obj)
        extra = [f'-DKUDNN_PINGPONG_DIGEST="{pingpong_digest()}"'] if src == "gemm_pingpong.hip" else []
        jobs.append([hipcc, *HIP_FLAGS, *extra, "-c", str(CSRC / src), "-o", str(obj)])
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(4, len(jobs))) as ex:
        list(ex.map(lambda c: _run(c, verbose), jobs))
    out = LIB / "libkudnn_hip.so"
    tmp = LIB / "libkudnn_hip.so.tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)], verbose)
    os.replace(tmp, out)
    return out


def build_cpp(verbose: bool = False) -> Path:
    """Compiles the KuDNN C++ API (host code only) into libkudnn.so on top of libkudnn_hip.so."""
    sources = sorted(HOST.glob("*.cpp"))
    out = LIB / "libkudnn.so"
    tmp = LIB / "libkudnn.so.tmp"
    cxx = os.environ.get("CXX", "g++")
    cmd = [cxx, *CXX_FLAGS, "-shared", "-I", str(INCLUDE), "-I", str(CSRC), *map(str, sources),
           "-L", str(LIB), "-lkudnn_hip", "-Wl,-rpath,$ORIGIN", "-o", str(tmp)]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


def build_all(verbose: bool = False) -> None:
    build_hip(verbose)
    build_cpp(verbose)


if __name__ == "__main__":
    build_all(verbose="-v" in sys.argv)
    print("built", LIB / "libkudnn_hip.so", LIB / "libkudnn.so")
