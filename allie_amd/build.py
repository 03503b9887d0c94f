"""Builds the gfx950 engine library ``allie_amd/liballie_amd.so`` in-tree.

``python -m allie_amd.build`` (or ``__graft_entry__.build()``) compiles every
``csrc/*.hip`` with hipcc for gfx950 and links one shared library; the host
rules library ``liballie_chess.so`` is built from ``csrc/*.cpp`` with g++.  Each
translation unit compiles in parallel; the library is replaced atomically.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "liballie_amd.so")
CHESS_LIB = os.path.join(HERE, "liballie_chess.so")
ARCH = os.environ.get("ALLIE_OFFLOAD_ARCH", "gfx950")

# Packed fp32 instructions (v_pk_*_f32) are kept out of every kernel: some of
# their forms have given wrong results now and then on the MI355X boxes this
# was built on; the host pass warns that it does not know the feature.
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found")


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    cmd = [_hipcc(), *FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build_chess(verbose: bool = False) -> str:
    """The host rules library (``csrc/*.cpp``, no GPU code) with the host
    C++ compiler."""
    cxx = os.environ.get("CXX") or shutil.which("g++") or shutil.which("c++")
    if not cxx:
        raise RuntimeError("no host C++ compiler (g++) found")
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.cpp")))
    tmp = f"{CHESS_LIB}.tmp{os.getpid()}"  # per process: concurrent first uses may build at once
    cmd = [cxx, "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", *srcs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"host build failed:\n{r.stderr}")
    os.replace(tmp, CHESS_LIB)
    if verbose:
        print(f"built {CHESS_LIB}")
    return CHESS_LIB


def build(verbose: bool = False) -> str:
    build_chess(verbose)
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
