"""Builds ``libscriptrs_fe.so`` in-tree with hipcc for gfx950.

Each source is compiled with an explicit hipcc line, then all are linked
into one shared library next to this file.  No CMake, no JIT cache: the
built ``.so`` travels with the source tree.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(CSRC, "_obj")
LIB = os.path.join(HERE, "libscriptrs_fe.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # Keep the compiler from forming packed fp32 (v_pk_*_f32) instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
    "-Wall", "-Wno-unused-command-line-argument",
]

SOURCES = [
    # (source, extra flags)
    ("sfe_kernels.hip", ["-x", "hip"]),
    ("sfe_vad.hip", ["-x", "hip"]),
    ("sfe_noalloc.hip", ["-x", "hip"]),
    # bit-exact table construction: every f32/f64 op rounded separately
    ("sfe_tables.cpp", ["-x", "hip", "-ffp-contract=off"]),
    ("sfe_capi.cpp", ["-x", "hip"]),
]


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    objs = []
    for src, extra in SOURCES:
        obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
        cmd = [HIPCC, *COMMON, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        objs.append(obj)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
