"""Builds ``libscriptrs_fe.so`` in-tree with hipcc for gfx950.

Each source is compiled with an explicit hipcc line, then all are linked
into one shared library next to this file.  No CMake, no JIT cache: the
built ``.so`` travels with the source tree.
"""
from __future__ import annotations

import os
import re
import subprocess
import sys
import tempfile

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
    ("sfe_share.cpp", ["-x", "hip"]),
    ("sfe_capi.cpp", ["-x", "hip"]),
]


# Kernel sources whose generated assembly is checked for MFMAs with a
# destination overlapping their own A or B operand.  The register allocator
# allows that overlap (it treats the operands as read at issue); whether the
# matrix cores read every block's operands before the destination is written
# is not documented, so the kernels are kept free of it.
MFMA_CHECKED = ("sfe_kernels.hip",)
_MFMA_RE = re.compile(r"\bv_mfma\w*\s+v\[(\d+):(\d+)\],\s*v(\d+),\s*v(\d+)")


def mfma_operand_overlaps(asm: str) -> list[str]:
    """Lines of ``asm`` where an MFMA's VGPR destination range contains its
    A or B operand register."""
    bad = []
    for line in asm.splitlines():
        m = _MFMA_RE.search(line)
        if m:
            d0, d1, a, b = map(int, m.groups())
            if d0 <= a <= d1 or d0 <= b <= d1:
                bad.append(line.strip())
    return bad


def lane_masked_loops(asm: str, kernel: str) -> int:
    """Loops of ``kernel`` in ``asm`` whose trip is controlled per lane (the
    back edge masks lanes out of exec: ``s_andn2_b64 exec, exec, ...``)."""
    m = re.search(r"^(_Z\S*" + kernel + r"\S*):", asm, re.M)
    if not m:
        raise RuntimeError(f"kernel {kernel} not found in the generated assembly")
    body = asm[m.start():asm.index(".Lfunc_end", m.start())]
    return body.count("s_andn2_b64 exec, exec")


# The log-mel kernels' work loop takes its units through a lane-0 counter
# broadcast with readfirstlane, which is only sound while all 64 lanes go
# round the loop together.  The compiler may instead structurise a loop with
# lane-conditional code into a per-lane (exec-masked) loop in which lanes
# leave at different iterations; a handoff probe built that way looped
# forever.  These kernels may have no per-lane loop at all.
# (one entry per sample type t and mel schedule m of each workgroup size)
LANE_LOOP_LIMITS = {"sfe_logmel_kernelI[t]Li12ELi[m]E": 0, "sfe_logmel_kernelI[t]Li4ELi[m]E": 0}


def vgpr_spills(asm: str) -> dict[str, int]:
    """Kernel name -> .vgpr_spill_count from the code object metadata."""
    out = {}
    for m in re.finditer(r"\.name:\s+(\S+)\n(?:(?!\.name:).)*?\.vgpr_spill_count:\s+(\d+)", asm, re.S):
        out[m.group(1)] = int(m.group(2))
    return out


def check_asm(src: str, extra: list[str], verbose: bool = False) -> None:
    with tempfile.TemporaryDirectory() as tmp:
        out = os.path.join(tmp, "k.s")
        cmd = [HIPCC, *COMMON, *extra, "--cuda-device-only", "-S", os.path.join(CSRC, src), "-o", out]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True, stderr=subprocess.DEVNULL)
        asm = open(out).read()
    bad = mfma_operand_overlaps(asm)
    if bad:
        raise RuntimeError(f"{src}: MFMA destination overlaps its own A/B operand:\n  " + "\n  ".join(bad))
    # A spill in these kernels puts scratch loads (and full vmcnt waits) into
    # their loops: the product and the measurement build must have none.
    spilled = {k: n for k, n in vgpr_spills(asm).items() if n and ("logmel" in k or "norm" in k)}
    if spilled:
        raise RuntimeError(f"{src}: registers spilled in " + ", ".join(f"{k} ({n})" for k, n in spilled.items()))
    for pat, limit in LANE_LOOP_LIMITS.items():
        for t, m in ((t, m) for t in "fsi" for m in "01"):
            k = pat.replace("[t]", t).replace("[m]", m)
            n = lane_masked_loops(asm, k)
            if n > limit:
                raise RuntimeError(f"{src}: {k} has {n} per-lane loops (at most {limit}): its work loop "
                                   "must stay a wave-uniform loop")


LIB_TS = os.path.join(HERE, "libscriptrs_fe_ts.so")


def build(verbose: bool = False, timestamps: bool = False) -> str:
    """Builds the product library; with timestamps, the measurement build
    (kernels compiled with -DSFE_TIMESTAMPS, see sfe_debug_stamps) into
    libscriptrs_fe_ts.so instead."""
    obj_dir = os.path.join(OBJ, "ts") if timestamps else OBJ
    lib = LIB_TS if timestamps else LIB
    os.makedirs(obj_dir, exist_ok=True)
    objs = []
    for src, extra in SOURCES:
        obj = os.path.join(obj_dir, os.path.splitext(src)[0] + ".o")
        if timestamps and src == "sfe_kernels.hip":
            extra = [*extra, "-DSFE_TIMESTAMPS"]
        cmd = [HIPCC, *COMMON, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        objs.append(obj)
        if src in MFMA_CHECKED:
            check_asm(src, extra, verbose)
    tmp = lib + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv, timestamps="--timestamps" in sys.argv))
