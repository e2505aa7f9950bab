"""The log-mel kernel's FFT arithmetic (scriptrs_amd/csrc/sfe_fft.hpp: the
16-point DFTs with the window and the internal twiddles folded into fused
multiply-adds, the split with tangent-form twiddles) run on the host by
tests/fft_host_driver.cpp against float64 DFTs, including whole frames
through the device twiddle tables.  No GPU is used."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "scriptrs_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_fft_pieces_against_float64(tmp_path):
    exe = str(tmp_path / "fft_host")
    # host arithmetic exactly as written: fmaf where the header fuses, no
    # other contraction
    subprocess.run([HIPCC, "-O2", "-std=c++17", "-x", "hip", "--offload-arch=gfx950", "-ffp-contract=off",
                    "-Wno-unused-command-line-argument", "-I", os.path.join(ROOT, "include"), "-I", CSRC,
                    os.path.join(ROOT, "tests", "fft_host_driver.cpp"), os.path.join(CSRC, "sfe_tables.cpp"),
                    "-o", exe], check=True, stderr=subprocess.DEVNULL)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0 and "bad 0" in r.stdout, r.stdout + r.stderr
