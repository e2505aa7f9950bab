"""The C ABI's host logic under AddressSanitizer + UndefinedBehaviorSanitizer
(no GPU needed): sfe_capi.cpp, sfe_share.cpp and sfe_tables.cpp are rebuilt with the
sanitizers on their host pass only (hipcc -Xarch_host -fsanitize=...), linked
with the kernel objects that build() produced, and driven by
tests/host_sanitizer_driver.cpp: tables, the planner over lengths up to 8 h,
overlap configs including invalid ones, argument errors, and a context
creation that fails for lack of a device (checked for leaks)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "scriptrs_amd", "csrc")
OBJ = os.path.join(CSRC, "_obj")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_host_logic_under_asan_ubsan(tmp_path):
    kobjs = ("sfe_kernels.o", "sfe_vad.o", "sfe_noalloc.o")
    for o in kobjs:
        if not os.path.exists(os.path.join(OBJ, o)):
            pytest.skip("kernel objects not built (run build() first)")
    flags = ["-O1", "-g", "-std=c++17", "-fPIC", "--offload-arch=gfx950",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-I", os.path.join(ROOT, "include"), "-I", CSRC, "-x", "hip", "-Wno-unused-command-line-argument",
             "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
             "-Xarch_host", "-fno-omit-frame-pointer", "-Xarch_host", "-fno-sanitize-recover=all"]
    objs = []
    for src, extra in (("sfe_capi.cpp", []), ("sfe_share.cpp", []), ("sfe_tables.cpp", ["-ffp-contract=off"])):
        o = str(tmp_path / (src + ".o"))
        subprocess.run([HIPCC, *flags, *extra, "-c", os.path.join(CSRC, src), "-o", o], check=True,
                       stderr=subprocess.DEVNULL)
        objs.append(o)
    drv = str(tmp_path / "drv.o")
    subprocess.run([HIPCC, *flags, "-c", os.path.join(ROOT, "tests", "host_sanitizer_driver.cpp"), "-o", drv],
                   check=True, stderr=subprocess.DEVNULL)
    exe = str(tmp_path / "drv")
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-fsanitize=address,undefined", drv, *objs,
                    *(os.path.join(OBJ, o) for o in kobjs), "-o", exe], check=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="halt_on_error=1")
    r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "bad 0" in r.stdout, r.stdout
