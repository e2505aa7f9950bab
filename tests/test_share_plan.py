"""Shared frames planner (scriptrs_amd/csrc/sfe_share.cpp) on the host, no
GPU: tests/share_plan_driver.cpp replays the kernels' addressing over the
planned tables and checks that every frame an item's normalisation reads was
written by a log-mel entry from exactly the padded samples the item itself
would use (the key of a frame: its first sample in the recording, the zero
padding on each side and where preemphasis restarts).  Cases: long-form plans
(src/long_form/mod.rs) of several lengths, ragged clip batches, overlapping
tasks at mixed offsets modulo the hop, duplicated and nested tasks, tasks
shorter than a frame."""
import os
import subprocess

import numpy as np
import pytest

from scriptrs_amd.long_form import build_fast_execution_plan

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "scriptrs_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def _cases():
    rng = np.random.default_rng(7)
    cases = []
    for n in (16_000 * 30, 16_000 * 61, 16_000 * 600, 16_000 * 3600 // 4, 57_600_000):
        t = build_fast_execution_plan(n)
        cases.append([(c.audio_start, c.audio_end - c.audio_start) for c in t])
    # the 8 h plan: runs are cut at 2^20 shared frames
    t = build_fast_execution_plan(460_800_000)
    cases.append([(c.audio_start, c.audio_end - c.audio_start) for c in t])
    # the 1 h plan in shuffled order
    c = list(cases[4])
    rng.shuffle(c)
    cases.append(c)
    # clips back to back (nothing to share)
    off = np.concatenate([[0], np.cumsum(rng.integers(1, 320_000, 64))])
    cases.append([(int(off[i]), int(off[i + 1] - off[i])) for i in range(64)])
    # overlapping tasks at random starts (mixed residues modulo the hop), random lengths
    for _ in range(6):
        st = np.sort(rng.integers(0, 2_000_000, 40))
        cases.append([(int(s), int(rng.integers(1, 300_000))) for s in st])
    # hop-aligned overlapping tasks of random lengths, some duplicated, some nested
    for _ in range(6):
        st = np.sort(rng.integers(0, 10_000, 30)) * 160
        ln = rng.integers(1, 200_000, 30)
        c = [(int(s), int(l)) for s, l in zip(st, ln)]
        c += c[:5] + [(c[3][0] + 1600, max(1, c[3][1] // 3))]
        cases.append(c)
    # short tasks around the interior threshold, and a single long one
    cases.append([(160 * i, 160 * 33 + 255 + i) for i in range(0, 200, 7)])
    cases.append([(0, 1), (0, 255), (0, 256), (0, 257), (160, 5536), (320, 5536)])
    cases.append([(0, 57_600_000)])
    # 40,000 copies of one task: runs are cut at kMaxShareMembers (16384) members
    cases.append([(1600, 16_000)] * 40_000)
    return cases


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_shared_frames_plan(tmp_path):
    exe = str(tmp_path / "share_plan")
    subprocess.run([HIPCC, "-O1", "-std=c++17", "-x", "hip", "--cuda-host-only", "-I", CSRC,
                    "-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "share_plan_driver.cpp"),
                    os.path.join(CSRC, "sfe_share.cpp"), "-o", exe], check=True, stderr=subprocess.DEVNULL)
    lines = []
    cases = _cases()
    for share in (1, 0):
        for c in cases:
            lines.append(f"{len(c)} {share}")
            lines += [f"{s} {l}" for s, l in c]
    r = subprocess.run([exe], input="\n".join(lines) + "\n", capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    assert r.stdout.strip().endswith("bad 0"), r.stdout[-3000:]
    res = [ln.split() for ln in r.stdout.splitlines() if ln.startswith("case")]
    assert len(res) == 2 * len(cases)
    shared = [(int(x[3]), int(x[4])) for x in res[:len(cases)]]
    # the 1 h long-form plan: the ~2 s chunk overlaps are computed once
    q, own = shared[4]
    assert q < 0.88 * own, (q, own)
    # the 8 h plan, and the 1 h plan shuffled
    assert shared[5][0] < 0.88 * shared[5][1] and shared[6] == shared[4]
    # back-to-back clips: nothing shared
    assert shared[7][0] == shared[7][1]
    # the copies: three shared regions
    assert int(res[len(cases) - 1][8]) == 3 and shared[-1][0] < shared[-1][1]
