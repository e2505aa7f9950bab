"""Writes the committed fixtures under tests/golden/.

The reference ships no golden vectors (it has no fixtures and its Rust
cannot be built here), so the fixtures hold:
  * chunk tables of the long-form planner for the benchmark lengths and for
    edge lengths, from the pure-Python restatement in oracle/planner.py
    (itself pinned by the reference's planner tests, whose assertions are
    re-run in tests/test_oracle.py);
  * float64 log-mel of small inputs from tests/np_reference.py (numpy rfft +
    float64 Slaney filterbank), the exact values the f32 paths approximate.
Run from the repo root: python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

from oracle import planner  # noqa: E402
import np_reference as R  # noqa: E402


def plan_summary(n):
    t = planner.build_fast_execution_plan(n)
    lens = [x.audio_end - x.audio_start for x in t]
    return {
        "audio_len": n, "count": len(t),
        "first": [t[0].audio_start, t[0].audio_end, t[0].global_sample_offset, t[0].context_samples] if t else None,
        "last": [t[-1].audio_start, t[-1].audio_end, t[-1].global_sample_offset, t[-1].context_samples] if t else None,
        "sum_len": int(sum(lens)), "sum_frames": int(sum(l // 160 + 1 for l in lens)),
        "tasks": [[x.audio_start, x.audio_end, x.global_sample_offset, x.context_samples] for x in t] if len(t) <= 300 else None,
    }


def main():
    lens = [0, 1, 1280, 96_000, 238_080, 238_081, 240_000, 240_001, 444_160, 444_161, 600_000,
            1_000_000, 57_600_000, 460_800_000]
    with open(os.path.join(HERE, "planner_tables.json"), "w") as f:
        json.dump([plan_summary(n) for n in lens], f, indent=0)

    sr = 16000
    t = np.arange(sr, dtype=np.float32)
    cases = {
        "sine1k_1s": np.sin(np.float32(2 * np.pi) * np.float32(1000) * t / np.float32(sr)).astype(np.float32),
        "sine440_1s": np.sin(np.float32(2 * np.pi) * np.float32(440) * t / np.float32(sr)).astype(np.float32),
        "impulse_4000": np.eye(1, 4000, 1234, dtype=np.float32)[0] * np.float32(0.5),
        "chirp_7777": np.sin(2 * np.pi * (50 + 3000 * np.arange(7777) / 7777) * np.arange(7777) / sr).astype(np.float32),
    }
    rng = np.random.default_rng(20260101)
    cases["noise_5000"] = (0.1 * rng.standard_normal(5000)).astype(np.float32)
    out = {}
    for k, a in cases.items():
        out[k + "_audio"] = a
        out[k + "_logmel_raw64"] = R.logmel_raw(a).astype(np.float32)  # f64 values, stored rounded to f32
        out[k + "_features64"] = R.extract(a).astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "logmel_small.npz"), **out)


if __name__ == "__main__":
    main()
