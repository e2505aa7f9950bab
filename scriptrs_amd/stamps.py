"""Per-wave and per-workgroup timelines of the two kernels, from the
measurement build of the library (kernels compiled with -DSFE_TIMESTAMPS).

    python -m scriptrs_amd.build --timestamps      # writes libscriptrs_fe_ts.so
    python -m scriptrs_amd.stamps --workload config3 --warmup 200

Runs the workload's extraction `--warmup` times, then once more with the
kernels writing s_memrealtime stamps (a 100 MHz clock common to all CUs,
10 ns resolution; see sfe_debug_stamps in include/scriptrs_fe.h), and prints
one JSON object:
  logmel: kernel span (first wave start to last wave end), spread of the
    wave starts, prologue (wave start to its first unit) and its steps,
    wave end percentiles, units per wave and microseconds per unit;
  norm: span, and per workgroup the time to its first reduced statistics
    (loads landed), the statistics, and the stores, plus how many
    workgroups were in each phase at the median instant.
The stamps add a few stores per wave; the figures describe the kernels'
shape, not their exact product timing (bench.py times the product build).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys

import numpy as np

from . import _lib

_HERE = os.path.dirname(os.path.abspath(__file__))
TS_LIB = os.path.join(_HERE, "libscriptrs_fe_ts.so")
LOGMEL_WORDS = 8 * 65536   # words before the normalisation region (8 per wave)
NORM_WORDS = 4 * 65536


def workload(name: str):
    from .long_form import ChunkTask, build_fast_execution_plan
    from . import synth
    if name == "config1":
        x = synth.sinusoids(160_000, 1)
        return x, [ChunkTask(0, x.size, 0, 0)]
    if name == "config2":
        x = synth.dense_batch(64, 240_000, 1000).reshape(-1)
        return x, [ChunkTask(i * 240_000, (i + 1) * 240_000, i * 240_000, 0) for i in range(64)]
    if name == "config3":
        x = synth.speech_like(57_600_000, 3)
        return x, build_fast_execution_plan(x.size)
    if name == "config4":
        x, off = synth.ragged_batch(256, 4)
        return x, [ChunkTask(int(off[i]), int(off[i + 1]), int(off[i]), 0) for i in range(256)]
    raise SystemExit(f"unknown workload {name}")


def pct(a, q):
    return float(np.percentile(a, q)) if len(a) else None


def summarize(st: np.ndarray) -> dict:
    us = 0.01  # 10 ns ticks -> microseconds
    lm = st[:LOGMEL_WORDS].reshape(-1, 8)
    lm = lm[lm[:, 0] > 0]
    nm = st[LOGMEL_WORDS:].reshape(-1, 4)
    nm = nm[nm[:, 0] > 0]
    out = {}
    if len(lm):
        t0 = lm[:, 0].min()
        start, first, end, units, mel, itm = (
            (lm[:, i] - (0 if i == 3 else t0)).astype(np.float64) for i in range(6))
        busy = units > 0
        per_unit = (end[busy] - first[busy]) / units[busy] * us
        out["logmel"] = {
            "waves": int(len(lm)), "span_us": float(end.max() * us),
            "start_spread_us": float(start.max() * us),
            "prologue_us": {"p50": pct((first - start) * us, 50), "p90": pct((first - start) * us, 90)},
            # from the wave's start to its item descriptors' first use (p50)
            "items_loaded_us_p50": pct((itm[busy] - start[busy]) * us, 50),
            "wave_end_us": {"p10": pct(end * us, 10), "p50": pct(end * us, 50), "p90": pct(end * us, 90),
                            "max": float(end.max() * us)},
            "units_per_wave": {"min": int(units.min()), "p50": pct(units, 50), "max": int(units.max())},
            "units_total": int(units.sum()),
            "us_per_unit": {"p10": pct(per_unit, 10), "p50": pct(per_unit, 50), "p90": pct(per_unit, 90)},
        }
    if len(nm):
        t0 = nm[:, 0].min()
        s, a, b, e = ((nm[:, i] - t0).astype(np.float64) * us for i in range(4))
        mid = (e.max()) / 2
        out["norm"] = {
            "workgroups": int(len(nm)), "span_us": float(e.max()),
            "load_and_first_sum_us": {"p50": pct(a - s, 50), "p90": pct(a - s, 90)},
            "statistics_us": {"p50": pct(b - a, 50), "p90": pct(b - a, 90)},
            "stores_us": {"p50": pct(e - b, 50), "p90": pct(e - b, 90)},
            "lifetime_us": {"p50": pct(e - s, 50), "p90": pct(e - s, 90)},
            "at_half_span": {"loading": int(((s <= mid) & (a > mid)).sum()),
                             "statistics": int(((a <= mid) & (b > mid)).sum()),
                             "storing": int(((b <= mid) & (e > mid)).sum())},
        }
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", default="config3", choices=["config1", "config2", "config3", "config4"])
    ap.add_argument("--warmup", type=int, default=200)
    args = ap.parse_args()
    if not os.path.exists(TS_LIB):
        print(f"{TS_LIB} is not built: python -m scriptrs_amd.build --timestamps", file=sys.stderr)
        return 2
    _lib.LIB_PATH = TS_LIB  # before the first call loads the library
    import torch
    from .frontend import ParakeetFeatureExtractor, TaskTable
    x, tasks = workload(args.workload)
    tt = TaskTable(tasks)
    ext = ParakeetFeatureExtractor()
    dev = torch.from_numpy(x).cuda()
    out = torch.empty(int(tt.frame_offsets[-1]) * 128, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()
    for _ in range(args.warmup):
        ext.extract_chunks(dev, tt, stream=stream, out=out)
    torch.cuda.synchronize()
    buf = torch.zeros(LOGMEL_WORDS + NORM_WORDS, dtype=torch.int64, device="cuda")
    L = _lib.lib()
    if L.sfe_debug_stamps(ctypes.c_void_p(buf.data_ptr()), buf.numel()) != _lib.SFE_OK:
        print(_lib.last_error(), file=sys.stderr)
        return 1
    ext.extract_chunks(dev, tt, stream=stream, out=out)
    torch.cuda.synchronize()
    L.sfe_debug_stamps(None, 0)
    res = {"workload": args.workload, "warmup": args.warmup, **summarize(buf.cpu().numpy())}
    print(json.dumps(res))
    ext.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
