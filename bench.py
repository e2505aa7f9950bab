"""Benchmark of the MI355X log-mel front end (one JSON line on stdout).

A step is one pass of the front end over one batch of synthetic input: the
log-mel kernel, then the normalisation kernel, over every chunk of the
workload.  The default workload is the 1-hour long-form recording (BASELINE
config 3): 57.6M samples split into 280 overlapping chunk tasks by scriptrs'
planner, all featurized in one launch sequence with the input already
resident in HBM.  The north-star bandwidth target is stated on this config.
Other workloads: config1/2/4 (resident), config5 (8 h streamed from pinned
host memory in 60 s windows: PCIe-inclusive, never the headline figure),
vad1h (the Silero VAD model inputs of the config-3 recording: one framing
kernel, bytes in + 576 floats out per 512-sample window), config1host (the
config-1 clip through the reference's own entry point, extract(&[f32]) on
host memory: copy in, both kernels, copy out and synchronise per call).
--pcm i16 feeds 16-bit PCM decoded in the kernel.

value      = audio seconds featurized per second (RTFx), whole job
roofline   = the whole path (log-mel then normalisation): algorithmic HBM
             bytes (input bytes per unique sample + 128 output values per
             frame) over the summed durations of both kernels (HIP events on
             the stream they run on), against the 8 TB/s HBM peak; traffic =
             HBM bytes per step of both kernels from the committed rocprofv3
             FETCH_SIZE/WRITE_SIZE runs (the raw log-mel round trip between
             them is above the algorithmic bytes)
logmel     = the log-mel kernel alone: its HBM figure and its vector-issue
             bound (SQ_INSTS_VALU), the limit it is near
cpu_baseline = the CPU oracle (C restatement of src/frontend.rs), timed on
             this host with 4 worker threads (the reference's default
             LongFormConfig::worker_count), over the whole workload: 1 warmup
             then --cpu-runs timed runs (mean, p50, p95); the same again on
             all of the box's CPU share (16 threads) as cpu_baseline_all_cores
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

SR = 16_000
HBM_PEAK_GBS = 8000.0
VALU_PEAK_INSTS_PER_S = 256 * 4 * 2.4e9 / 4  # CUs x SIMDs x clock / 4 cycles per wave64 instruction


def measured_profile(fname: str, applies: bool, key: str = "traffic_bytes"):
    """A per-launch figure from the committed rocprofv3 counter runs, or None:
    traffic_bytes (FETCH_SIZE / WRITE_SIZE, each scaled by what the counter
    reads for a plain copy) or valu_insts_per_launch (SQ_INSTS_VALU).  Only
    valid for the kernel sources those runs measured: the file records the
    sha256 of their concatenation."""
    import hashlib
    tfile = os.path.join(ROOT, "profiles", fname)
    if not applies or not os.path.exists(tfile):
        return None
    t = json.load(open(tfile))
    files = t["kernel_source"]
    h = hashlib.sha256()
    for f in [files] if isinstance(files, str) else files:
        h.update(open(os.path.join(ROOT, f), "rb").read())
    return t.get(key) if h.hexdigest() == t["kernel_source_sha256"] else None


def measured_traffic(fname: str, applies: bool):
    return measured_profile(fname, applies)


def warm_up(step, steps: int, min_s: float) -> None:
    """At least `steps` untimed steps and `min_s` seconds of them (unless
    steps is 0), for the extra configs reported beside the headline (whose
    warmup is exactly --warmup steps): the GPU idles while a workload is
    synthesized, and its clock ramps back up over tens of milliseconds of
    load."""
    import torch
    if steps <= 0:
        return
    t0 = time.perf_counter()
    done = 0
    while done < steps or time.perf_counter() - t0 < min_s:
        for _ in range(steps - done if done < steps else max(1, steps // 4)):
            step()
            done += 1
        torch.cuda.synchronize()


def make_workload(name: str):
    from scriptrs_amd import synth
    from scriptrs_amd.long_form import build_fast_execution_plan, ChunkTask
    if name == "config1":
        x = synth.sinusoids(160_000, 1)
        return x, [ChunkTask(0, x.size, 0, 0)], "one 10 s clip"
    if name == "config2":
        x = synth.dense_batch(64, 240_000, 1000).reshape(-1)
        return x, [ChunkTask(i * 240_000, (i + 1) * 240_000, i * 240_000, 0) for i in range(64)], "64 x 15 s dense batch"
    if name == "config3":
        x = synth.speech_like(57_600_000, 3)
        return x, build_fast_execution_plan(x.size), "1 h long-form recording, 280 overlap chunks, one batched pass"
    if name == "config5":
        x = synth.speech_like(460_800_000, 5)
        return x, build_fast_execution_plan(x.size), \
            "8 h recording streamed from pinned host memory in 60 s double-buffered windows"
    if name == "config4":
        x, off = synth.ragged_batch(256, 4)
        return x, [ChunkTask(int(off[i]), int(off[i + 1]), int(off[i]), 0) for i in range(256)], \
            "256 ragged clips 1-20 s, flat buffer + offsets"
    raise SystemExit(f"unknown workload {name}")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=5,
                    help="untimed steps first (the first is also reported as first_call_ms); the GPU clock ramps "
                         "up over the first tens of ms of load, so more warmup gives the steady-clock figure")
    ap.add_argument("--workload", default="config3", choices=["config1", "config1host", "config2", "config3", "config4", "config5", "vad1h"])
    ap.add_argument("--pcm", default="f32", choices=["f32", "i16"],
                    help="input samples: f32, or 16-bit PCM decoded in the kernel")
    ap.add_argument("--dtype", default="f32", choices=["f32", "bf16"])
    ap.add_argument("--window-samples", type=int, default=960_000,
                    help="config5: device window length in samples (60 s at 16 kHz by default)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-other-configs", dest="other_configs", action="store_false",
                    help="config3 only: skip the short runs of configs 1, 2 and 4 reported beside it")
    ap.add_argument("--no-config5", dest="config5", action="store_false",
                    help="config3 only: leave config 5 (8 h streamed, about 40 s with its synthesis) out of "
                         "the other configs")
    ap.add_argument("--no-steady", dest="steady", action="store_false",
                    help="skip the extra steady-clock timing reported beside the headline")
    ap.add_argument("--cpu-runs", type=int, default=5, help="timed runs of each CPU baseline leg")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB per step (calibrates the HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the path shards by chunk with no collective; see the design notes)", file=sys.stderr)
        return 2

    import torch
    if args.copy_calibration:
        n = args.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(args.warmup + args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_read": 4 * n, "bytes_written": 4 * n}), flush=True)
        return 0
    if args.workload == "vad1h":
        return bench_vad(args)
    if args.workload == "config1host":
        return bench_host_clip(args)
    from scriptrs_amd import ParakeetFeatureExtractor, TaskTable, _lib

    x, tasks, desc = make_workload(args.workload)
    n_audio = int(x.size)
    frames = np.array([(t.audio_end - t.audio_start) // 160 + 1 for t in tasks], np.int64)
    F = int(frames.sum())
    print(f"[bench] workload {args.workload}: {desc}; N_audio={n_audio} tasks={len(tasks)} F_out={F}",
          file=sys.stderr, flush=True)

    ext = ParakeetFeatureExtractor()
    tasks = TaskTable(tasks)  # the plan in the C ABI layout, built once
    out_dt = torch.float32 if args.dtype == "f32" else torch.bfloat16
    out = torch.empty(F * 128, dtype=out_dt, device="cuda")
    stream = torch.cuda.current_stream()
    if args.pcm == "i16":
        x = np.clip(np.round(x.astype(np.float64) * 32767.0), -32768, 32767).astype(np.int16)
    in_bytes = x.itemsize
    streamed = args.workload == "config5"
    if streamed:
        # a new pinned host tensor (page-locked at allocation)
        host = torch.from_numpy(x).pin_memory().numpy()

        def step():
            ext.extract_chunks_streamed(host, tasks, window_samples=args.window_samples, dtype=args.dtype, out=out)
    else:
        dev = torch.from_numpy(x).cuda()

        def step():
            if args.pcm == "i16":
                ext.extract_chunks_pcm(dev, tasks, dtype=args.dtype, stream=stream, out=out)
            else:
                ext.extract_chunks(dev, tasks, dtype=args.dtype, stream=stream, out=out)
    # The first call of the process, timed on its own (host wall clock to the
    # end of its device work): code-object load, scratch allocation, planning
    # and the item-table upload, then both kernels.  It is the first warmup
    # step.
    first_call_ms = None
    if args.warmup > 0:
        torch.cuda.synchronize()
        f0 = time.perf_counter()
        step()
        torch.cuda.synchronize()
        first_call_ms = (time.perf_counter() - f0) * 1e3
    for _ in range(args.warmup - 1):
        step()
    torch.cuda.synchronize()

    # Wall clock of K steps with nothing else on the stream ...
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    # ... then the same K steps again with HIP events around every kernel
    # launch, on the stream each runs on (the per-kernel times; the events
    # add small gaps, so they are kept out of the wall-clock run).
    L = _lib.lib()
    ctx = ext._handle()
    L.sfe_set_timing(ctx, 1)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    lm, nm, nl = ctypes.c_double(), ctypes.c_double(), ctypes.c_int32()
    L.sfe_get_timing(ctx, ctypes.byref(lm), ctypes.byref(nm), ctypes.byref(nl))
    L.sfe_set_timing(ctx, 0)

    # The same steps once the GPU clock has ramped up (after 50 ms or more of
    # back-to-back steps), reported beside the headline, never as it: the
    # median of 5 windows of --steps steps.  (A process's enqueue has been
    # seen to block once for about 35 ms inside the HIP runtime around its
    # 512th dispatch; the GPU idles meanwhile and a window holding it is an
    # outlier.)
    steady_ms = None
    if args.steady:
        warm_up(step, 200, 0.05)
        windows = []
        for _ in range(5):
            torch.cuda.synchronize()
            s0 = time.perf_counter()
            for _ in range(args.steps):
                step()
            torch.cuda.synchronize()
            windows.append((time.perf_counter() - s0) / args.steps * 1e3)
        steady_ms = float(np.median(windows))

    # One call on a fresh context of this warm process: planning (shared
    # frames), the item-table upload and the context's scratch allocation
    # are paid again, the code objects are loaded already.
    fresh_ms = None
    if not streamed:
        ext2 = ParakeetFeatureExtractor()
        ext2._handle()
        torch.cuda.synchronize()
        f0 = time.perf_counter()
        if args.pcm == "i16":
            ext2.extract_chunks_pcm(dev, tasks, dtype=args.dtype, stream=stream, out=out)
        else:
            ext2.extract_chunks(dev, tasks, dtype=args.dtype, stream=stream, out=out)
        torch.cuda.synchronize()
        fresh_ms = (time.perf_counter() - f0) * 1e3
        ext2.close()

    sec = (t1 - t0) / args.steps
    audio_sec = n_audio / SR
    # per step (a call may run as several log-mel/normalisation batches)
    logmel_ms = lm.value / args.steps
    norm_ms = nm.value / args.steps
    out_bytes = 4 if args.dtype == "f32" else 2
    # Algorithmic bytes of the whole front end: every unique input sample read
    # once, every output frame written once (128 features).  The raw log-mel
    # round trip between the two kernels is not algorithmic: it shows up as
    # traffic above these bytes.
    alg_path = in_bytes * n_audio + 128 * out_bytes * F
    alg_logmel = in_bytes * n_audio + 512 * F         # log-mel alone: read audio once, write raw f32 log-mel
    path_ms = logmel_ms + norm_ms
    achieved = alg_path / (path_ms * 1e-3) / 1e9
    prof = "sfe_logmel_longform_1h_traffic.json"
    applies = args.workload == "config3" and args.pcm == "f32" and args.dtype == "f32"
    t_logmel = measured_profile(prof, applies)
    t_norm = measured_profile(prof, applies, "norm_traffic_bytes")

    result = {
        "metric": "audio-sec featurized/sec (RTFx) + achieved HBM GB/s vs peak, 1 MI355X",
        "value": audio_sec / sec,
        "unit": "audio-s/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": sec * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded, scriptrs_amd/synth.py)",
        "config": {"workload": f"{args.workload}: {desc}", "n_audio_samples": n_audio, "chunks": len(tasks),
                   "frames_out": F, "out_dtype": args.dtype, "input": args.pcm,
                   "input_location": "pinned host memory (PCIe-inclusive)" if streamed else "HBM"},
        # The whole path (log-mel then normalisation): algorithmic bytes over
        # the summed durations of both kernels (HIP events on their stream).
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS,
                     "traffic": (t_logmel + t_norm) if (t_logmel and t_norm) else None,
                     "traffic_over_alg": (t_logmel + t_norm) / alg_path if (t_logmel and t_norm) else None,
                     "kernels": ["sfe_logmel_kernel", "sfe_norm_kernel"], "kernel_ms": path_ms,
                     "alg_bytes": alg_path},
        "kernels_ms": {"sfe_logmel_kernel": logmel_ms, "sfe_norm_kernel": norm_ms},
        # wall clock of single calls outside the timed steps (see above)
        "first_call_ms": first_call_ms,
        "steady_clock_ms_per_step": steady_ms,
        "fresh_context_call_ms": fresh_ms,
    }
    # The log-mel kernel alone: its HBM figure, and the limit it is actually
    # near, vector issue (SQ_INSTS_VALU against one wave64 fp32 instruction per
    # SIMD per 4 cycles at 2.4 GHz; 157.3 TFLOP/s counts packed FMA).
    lg = {"bound": "valu", "kernel": "sfe_logmel_kernel", "kernel_ms": logmel_ms, "alg_bytes": alg_logmel,
          "hbm_achieved": alg_logmel / (logmel_ms * 1e-3) / 1e9, "hbm_frac": alg_logmel / (logmel_ms * 1e-3) / 1e9 /
          HBM_PEAK_GBS, "traffic": t_logmel}
    valu = measured_profile(prof, applies, "valu_insts_per_launch")
    if valu:
        peak = VALU_PEAK_INSTS_PER_S
        lg["valu_bound"] = {"insts_per_launch": valu, "peak_insts_per_s": peak,
                            "floor_ms": valu / peak * 1e3, "frac": valu / peak * 1e3 / logmel_ms}
    result["logmel"] = lg
    if not streamed and args.workload == "config3" and args.other_configs:
        result["other_configs_ms_per_step"] = other_configs(ext, args)
    if streamed:
        result["h2d_gbps"] = in_bytes * n_audio / sec / 1e9
        result["config"]["window_samples"] = args.window_samples

    if not args.no_cpu and not streamed:
        import oracle
        starts = tasks.array[:, 0]
        lens = tasks.array[:, 1] - tasks.array[:, 0]
        xf = x if x.dtype == np.float32 else x.astype(np.float32) / np.float32(32767.0)
        oracle.extract_spans(xf, starts[:1], lens[:1], 1)  # load + warm
        # The reference's long-form default is 4 workers (src/long_form.rs:78);
        # the box's CPU share for one GPU is 16 threads.
        all_cores = max(1, min(16, os.cpu_count() or 1))
        legs = {}
        want = None
        for nt in (4, all_cores):
            times = []
            for _ in range(args.cpu_runs):
                c0 = time.perf_counter()
                want, _ = oracle.extract_spans(xf, starts, lens, nt)
                times.append(time.perf_counter() - c0)
            legs[nt] = np.array(times)
        t4 = legs[4]
        result["cpu_baseline"] = {"value": audio_sec / t4.mean(), "unit": "audio-s/s", "cores": 4, "kind": "port",
                                  "sample": f"the whole {args.workload} workload ({len(tasks)} items), "
                                            f"oracle/sfe_oracle.c with 4 worker threads, {args.cpu_runs} runs "
                                            "after a warmup; value from the mean run time",
                                  "p50_s": float(np.percentile(t4, 50)), "p95_s": float(np.percentile(t4, 95))}
        ta = legs[all_cores]
        result["cpu_baseline_all_cores"] = {"value": audio_sec / ta.mean(), "unit": "audio-s/s", "cores": all_cores,
                                            "kind": "port", "p50_s": float(np.percentile(ta, 50)),
                                            "p95_s": float(np.percentile(ta, 95))}
        got = out.float().cpu().numpy()
        err = np.abs(got - want)
        tol = 1e-4 + 1e-3 * np.abs(want)
        # A summary only: the parity gate is tests/test_gpu_parity.py, whose
        # bound also admits the f32 FFT noise of bins near the 2^-24 guard.
        ok = (err <= tol) | np.isnan(want)
        result["parity"] = {"max_abs_err_vs_oracle": float(np.nanmax(err)),
                            "frac_within_1e-4_abs_1e-3_rel": float(ok.mean()),
                            "outside_flat_bar": int((~ok).sum())}
        # Every element outside the flat bar should have a non-zero f32 noise
        # envelope (a near-guard element, float64 mel energy at most 1e-6 of
        # its frame's energy, or a row holding one), as the GPU parity tests
        # require (tests/parity.py).
        if x.dtype == np.float32 and args.dtype == "f32":
            sys.path.insert(0, os.path.join(ROOT, "tests"))
            import np_reference as R
            fo = tasks.frame_offsets
            near = np.zeros(want.size, bool)
            for i in range(len(starts)):
                a = x[int(starts[i]):int(starts[i] + lens[i])]
                near[128 * fo[i]:128 * fo[i + 1]] = (R.f32_noise_envelope(a) > 0).reshape(-1)
            result["parity"]["outside_flat_bar_all_in_envelope"] = bool(not (~ok & ~near).any())
    print(json.dumps(result), flush=True)
    ext.close()
    return 0


def other_configs(ext, args, steps: int = 50, warmup: int = 50) -> dict:
    """Wall-clock ms per step of configs 1, 2 and 4 (resident, f32), run
    after the headline workload in the same process: one launch sequence per
    step, timed over `steps` steps after at least `warmup` untimed ones
    (and at least 100 ms of them); and config 5 (streamed) unless
    --no-config5."""
    import torch
    from scriptrs_amd import TaskTable
    res = {}
    stream = torch.cuda.current_stream()
    for name in ("config1", "config2", "config4"):
        x, tasks, _ = make_workload(name)
        tt = TaskTable(tasks)
        dev = torch.from_numpy(x).cuda()
        out = torch.empty(int(tt.frame_offsets[-1]) * 128, dtype=torch.float32, device="cuda")
        warm_up(lambda: ext.extract_chunks(dev, tt, stream=stream, out=out), warmup, 0.1)
        t0 = time.perf_counter()
        for _ in range(steps):
            ext.extract_chunks(dev, tt, stream=stream, out=out)
        torch.cuda.synchronize()
        res[name] = (time.perf_counter() - t0) / steps * 1e3
        del dev, out
    if args.config5:
        # Config 5: the 8 h recording streamed from pinned host memory in 60 s
        # windows (PCIe-bound, 33 ms per step): 1 warmup and 3 timed steps.
        x, tasks, _ = make_workload("config5")
        tt = TaskTable(tasks)
        host = torch.from_numpy(x).pin_memory().numpy()
        del x
        out = torch.empty(int(tt.frame_offsets[-1]) * 128, dtype=torch.float32, device="cuda")
        ext.extract_chunks_streamed(host, tt, window_samples=960_000, out=out)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(3):
            ext.extract_chunks_streamed(host, tt, window_samples=960_000, out=out)
        torch.cuda.synchronize()
        res["config5"] = (time.perf_counter() - t0) / 3 * 1e3
        del host, out
    return res


def bench_host_clip(args) -> int:
    """One 10 s clip per call through sfe_extract: host samples in, host
    features out, synchronous (ParakeetFeatureExtractor::extract,
    src/frontend.rs:104-118).  Latency-bound: PCIe round trips and launches."""
    import torch  # noqa: F401  (loads the HIP runtime the library shares)
    from scriptrs_amd import ParakeetFeatureExtractor, synth
    x = synth.sinusoids(160_000, 1)
    ext = ParakeetFeatureExtractor()
    for _ in range(max(args.warmup, 3)):
        ext.extract(x)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ext.extract(x)
    sec = (time.perf_counter() - t0) / args.steps
    result = {
        "metric": "audio-sec featurized/sec (RTFx) + achieved HBM GB/s vs peak, 1 MI355X",
        "value": x.size / SR / sec, "unit": "audio-s/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": sec * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (seeded, scriptrs_amd/synth.py)",
        "config": {"workload": "config1host: one 10 s clip per extract() call, host buffers in and out",
                   "n_audio_samples": int(x.size), "input_location": "pageable host memory"},
    }
    if not args.no_cpu:
        import oracle
        oracle.extract(x)
        times = []
        for _ in range(args.cpu_runs):
            c0 = time.perf_counter()
            oracle.extract(x)
            times.append(time.perf_counter() - c0)
        t = np.array(times)
        result["cpu_baseline"] = {"value": x.size / SR / t.mean(), "unit": "audio-s/s", "cores": 1, "kind": "port",
                                  "sample": f"the same clip, oracle/sfe_oracle.c, 1 thread, {args.cpu_runs} runs",
                                  "p50_s": float(np.percentile(t, 50)), "p95_s": float(np.percentile(t, 95))}
    print(json.dumps(result), flush=True)
    ext.close()
    return 0


def bench_vad(args) -> int:
    """The VAD framing kernel over the 1 h recording, resident in HBM."""
    import torch
    from scriptrs_amd import SileroVadFramer, synth, vad_num_windows

    x = synth.speech_like(57_600_000, 3)
    if args.pcm == "i16":
        x = np.clip(np.round(x.astype(np.float64) * 32767.0), -32768, 32767).astype(np.int16)
    n_audio = int(x.size)
    n_win = vad_num_windows(n_audio)
    desc = f"Silero VAD model inputs of the 1 h recording ({n_win} windows of [64 context | 512])"
    print(f"[bench] workload vad1h: {desc}; N_audio={n_audio}", file=sys.stderr, flush=True)
    framer = SileroVadFramer()
    dev = torch.from_numpy(x).cuda()
    out = torch.empty((n_win, 576), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()

    def step():
        framer.model_inputs(dev, stream=stream, out=out)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    # kernel time: events on the stream the kernel runs on (torch's current)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ev[0].record(stream)
    for _ in range(args.steps):
        step()
    ev[1].record(stream)
    torch.cuda.synchronize()
    kernel_ms = ev[0].elapsed_time(ev[1]) / args.steps
    sec = (t1 - t0) / args.steps
    alg = x.itemsize * n_audio + 4 * 576 * n_win  # read each sample once, write every model input
    achieved = alg / (kernel_ms * 1e-3) / 1e9
    result = {
        "metric": "audio-sec featurized/sec (RTFx) + achieved HBM GB/s vs peak, 1 MI355X",
        "value": n_audio / SR / sec,
        "unit": "audio-s/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": sec * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (seeded, scriptrs_amd/synth.py)",
        "config": {"workload": f"vad1h: {desc}", "n_audio_samples": n_audio, "windows": n_win,
                   "input": args.pcm, "input_location": "HBM"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS,
                     "traffic": measured_traffic("sfe_vad_frames_1h_traffic.json", args.pcm == "f32"),
                     "kernel": "sfe_vad_frames_kernel",
                     "kernel_ms": kernel_ms, "alg_bytes": alg},
        "kernels_ms": {"sfe_vad_frames_kernel": kernel_ms},
    }
    if not args.no_cpu:
        import oracle
        xf = x if x.dtype == np.float32 else x.astype(np.float32) / np.float32(32767.0)
        oracle.vad_frames(xf[:4096])  # load + warm
        times = []
        for _ in range(args.cpu_runs):
            c0 = time.perf_counter()
            want = oracle.vad_frames(xf)
            times.append(time.perf_counter() - c0)
        t = np.array(times)
        result["cpu_baseline"] = {"value": n_audio / SR / t.mean(), "unit": "audio-s/s", "cores": 1,
                                  "kind": "port", "sample": "the whole vad1h workload, oracle/sfe_oracle.c "
                                                            f"(the reference's window loop), 1 thread, {args.cpu_runs} "
                                                            "runs after a warmup; value from the mean run time",
                                  "p50_s": float(np.percentile(t, 50)), "p95_s": float(np.percentile(t, 95))}
        result["parity"] = {"bit_exact_vs_oracle": bool(np.array_equal(out.cpu().numpy(), want))}
    print(json.dumps(result), flush=True)
    framer.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
