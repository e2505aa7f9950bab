"""GPU: the host paths above the batched kernels, as the reference's callers
use them.

* ``ChunkPreparer::prepare`` / ``TranscriptionPipeline::prepare_chunk``
  (src/pipeline.rs:145-164, :201-216): a valid clip returns the features
  with ``feature_frames == T`` and ``target_frames == 1501``; a clip one
  sample past 15 s is ``AudioTooLong``; both through a live context, in
  Python and through the C ABI's ``sfe_prepare_chunk``.
* ``featurize_long_form``, the batched replacement of the long-form workers
  (src/long_form.rs:266-342): a recording that fits one chunk becomes one
  task over the whole recording (src/long_form.rs:161-163); a longer one is
  planned and every task is featurized, in task order, with the frame
  offsets of the oracle's planner and values against the oracle.
* The measurement build's stamps (scriptrs_amd/stamps.py) are consistent.
"""
import ctypes
import json
import os

import numpy as np
import pytest

import np_reference as R
import oracle
from conftest import assert_parity
from oracle import planner
from scriptrs_amd import (AudioTooLong, ChunkPreparer, TranscriptionConfig, _lib, featurize_long_form, synth)

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _flush(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def preparer():
    p = ChunkPreparer()
    yield p
    p.extractor.close()


@pytest.mark.parametrize("n", [1, 160_000, 240_000])
def test_chunk_preparer_success_path(preparer, n):
    _flush(f"case: ChunkPreparer.prepare length {n}")
    a = synth.sinusoids(n, 300 + n)
    pc = preparer.prepare(a)
    T = n // 160 + 1
    assert pc.feature_frames == T == pc.features.shape[0]
    assert pc.target_frames == 1501 == TranscriptionConfig().max_feature_frames()
    assert pc.features.shape == (T, 128)
    assert_parity(pc.features, oracle.extract(a).T, R.extract(a).T, R.f32_noise_envelope(a).T, what=f"prepare {n}")


def test_chunk_preparer_too_long_through_live_context(preparer):
    _flush("case: ChunkPreparer.prepare 240001 samples")
    preparer.prepare(np.zeros(16_000, np.float32))  # the context is live
    with pytest.raises(AudioTooLong) as e:
        preparer.prepare(np.zeros(240_001, np.float32))
    assert e.value.max_seconds == 15.0 and abs(e.value.actual_seconds - 240_001 / 16_000) < 1e-12


def test_sfe_prepare_chunk_c_abi(preparer):
    _flush("case: sfe_prepare_chunk through the C ABI")
    L = _lib.lib()
    ctx = preparer.extractor._handle()
    a = synth.sinusoids(200_000, 77)
    T = 200_000 // 160 + 1
    out = np.full((128, T), np.nan, np.float32)
    ff = ctypes.c_int64(-1)
    fp = lambda x: x.ctypes.data_as(ctypes.POINTER(ctypes.c_float))  # noqa: E731
    rc = L.sfe_prepare_chunk(ctx, fp(a), a.size, fp(out), out.size, ctypes.byref(ff))
    assert rc == _lib.SFE_OK, _lib.last_error()
    assert ff.value == T
    assert_parity(out, oracle.extract(a), R.extract(a), R.f32_noise_envelope(a), what="sfe_prepare_chunk")
    big = np.zeros(240_001, np.float32)
    ff.value = -1
    rc = L.sfe_prepare_chunk(ctx, fp(big), big.size, fp(out), out.size, ctypes.byref(ff))
    assert rc == _lib.SFE_AUDIO_TOO_LONG and ff.value == -1
    assert "actual=15.00s max=15.00s" in _lib.last_error()
    rc = L.sfe_prepare_chunk(ctx, fp(big), 0, fp(out), out.size, ctypes.byref(ff))
    assert rc == _lib.SFE_EMPTY_AUDIO


def _check_long_form(lf, rec, want_tasks):
    got = [(t.audio_start, t.audio_end, t.global_sample_offset, t.context_samples) for t in lf.tasks]
    assert got == want_tasks
    starts = [t[0] for t in want_tasks]
    lens = [t[1] - t[0] for t in want_tasks]
    want, wfo = oracle.extract_spans(rec, starts, lens)
    assert np.array_equal(lf.frame_offsets, wfo)
    feats = lf.features.cpu().numpy()
    for i, (s, n) in enumerate(zip(starts, lens)):
        a, b = int(wfo[i]), int(wfo[i + 1])
        chunk = lf.chunk(i).cpu().numpy()
        assert chunk.shape == (128, b - a)
        assert np.array_equal(chunk.reshape(-1), feats[128 * a:128 * b])
        x = rec[s:s + n]
        assert_parity(chunk, want[128 * a:128 * b].reshape(128, -1), R.extract(x), R.f32_noise_envelope(x),
                      what=f"task {i}")


def test_featurize_long_form_single_chunk_branch(preparer):
    import torch
    _flush("case: featurize_long_form 200000 samples (one task)")
    rec = synth.speech_like(200_000, 31)
    lf = featurize_long_form(preparer.extractor, torch.from_numpy(rec).cuda())
    torch.cuda.synchronize()
    _check_long_form(lf, rec, [(0, rec.size, 0, 0)])


@pytest.mark.parametrize("n", [240_001, 1_000_003])
def test_featurize_long_form_planned_branch(preparer, n):
    import torch
    _flush(f"case: featurize_long_form {n} samples (planned)")
    rec = synth.speech_like(n, 32)
    lf = featurize_long_form(preparer.extractor, torch.from_numpy(rec).cuda())
    torch.cuda.synchronize()
    want = [(t.audio_start, t.audio_end, t.global_sample_offset, t.context_samples)
            for t in planner.build_fast_execution_plan(n)]
    assert len(want) >= 2
    _check_long_form(lf, rec, want)


def test_measurement_build_stamps_are_consistent():
    """The measurement build's timelines (scriptrs_amd/stamps.py) on the
    config-1 clip: every log-mel wave and normalisation workgroup left
    ordered stamps, and the waves' units add up to the launch's quads."""
    import subprocess
    import sys
    from scriptrs_amd import stamps
    if not os.path.exists(stamps.TS_LIB):
        pytest.skip("measurement build not present (python -m scriptrs_amd.build --timestamps)")
    _flush("case: measurement build stamps, config 1")
    r = subprocess.run([sys.executable, "-m", "scriptrs_amd.stamps", "--workload", "config1", "--warmup", "3"],
                       capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 0, r.stdout + r.stderr
    res = json.loads(r.stdout.strip().splitlines()[-1])
    lm, nm = res["logmel"], res["norm"]
    assert lm["waves"] > 0 and lm["span_us"] > 0 and lm["prologue_us"]["p50"] >= 0
    assert lm["units_total"] == (1001 + 3) // 4
    assert nm["workgroups"] == 8 and nm["span_us"] > 0
    assert nm["lifetime_us"]["p50"] >= nm["stores_us"]["p50"] >= 0
