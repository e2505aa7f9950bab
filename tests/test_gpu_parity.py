"""GPU parity: the HIP path through the C ABI against the CPU oracle."""
import numpy as np
import pytest

import oracle
import np_reference as R
from conftest import assert_parity
from scriptrs_amd import synth

pytestmark = pytest.mark.gpu


def _flush(msg):
    print(msg, flush=True)


def test_config1_clip(extractor):
    _flush("case: config-1 10 s clip seed 1")
    a = synth.sinusoids(160_000, 1)
    got = extractor.extract(a)
    want = oracle.extract(a).T
    assert got.shape == (1001, 128)
    err, widened = assert_parity(got, want, R.extract(a).T, R.f32_noise_envelope(a).T, what="config1")
    print("max abs err", err, "widened", widened)


@pytest.mark.parametrize("n", [1, 2, 159, 160, 161, 319, 320, 400, 401, 511, 512, 513, 5119, 5120, 5121,
                               16_000, 48_123, 240_000])
def test_lengths(extractor, n):
    _flush(f"case: length {n}")
    a = synth.sinusoids(n, 100 + n)
    got = extractor.extract(a)
    want = oracle.extract(a).T
    assert got.shape == (n // 160 + 1, 128)
    assert_parity(got, want, R.extract(a).T, R.f32_noise_envelope(a).T, what=f"len {n}")


def test_zero_audio_matches_reference_rounding(extractor):
    """Digital silence: every row is constant ln(2^-24); the reference's
    sequential f32 mean leaves x - mean != 0, so the output is a constant
    that the GPU must reproduce bit for bit."""
    _flush("case: zero audio")
    for n in (16_000, 160_000, 240_000):
        a = np.zeros(n, np.float32)
        got = extractor.extract(a)
        want = oracle.extract(a).T
        assert np.array_equal(got, want), n


def test_dense_batch(extractor):
    import torch
    _flush("case: dense batch 8 x 240000")
    x = synth.dense_batch(8, 240_000, 7)
    dev = torch.from_numpy(x.reshape(-1)).cuda()
    off = np.arange(9, dtype=np.int64) * 240_000
    out, fo = extractor.extract_batch(dev, off)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    assert list(np.diff(fo)) == [1501] * 8
    for i in range(8):
        want = oracle.extract(x[i])
        assert_parity(out[128 * fo[i]:128 * fo[i + 1]].reshape(128, -1), want, R.extract(x[i]),
                      R.f32_noise_envelope(x[i]), what=f"clip {i}")


def test_ragged_batch(extractor):
    import torch
    _flush("case: ragged batch 24")
    flat, off = synth.ragged_batch(24, 11)
    dev = torch.from_numpy(flat).cuda()
    out, fo = extractor.extract_batch(dev, off)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    want, wfo = oracle.extract_spans(flat, off[:-1], np.diff(off))
    assert np.array_equal(fo, wfo)
    clips = [flat[off[i]:off[i + 1]] for i in range(24)]
    ref = np.concatenate([R.extract(c).reshape(-1) for c in clips])
    env = np.concatenate([R.f32_noise_envelope(c).reshape(-1) for c in clips])
    assert_parity(out, want, ref, env, what="ragged")


def test_long_form_chunks(extractor):
    import torch
    from scriptrs_amd import build_fast_execution_plan
    _flush("case: long form 1.5M samples")
    rec = synth.speech_like(1_500_000, 5)
    tasks = build_fast_execution_plan(rec.size)
    dev = torch.from_numpy(rec).cuda()
    out, fo = extractor.extract_chunks(dev, tasks)
    torch.cuda.synchronize()
    starts = [t.audio_start for t in tasks]
    lens = [t.audio_end - t.audio_start for t in tasks]
    want, wfo = oracle.extract_spans(rec, starts, lens)
    assert np.array_equal(fo, wfo)
    ref = np.concatenate([R.extract(rec[s:s + n]).reshape(-1) for s, n in zip(starts, lens)])
    env = np.concatenate([R.f32_noise_envelope(rec[s:s + n]).reshape(-1) for s, n in zip(starts, lens)])
    err, widened = assert_parity(out.cpu().numpy(), want, ref, env, what="long form")
    print("max abs err", err, "widened", widened)


def test_bf16_matches_rounded_f32(extractor):
    import torch
    _flush("case: bf16 output")
    flat, off = synth.ragged_batch(6, 3)
    dev = torch.from_numpy(flat).cuda()
    o32, _ = extractor.extract_batch(dev, off, dtype="f32")
    o16, _ = extractor.extract_batch(dev, off, dtype="bf16")
    torch.cuda.synchronize()
    assert torch.equal(o32.to(torch.bfloat16), o16)


def test_streamed_equals_resident(extractor):
    import torch
    from scriptrs_amd import build_fast_execution_plan
    _flush("case: streamed 3M samples")
    rec = synth.speech_like(3_000_000, 9)
    tasks = build_fast_execution_plan(rec.size)
    a, fa = extractor.extract_chunks(torch.from_numpy(rec).cuda(), tasks)
    b, fb = extractor.extract_chunks_streamed(rec, tasks, window_samples=960_000)
    torch.cuda.synchronize()
    assert np.array_equal(fa, fb)
    assert torch.equal(a, b)


@pytest.mark.parametrize("pinned", [False, True])
def test_streamed_ring_wraps_equals_resident(extractor, pinned):
    """One task per window (250,000-sample windows) over 12 M samples: about
    58 windows, so the device ring of window slots wraps many times and the
    normalisation runs at its 32-window boundary and at the end."""
    import torch
    from scriptrs_amd import build_fast_execution_plan
    _flush(f"case: streamed ring wrap pinned={pinned}")
    rec = synth.speech_like(12_000_000, 19)
    host = torch.from_numpy(rec).pin_memory().numpy() if pinned else rec
    tasks = build_fast_execution_plan(rec.size)
    assert len(tasks) > 40
    a, fa = extractor.extract_chunks(torch.from_numpy(rec).cuda(), tasks)
    b, fb = extractor.extract_chunks_streamed(host, tasks, window_samples=250_000)
    torch.cuda.synchronize()
    assert np.array_equal(fa, fb)
    assert torch.equal(a, b)


@pytest.mark.parametrize("window", [250_000, 960_000])
def test_streamed_sparse_tasks_equal_resident(extractor, window):
    """Every third chunk task only (a plan with gaps, as speech regions
    give): batches of windows must not copy past their device half, and
    gaps larger than a window split batches."""
    import torch
    from scriptrs_amd import build_fast_execution_plan
    _flush(f"case: streamed sparse tasks window={window}")
    rec = synth.speech_like(12_000_000, 21)
    tasks = build_fast_execution_plan(rec.size)[::3]
    a, fa = extractor.extract_chunks(torch.from_numpy(rec).cuda(), tasks)
    b, fb = extractor.extract_chunks_streamed(rec, tasks, window_samples=window)
    torch.cuda.synchronize()
    assert np.array_equal(fa, fb)
    assert torch.equal(a, b)


def test_long_form_large_call(extractor):
    """A 36 M-sample long form in one call (175 chunk tasks, so every
    log-mel workgroup spans item boundaries): frame offsets exact for every
    chunk, values checked on chunks at the ends and around each quarter."""
    import torch
    from scriptrs_amd import build_fast_execution_plan
    _flush("case: long form 36M samples")
    rec = synth.speech_like(36_000_000, 21)
    tasks = build_fast_execution_plan(rec.size)
    assert sum(((t.audio_end - t.audio_start) // 160 + 1 + 15) // 16 for t in tasks) >= 4 * 4096
    dev = torch.from_numpy(rec).cuda()
    out, fo = extractor.extract_chunks(dev, tasks)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    starts = [t.audio_start for t in tasks]
    lens = [t.audio_end - t.audio_start for t in tasks]
    want_fo = np.concatenate([[0], np.cumsum([n // 160 + 1 for n in lens])])
    assert np.array_equal(fo, want_fo)
    n = len(tasks)
    pick = sorted(set([0, 1, n - 2, n - 1] + [i + d for i in (n // 4, n // 2, 3 * n // 4) for d in (-1, 0, 1)]))
    for i in pick:
        a = rec[starts[i]:starts[i] + lens[i]]
        got = out[128 * fo[i]:128 * fo[i + 1]].reshape(128, -1)
        assert_parity(got, oracle.extract(a), R.extract(a), R.f32_noise_envelope(a), what=f"chunk {i}")


def test_encoder_input_layout(extractor):
    """sfe_extract_chunks_padded writes what EncoderInputBuffer::copy_from_features
    builds (src/model.rs:241-278): per chunk [128, target_frames], the packed
    features in the first T columns, zeros after; bit-identical to the packed
    output of sfe_extract_chunks."""
    import torch
    from scriptrs_amd import build_fast_execution_plan
    _flush("case: encoder input layout")
    rec = synth.speech_like(1_300_000, 17)
    tasks = build_fast_execution_plan(rec.size)
    dev = torch.from_numpy(rec).cuda()
    packed, fo = extractor.extract_chunks(dev, tasks)
    enc, ff = extractor.extract_chunks_encoder_input(dev, tasks)
    torch.cuda.synchronize()
    packed = packed.cpu().numpy()
    enc = enc.cpu().numpy()
    assert enc.shape == (len(tasks), 128, 1501)
    assert np.array_equal(ff, np.diff(fo))
    for i in range(len(tasks)):
        T = int(ff[i])
        want = packed[128 * fo[i]:128 * fo[i + 1]].reshape(128, T)
        assert np.array_equal(enc[i, :, :T], want), i
        assert not enc[i, :, T:].any(), i


def test_encoder_input_layout_bf16(extractor):
    """The encoder layout in bf16: the packed bf16 output in the first T
    columns, zeros after."""
    import torch
    from scriptrs_amd import build_fast_execution_plan
    _flush("case: encoder input layout bf16")
    rec = synth.speech_like(700_000, 27)
    tasks = build_fast_execution_plan(rec.size)
    dev = torch.from_numpy(rec).cuda()
    packed, fo = extractor.extract_chunks(dev, tasks, dtype="bf16")
    enc, ff = extractor.extract_chunks_encoder_input(dev, tasks, dtype="bf16")
    torch.cuda.synchronize()
    assert enc.dtype == torch.bfloat16 and tuple(enc.shape) == (len(tasks), 128, 1501)
    for i in range(len(tasks)):
        T = int(ff[i])
        want = packed[128 * fo[i]:128 * fo[i + 1]].reshape(128, T)
        assert torch.equal(enc[i, :, :T], want), i
        assert not enc[i, :, T:].any(), i


def test_recording_at_4_byte_offset(extractor):
    """A device recording that starts 4 bytes past a 16-byte boundary (a
    slice of a larger buffer): bit-identical to the same samples at an
    aligned address, for the chunk path and a ragged batch."""
    import torch
    from scriptrs_amd import build_fast_execution_plan
    _flush("case: recording at a 4-byte offset")
    rec = synth.speech_like(900_001, 33)
    tasks = build_fast_execution_plan(rec.size - 1)
    big = torch.from_numpy(rec).cuda()
    off = big[1:]
    assert off.data_ptr() % 16 == 4
    aligned = off.clone()
    assert aligned.data_ptr() % 16 == 0
    a, fa = extractor.extract_chunks(aligned, tasks)
    b, fb = extractor.extract_chunks(off, tasks)
    offsets = np.array([0, 160_001, 400_003, 900_000], np.int64)
    c, fc = extractor.extract_batch(aligned, offsets)
    d, fd = extractor.extract_batch(off, offsets)
    torch.cuda.synchronize()
    assert np.array_equal(fa, fb) and torch.equal(a, b)
    assert np.array_equal(fc, fd) and torch.equal(c, d)


def test_encoder_input_rejects_overlong_chunk(extractor):
    import torch
    from scriptrs_amd import ChunkTask
    from scriptrs_amd.frontend import InvalidModelOutput
    _flush("case: encoder input overlong chunk")
    rec = synth.sinusoids(400_000, 3)
    dev = torch.from_numpy(rec).cuda()
    with pytest.raises(InvalidModelOutput, match="exceeded encoder target"):
        extractor.extract_chunks_encoder_input(dev, [ChunkTask(0, 300_000, 0, 0)])


def _pcm16(x):
    return np.clip(np.round(x.astype(np.float64) * 32767.0), -32768, 32767).astype(np.int16)


def test_pcm16_chunks_equal_f32_of_decoded(extractor):
    """16-bit PCM decoded in the kernel gives bit-identical features to the
    f32 path over the reference's decode (value as f32 / 32767.0)."""
    import torch
    from scriptrs_amd import build_fast_execution_plan
    _flush("case: pcm16 long form")
    pcm = _pcm16(synth.speech_like(1_500_000, 23))
    dec = pcm.astype(np.float32) / np.float32(32767.0)
    tasks = build_fast_execution_plan(pcm.size)
    a, fa = extractor.extract_chunks(torch.from_numpy(dec).cuda(), tasks)
    b, fb = extractor.extract_chunks_pcm(torch.from_numpy(pcm).cuda(), tasks)
    torch.cuda.synchronize()
    assert np.array_equal(fa, fb)
    assert torch.equal(a, b)


def test_pcm12_in_int16_chunks_equal_f32_of_decoded(extractor):
    """12-bit samples in int16 containers (scale 2047)."""
    import torch
    from scriptrs_amd import build_fast_execution_plan
    _flush("case: pcm12 in int16 long form")
    x = synth.speech_like(600_000, 29)
    pcm = np.clip(np.round(x * 2047.0), -2048, 2047).astype(np.int16)
    dec = pcm.astype(np.float32) / np.float32(2047.0)
    tasks = build_fast_execution_plan(pcm.size)
    a, fa = extractor.extract_chunks(torch.from_numpy(dec).cuda(), tasks)
    b, fb = extractor.extract_chunks_pcm(torch.from_numpy(pcm).cuda(), tasks, bits_per_sample=12)
    torch.cuda.synchronize()
    assert np.array_equal(fa, fb)
    assert torch.equal(a, b)


def test_pcm24_in_int32_equals_f32_of_decoded(extractor):
    import torch
    from scriptrs_amd import build_fast_execution_plan
    _flush("case: pcm24 in int32")
    x = synth.speech_like(700_000, 29).astype(np.float64)
    pcm = np.clip(np.round(x * 8388607.0), -8388608, 8388607).astype(np.int32)
    dec = pcm.astype(np.float32) / np.float32(8388607.0)
    tasks = build_fast_execution_plan(pcm.size)
    a, _ = extractor.extract_chunks(torch.from_numpy(dec).cuda(), tasks)
    b, _ = extractor.extract_chunks_pcm(torch.from_numpy(pcm).cuda(), tasks, bits_per_sample=24)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_pcm16_streamed_equals_resident(extractor):
    import torch
    from scriptrs_amd import build_fast_execution_plan
    _flush("case: pcm16 streamed")
    pcm = _pcm16(synth.speech_like(3_000_000, 31))
    tasks = build_fast_execution_plan(pcm.size)
    a, fa = extractor.extract_chunks_pcm(torch.from_numpy(pcm).cuda(), tasks)
    b, fb = extractor.extract_chunks_streamed(pcm, tasks, window_samples=960_000)
    torch.cuda.synchronize()
    assert np.array_equal(fa, fb)
    assert torch.equal(a, b)


def test_calls_on_two_streams_and_repeated_plans(extractor):
    """Back-to-back calls on different streams share the context's item table
    and raw scratch: the second call is ordered after the first on the GPU.
    A repeated plan reuses the uploaded item table and gives identical output."""
    import torch
    from scriptrs_amd import TaskTable, build_fast_execution_plan
    _flush("case: two streams, repeated plan")
    ra = synth.speech_like(1_200_000, 41)
    rb = synth.speech_like(900_000, 43)
    ta = TaskTable(build_fast_execution_plan(ra.size))
    tb = TaskTable(build_fast_execution_plan(rb.size))
    da, db = torch.from_numpy(ra).cuda(), torch.from_numpy(rb).cuda()
    want_a, _ = extractor.extract_chunks(da, ta)
    want_b, _ = extractor.extract_chunks(db, tb)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = []
    for _ in range(3):
        oa, _ = extractor.extract_chunks(da, ta, stream=s1)
        ob, _ = extractor.extract_chunks(db, tb, stream=s2)
        oa2, _ = extractor.extract_chunks(da, ta, stream=s2)
        outs.append((oa, ob, oa2))
    torch.cuda.synchronize()
    for oa, ob, oa2 in outs:
        assert torch.equal(oa, want_a)
        assert torch.equal(ob, want_b)
        assert torch.equal(oa2, want_a)


def test_call_after_the_previous_calls_stream_was_destroyed(extractor):
    """A caller may destroy a stream right after a call on it (per-request
    streams).  The next call, on another stream, is still ordered after the
    first (they share the context's item table and raw scratch) and nothing
    is enqueued on the destroyed stream."""
    import ctypes
    import torch
    from scriptrs_amd import TaskTable, build_fast_execution_plan
    _flush("case: previous call's stream destroyed")
    hip = ctypes.CDLL("libamdhip64.so.7")  # the runtime torch has loaded
    ra = synth.speech_like(1_200_000, 44)
    rb = synth.speech_like(700_000, 45)
    ta = TaskTable(build_fast_execution_plan(ra.size))
    tb = TaskTable(build_fast_execution_plan(rb.size))
    da, db = torch.from_numpy(ra).cuda(), torch.from_numpy(rb).cuda()
    want_a, _ = extractor.extract_chunks(da, ta)
    want_b, _ = extractor.extract_chunks(db, tb)
    torch.cuda.synchronize()
    for rep in range(3):
        s = ctypes.c_void_p()
        assert hip.hipStreamCreate(ctypes.byref(s)) == 0
        oa, _ = extractor.extract_chunks(da, ta, stream=s.value)
        assert hip.hipStreamDestroy(s) == 0
        ob, _ = extractor.extract_chunks(db, tb)  # torch's current stream
        torch.cuda.synchronize()
        assert torch.equal(oa, want_a), rep
        assert torch.equal(ob, want_b), rep


@pytest.mark.parametrize("n", [327_680, 327_840, 480_000])
def test_items_longer_than_register_budget(extractor, n):
    """T > 2048 frames takes the normalisation kernel's streaming path
    (327,680 samples -> T = 2049; 480,000 -> T = 3001)."""
    _flush(f"case: long item {n}")
    a = synth.sinusoids(n, 300 + n % 97)
    got = extractor.extract(a)
    want = oracle.extract(a).T
    assert got.shape == (n // 160 + 1, 128)
    assert_parity(got, want, R.extract(a).T, R.f32_noise_envelope(a).T, what=f"len {n}")


def test_config2_full_dense_batch(extractor):
    """BASELINE config 2 at full size: 64 x 15 s clips in one call; frame
    counts exact, every clip's rows normalised (mean ~ 0 as the reference's
    own test, src/frontend.rs:292-300), every clip checked element-wise."""
    import torch
    _flush("case: config 2 full")
    x = synth.dense_batch(64, 240_000, 1000)
    dev = torch.from_numpy(x.reshape(-1)).cuda()
    off = np.arange(65, dtype=np.int64) * 240_000
    out, fo = extractor.extract_batch(dev, off)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    assert list(np.diff(fo)) == [1501] * 64
    feats = out.reshape(64, 128, 1501)
    assert np.abs(feats.mean(axis=2)).max() < 1e-4
    for i in range(64):
        assert_parity(feats[i], oracle.extract(x[i]), R.extract(x[i]), R.f32_noise_envelope(x[i]), what=f"clip {i}")


def test_config4_full_ragged_batch(extractor):
    """BASELINE config 4 at full size: 256 clips of 1-20 s in one flat buffer;
    frame counts exact against the oracle, and every clip element-wise
    against it at the plain bar, widened only near the guard (the f32 FFT
    noise the envelope models)."""
    import torch
    _flush("case: config 4 full")
    flat, off = synth.ragged_batch(256, 4)
    dev = torch.from_numpy(flat).cuda()
    out, fo = extractor.extract_batch(dev, off)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    want, wfo = oracle.extract_spans(flat, off[:-1], np.diff(off), 4)
    assert np.array_equal(fo, wfo)
    err = np.abs(out - want)
    assert np.mean(err <= 1e-4 + 1e-3 * np.abs(want)) > 0.999
    for i in range(256):
        a = flat[off[i]:off[i + 1]]
        got = out[128 * fo[i]:128 * fo[i + 1]].reshape(128, -1)
        assert_parity(got, want[128 * fo[i]:128 * fo[i + 1]].reshape(128, -1), R.extract(a), R.f32_noise_envelope(a),
                      what=f"clip {i}")


def test_config3_full(extractor):
    """BASELINE config 3 at full size (57.6M samples, 280 chunk tasks): frame
    offsets exact, each chunk's rows normalised (mean ~ 0, the reference's
    invariant, src/frontend.rs:292-300), and every chunk element-wise against
    the oracle."""
    import torch
    from scriptrs_amd import TaskTable, build_fast_execution_plan
    _flush("case: config 3 full")
    rec = synth.speech_like(57_600_000, 3)
    tasks = TaskTable(build_fast_execution_plan(rec.size))
    assert tasks.n == 280 and tasks.frame_offsets[-1] == 418_312
    out, fo = extractor.extract_chunks(torch.from_numpy(rec).cuda(), tasks)
    torch.cuda.synchronize()
    assert np.array_equal(fo, tasks.frame_offsets)
    out = out.cpu().numpy()
    for i in range(tasks.n):
        rows = out[128 * fo[i]:128 * fo[i + 1]].reshape(128, -1)
        assert np.abs(rows.mean(axis=1)).max() < 1e-4, i
    starts = tasks.array[:, 0]
    lens = tasks.array[:, 1] - tasks.array[:, 0]
    want, wfo = oracle.extract_spans(rec, starts, lens, 8)
    assert np.array_equal(wfo, fo)
    for i in range(tasks.n):
        a = rec[int(starts[i]):int(starts[i] + lens[i])]
        sl = slice(128 * int(fo[i]), 128 * int(fo[i + 1]))
        got = out[sl].reshape(128, -1)
        assert_parity(got, want[sl].reshape(128, -1), R.extract(a), R.f32_noise_envelope(a), what=f"chunk {i}")


def test_long_form_past_2gib(extractor):
    """A 12 h recording in one resident call: 2.6 GB of features and 2.3 GB
    of raw log-mel, so chunks past the first 2 GiB of either are addressed
    with 64-bit offsets.  Frame offsets exact, every chunk's rows normalised,
    24 chunks at the start, middle and end bitwise equal to a separate call
    of just those tasks, and chunks past 2 GiB of output against the oracle.  (The hour is
    repeated with a different gain each time: synthesising 12 h takes
    minutes.)"""
    import torch
    from scriptrs_amd import TaskTable, build_fast_execution_plan
    _flush("case: 12 h resident, past 2 GiB")
    hour = synth.speech_like(57_600_000, 3)
    rec = np.concatenate([hour * np.float32(1.0 + 0.05 * k) for k in range(12)])
    del hour
    plan = build_fast_execution_plan(rec.size)
    tasks = TaskTable(plan)
    dev = torch.from_numpy(rec).cuda()
    out, fo = extractor.extract_chunks(dev, tasks)
    torch.cuda.synchronize()
    assert np.array_equal(fo, tasks.frame_offsets)
    assert 128 * 4 * int(fo[-1]) > 2**31 + 2**28
    out = out.cpu().numpy()

    def same_as_alone(first, count):
        t2 = TaskTable(plan[first:first + count])
        o2, _ = extractor.extract_chunks(dev, t2)
        torch.cuda.synchronize()
        o2 = o2.cpu().numpy()
        seg = out[128 * int(fo[first]):128 * int(fo[first + count])]
        bad = np.flatnonzero(seg.view(np.int32) != o2.view(np.int32))
        if bad.size:
            k = int(np.searchsorted(fo[first:first + count + 1] - fo[first], bad[0] // 128, side="right")) - 1
            print(f"tasks {first}+{count}: {bad.size} differ, first at element {int(bad[0])} (task {first + k}),"
                  f" max |diff| {float(np.abs(seg[bad] - o2[bad]).max()):.3g}", flush=True)
        return bad.size == 0

    # (24 tasks: calls of at most 16 items normalise with 8-wave workgroups,
    # whose sums group the frames differently)
    ok = [same_as_alone(0, 24), same_as_alone(tasks.n // 2, 24), same_as_alone(tasks.n - 24, 24)]
    assert all(ok), ok
    for i in range(tasks.n):
        rows = out[128 * fo[i]:128 * fo[i + 1]].reshape(128, -1)
        assert np.abs(rows.mean(axis=1)).max() < 1e-4, i
    past = [i for i in range(tasks.n) if 128 * 4 * int(fo[i]) >= 2**31]
    for i in (past[0], past[len(past) // 2], tasks.n - 1):
        s0, s1 = (int(v) for v in tasks.array[i, :2])
        a = rec[s0:s1]
        got = out[128 * int(fo[i]):128 * int(fo[i + 1])].reshape(128, -1)
        assert_parity(got, oracle.extract(a), R.extract(a), R.f32_noise_envelope(a), what=f"chunk {i}")


@pytest.mark.parametrize("sr,pre", [(8000, 0.97), (11025, 0.97), (22050, 0.97), (44100, 0.97), (48000, 0.97),
                                    (3500, 0.97), (96000, 0.97), (107000, 0.97), (16000, 0.0), (16000, 0.5)])
def test_other_sample_rates_and_preemphasis(sr, pre):
    """A TranscriptionConfig with another sample rate (the mel filterbank's
    band edges; at 8, 11.025, 44.1 and 48 kHz the filters need the wider mel
    schedule, at 22.05 kHz the default one fits) or another preemphasis
    coefficient (src/config.rs:11-27, src/frontend.rs:150-223; 3.5 and 107 kHz
    are the ends of the range sfe_create takes), against the
    oracle under the same config: one 10 s clip (extract, 4-wave launch) and
    64 clips of 125,000 samples (extract_batch, the 12-wave launch).  Filters
    that fall between FFT bins (the 11 and 13 lowest at 44.1 and 48 kHz)
    give constant rows, bitwise equal to the oracle's replay of the
    reference's sequential f32 sums."""
    import torch
    from scriptrs_amd import ParakeetFeatureExtractor, TranscriptionConfig
    _flush(f"case: sample rate {sr}, preemphasis {pre}")
    ext = ParakeetFeatureExtractor(TranscriptionConfig(sample_rate=sr, preemphasis=pre))
    empty = ~oracle.mel_filterbank(512, 128, sr).any(axis=1)

    def check(got, a, what):
        want = oracle.extract_cfg(a, sr, pre)
        assert np.array_equal(got[empty].view(np.int32), want[empty].view(np.int32)), what
        assert_parity(got[~empty], want[~empty], R.extract(a, sr=sr, preemph=pre)[~empty],
                      R.f32_noise_envelope(a, sr=sr, preemph=pre)[~empty], what=what)

    try:
        a = synth.speech_like(10 * sr, 9)
        check(np.ascontiguousarray(ext.extract(a).T), a, f"{sr} Hz clip")
        x = synth.speech_like(64 * 125_000, 10)
        off = np.arange(65, dtype=np.int64) * 125_000
        out, fo = ext.extract_batch(torch.from_numpy(x).cuda(), off)
        torch.cuda.synchronize()
        out = out.cpu().numpy()
        for i in (0, 31, 63):
            check(out[128 * fo[i]:128 * fo[i + 1]].reshape(128, -1), x[off[i]:off[i + 1]], f"{sr} Hz batch clip {i}")
    finally:
        ext.close()


@pytest.mark.parametrize("seed", [101, 202, 303])
def test_random_ragged_batch(extractor, seed):
    """48 clips of random lengths from 1 sample to 25 s (a few tiny ones
    forced), each checked against the oracle."""
    import torch
    _flush(f"case: random ragged batch seed {seed}")
    rng = np.random.default_rng(seed)
    lens = rng.integers(1, 400_000, 48)
    lens[:4] = [1, 2, 159, 161]
    rng.shuffle(lens)
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    flat = synth.sinusoids(int(off[-1]), seed)
    out, fo = extractor.extract_batch(torch.from_numpy(flat).cuda(), off)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    assert np.array_equal(fo, np.concatenate([[0], np.cumsum(lens // 160 + 1)]))
    for i in range(len(lens)):
        a = flat[off[i]:off[i + 1]]
        got = out[128 * fo[i]:128 * fo[i + 1]].reshape(128, -1)
        assert_parity(got, oracle.extract(a), R.extract(a), R.f32_noise_envelope(a), what=f"clip {i} len {lens[i]}")


@pytest.mark.parametrize("seed", [404, 505])
def test_random_chunk_tables(extractor, seed):
    """Chunk tasks at random, unsorted and overlapping positions of one
    recording (the resident path takes any order), each checked against the
    oracle on its own span."""
    import torch
    from scriptrs_amd import ChunkTask
    _flush(f"case: random chunk table seed {seed}")
    rng = np.random.default_rng(seed)
    rec = synth.speech_like(3_000_000, seed)
    tasks = []
    for _ in range(40):
        n = int(rng.integers(1, 240_001))
        s = int(rng.integers(0, rec.size - n + 1))
        tasks.append(ChunkTask(s, s + n, s, 0))
    out, fo = extractor.extract_chunks(torch.from_numpy(rec).cuda(), tasks)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    for i, t in enumerate(tasks):
        a = rec[t.audio_start:t.audio_end]
        got = out[128 * fo[i]:128 * fo[i + 1]].reshape(128, -1)
        assert_parity(got, oracle.extract(a), R.extract(a), R.f32_noise_envelope(a), what=f"task {i}")


def test_config5_full_streamed_equals_resident(extractor):
    """Config 5 at full size: the 8 h recording (460.8 M samples, 2,236
    chunk tasks) streamed from pinned host memory in 60 s windows is
    bit-identical to the same plan featurized from HBM, in f32 and bf16, and
    the bf16 output equals the f32 output rounded to bf16 (the resident path
    is checked against the oracle by the other tests)."""
    import torch
    from scriptrs_amd import TaskTable, build_fast_execution_plan
    _flush("case: config 5 full size, streamed vs resident")
    rec = synth.speech_like(460_800_000, 5)
    tasks = TaskTable(build_fast_execution_plan(rec.size))
    assert tasks.n == 2236 and int(tasks.frame_offsets[-1]) == 3_347_116
    host = torch.from_numpy(rec).pin_memory().numpy()
    dev = torch.from_numpy(rec).cuda()
    a32 = None
    for dtype in ("f32", "bf16"):
        a, fa = extractor.extract_chunks(dev, tasks, dtype=dtype)
        b, fb = extractor.extract_chunks_streamed(host, tasks, window_samples=960_000, dtype=dtype)
        torch.cuda.synchronize()
        assert np.array_equal(fa, fb)
        assert torch.equal(a, b), dtype
        if dtype == "f32":
            a32 = a
        else:
            # the bf16 output at full size is the f32 output rounded to nearest even
            assert torch.equal(a32.to(torch.bfloat16), b)
        del a, b


def test_contexts_on_concurrent_host_threads():
    """One context per host thread (the reference's extractor is !Sync, one
    per worker: src/long_form.rs:288-295): four threads, each with its own
    extractor and stream, run chunk calls at the same time; every result is
    bit-identical to a single-threaded run."""
    import threading
    import torch
    from scriptrs_amd import ParakeetFeatureExtractor, build_fast_execution_plan
    _flush("case: four host threads, one context each")
    rec = synth.speech_like(2_000_000, 37)
    tasks = build_fast_execution_plan(rec.size)
    dev = torch.from_numpy(rec).cuda()
    ref_ext = ParakeetFeatureExtractor()
    want, wfo = ref_ext.extract_chunks(dev, tasks)
    torch.cuda.synchronize()
    ref_ext.close()
    results, errors = {}, []

    def work(k):
        try:
            ext = ParakeetFeatureExtractor()
            stream = torch.cuda.Stream()
            for r in range(5):
                out, fo = ext.extract_chunks(dev, tasks, stream=stream)
                stream.synchronize()
                results[(k, r)] = (out.clone(), fo)
            ext.close()
        except Exception as e:  # surfaced below
            errors.append(repr(e))

    th = [threading.Thread(target=work, args=(k,)) for k in range(4)]
    for t in th:
        t.start()
    for t in th:
        t.join(timeout=120)
    assert not errors, errors
    assert len(results) == 20
    for (k, r), (out, fo) in results.items():
        assert np.array_equal(fo, wfo), (k, r)
        assert torch.equal(out, want), (k, r)


def test_streamed_window_far_longer_than_recording(extractor):
    """A window of 2^40 samples is clamped to the recording: the device ring
    and batch sizes stay small, and the result equals the resident path."""
    import torch
    from scriptrs_amd import build_fast_execution_plan
    _flush("case: streamed, window 2^40 samples")
    rec = synth.speech_like(700_000, 13)
    tasks = build_fast_execution_plan(rec.size)
    a, fa = extractor.extract_chunks(torch.from_numpy(rec).cuda(), tasks)
    b, fb = extractor.extract_chunks_streamed(rec, tasks, window_samples=1 << 40)
    torch.cuda.synchronize()
    assert np.array_equal(fa, fb)
    assert torch.equal(a, b)


@pytest.mark.parametrize("seed", [606, 707])
def test_shared_frames_equal_own_frames(extractor, seed):
    """Frames that overlapping hop-aligned tasks share are computed once
    (the default); the output is bitwise what every task computing its own
    frames gives, for nested, duplicated and partly overlapping tasks, in f32,
    bf16 and the padded encoder-input layout, and matches the oracle."""
    import torch
    from scriptrs_amd import ChunkTask
    _flush(f"case: shared frames seed {seed}")
    rng = np.random.default_rng(seed)
    rec = synth.speech_like(3_000_000, seed)
    tasks = []
    for _ in range(40):
        n = int(rng.integers(1, 240_001))
        s = 160 * int(rng.integers(0, (rec.size - n) // 160 + 1))
        tasks.append(ChunkTask(s, s + n, s, 0))
    tasks += tasks[:4] + [ChunkTask(tasks[5].audio_start + 3200, tasks[5].audio_start + 3200 + 50_000, 0, 0)]
    dev = torch.from_numpy(rec).cuda()
    try:
        got = {}
        for share in (True, False):
            extractor.set_frame_sharing(share)
            got[share] = [extractor.extract_chunks(dev, tasks, dtype=d)[0] for d in ("f32", "bf16")]
            got[share].append(extractor.extract_chunks_encoder_input(dev, tasks, target_frames=1501)[0])
        torch.cuda.synchronize()
    finally:
        extractor.set_frame_sharing(True)
    for a, b in zip(got[True], got[False]):
        assert torch.equal(a, b)
    out = got[True][0].cpu().numpy()
    fo = np.concatenate([[0], np.cumsum([(t.audio_end - t.audio_start) // 160 + 1 for t in tasks])])
    for i, t in enumerate(tasks[:12]):
        a = rec[t.audio_start:t.audio_end]
        g = out[128 * fo[i]:128 * fo[i + 1]].reshape(128, -1)
        assert_parity(g, oracle.extract(a), R.extract(a), R.f32_noise_envelope(a), what=f"task {i}")


@pytest.mark.parametrize("window", [240_000, 700_000])
def test_streamed_shared_frames_equal_own_frames(extractor, window):
    """The streamed path shares frames among the overlapping tasks of one
    batch of windows: random hop-aligned and unaligned tasks (ordered by
    start, as the streamed entry point takes them, with duplicates and a
    nested one) streamed with sharing on, streamed with sharing off and
    featurized from HBM without sharing are bitwise the same."""
    import torch
    from scriptrs_amd import ChunkTask
    _flush(f"case: streamed shared frames window={window}")
    rng = np.random.default_rng(808)
    rec = synth.speech_like(6_000_000, 808)
    tasks = []
    for _ in range(60):
        n = int(rng.integers(1, 240_001))
        s = int(rng.integers(0, (rec.size - n) // 160 + 1)) * 160 + int(rng.integers(0, 2)) * int(rng.integers(0, 160))
        s = min(s, rec.size - n)
        tasks.append(ChunkTask(s, s + n, s, 0))
    tasks += tasks[:3] + [ChunkTask(tasks[7].audio_start + 1600, tasks[7].audio_start + 1600 + 30_000, 0, 0)]
    tasks.sort(key=lambda t: t.audio_start)
    try:
        got = {}
        for share in (True, False):
            extractor.set_frame_sharing(share)
            got[share] = extractor.extract_chunks_streamed(rec, tasks, window_samples=window)
        own, fo = extractor.extract_chunks(torch.from_numpy(rec).cuda(), tasks)
        torch.cuda.synchronize()
    finally:
        extractor.set_frame_sharing(True)
    for share in (True, False):
        assert np.array_equal(got[share][1], fo)
        assert torch.equal(got[share][0], own), share


def test_config3_shared_frames_equal_own_frames(extractor):
    """Config 3 at full size: the 280 chunks with their ~2 s overlaps
    computed once give bitwise the output of every chunk on its own."""
    import torch
    from scriptrs_amd import TaskTable, build_fast_execution_plan
    _flush("case: config 3 shared frames")
    rec = synth.speech_like(57_600_000, 3)
    tasks = TaskTable(build_fast_execution_plan(rec.size))
    dev = torch.from_numpy(rec).cuda()
    try:
        a, _ = extractor.extract_chunks(dev, tasks)
        extractor.set_frame_sharing(False)
        b, _ = extractor.extract_chunks(dev, tasks)
        torch.cuda.synchronize()
    finally:
        extractor.set_frame_sharing(True)
    assert torch.equal(a, b)


def test_norm_class_does_not_change_results(extractor):
    """The normalisation kernel's register class follows the batch's longest
    item (16, 24 or 24 + 8 rounds of 64 frames in registers, or the
    streaming path past 2048 frames); every class sums the same rounds in the
    same groups, so 17 clips give bitwise the same features whichever longer
    clip joins their batch (17 clips: past the 8-wave few-item variant)."""
    import torch
    rng = np.random.default_rng(77)
    lens = [int(v) for v in rng.integers(16_000, 160_000, 17)]  # at most 1000 frames
    base = None
    for extra in (None, 192_000, 288_000, 400_000):  # 1201, 1801, 2501 frames
        _flush(f"case: norm class, extra clip {extra}")
        ls = lens + ([extra] if extra else [])
        off = np.concatenate([[0], np.cumsum(ls)]).astype(np.int64)
        flat = synth.speech_like(int(off[-1]), 12)
        flat[:off[17]] = synth.speech_like(int(off[17]), 13)  # the 17 clips' samples equal in every batch
        out, fo = extractor.extract_batch(torch.from_numpy(flat).cuda(), off)
        torch.cuda.synchronize()
        got = out[:128 * int(fo[17])].cpu()
        if base is None:
            base = got
        else:
            assert torch.equal(got, base), extra


@pytest.mark.parametrize("frames", [(700, 1024), (1100, 1536)])
def test_batch_split_into_calls_is_bitwise_the_same(extractor, frames):
    """240 clips in one call (1,920 16-feature slabs of normalisation, more
    than the GPU holds workgroups at once) and the same clips in four calls
    of 60 give bitwise the same features: each call's longest clip is in the
    same register class (16 or 24 rounds of 64 frames), and the sums run in
    the same groups whatever the batch.  Clips of the full batch are also
    checked against the oracle."""
    import torch
    lo, hi = frames
    rng = np.random.default_rng(hi)
    n, part = 240, 60  # 1920 slabs in one call: more than 4 workgroups on each of 256 CUs
    T = rng.integers(lo, hi + 1, n)
    T[::part] = hi
    lens = (T - 1) * 160 + rng.integers(0, 160, n)
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    flat = synth.speech_like(int(off[-1]), 31)
    dev = torch.from_numpy(flat).cuda()
    _flush(f"case: batch split into calls, {n} clips of {lo}-{hi} frames")
    whole, fo = extractor.extract_batch(dev, off)
    torch.cuda.synchronize()
    whole = whole.cpu()
    for p0 in range(0, n, part):
        o = off[p0:p0 + part + 1]
        got, _ = extractor.extract_batch(dev[int(o[0]):], o - o[0])
        torch.cuda.synchronize()
        assert torch.equal(got.cpu(), whole[128 * int(fo[p0]):128 * int(fo[p0 + part])]), p0
    for i in (0, 1, n // 2, n - 1):
        x = flat[off[i]:off[i + 1]]
        got = whole[128 * int(fo[i]):128 * int(fo[i + 1])].numpy().reshape(128, -1)
        assert_parity(got, oracle.extract(x), R.extract(x), R.f32_noise_envelope(x), what=f"clip {i}")


def test_random_tables_shared_equal_own_bitwise(extractor):
    """150 random task tables over one 500 s recording (hop-aligned,
    arbitrary, clustered and duplicated starts; lengths 1 sample to 15 s):
    sharing on and off, and the allocation-free entry point, give bitwise the
    same features (compared as bits: 1-frame tasks are NaN, as in the
    reference, src/frontend.rs:225-241)."""
    import torch
    from scriptrs_amd import TaskTable
    _flush("case: 150 random tables, shared vs own")
    rng = np.random.default_rng(2024)
    rec = synth.speech_like(8_000_000, 5)
    dev = torch.from_numpy(rec).cuda()

    def bits_equal(x, y):
        return torch.equal(x.view(torch.int32), y.view(torch.int32))

    try:
        for case in range(150):
            kind = case % 4
            n = int(rng.integers(1, 300))
            tasks = []
            for _ in range(n):
                L = int(rng.integers(1, 240_001)) if rng.random() < 0.9 else int(rng.integers(1, 2000))
                if kind == 0:
                    s = 160 * int(rng.integers(0, (rec.size - L) // 160 + 1))
                elif kind == 1:
                    s = int(rng.integers(0, rec.size - L + 1))
                elif kind == 2:
                    s = min(rec.size - L, 160 * 16000 * int(rng.integers(0, 20)) + 160 * int(rng.integers(0, 4000)))
                else:
                    s = min(rec.size - L, 160 * 800 * int(rng.integers(0, 50)))
                tasks.append((s, s + L, s, 0))
            if kind == 3:
                tasks += tasks[: n // 2]
            tt = TaskTable(np.array(tasks, np.int64))
            extractor.set_frame_sharing(True)
            a, fa = extractor.extract_chunks(dev, tt)
            c, fc = extractor.extract_chunks_noalloc(dev, tt) if int(tt.frame_offsets[-1]) < 100_000 else (a, fa)
            extractor.set_frame_sharing(False)
            b, fb = extractor.extract_chunks(dev, tt)
            torch.cuda.synchronize()
            assert np.array_equal(fa, fb) and np.array_equal(fa, fc), case
            assert bits_equal(a, b), f"case {case} kind {kind}: shared != own"
            assert bits_equal(a, c), f"case {case} kind {kind}: noalloc != extract_chunks"
    finally:
        extractor.set_frame_sharing(True)
