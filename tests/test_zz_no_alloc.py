"""GPU: the allocation-free entry point sfe_extract_chunks_noalloc, called
through the C ABI, against sfe_extract_chunks (same kernels, so the results
must be bit-identical): two calls in a row, the second smaller, plus the
limits it rejects."""
import ctypes

import numpy as np
import pytest

from scriptrs_amd import ChunkTask, TaskTable, _lib, build_fast_execution_plan, synth

pytestmark = pytest.mark.gpu


def _flush(msg):
    print(msg, flush=True)


def _noalloc(ctx, dev, tt, out, dtype_code, stream):
    fo = np.zeros(tt.n + 1, np.int64)
    rc = _lib.lib().sfe_extract_chunks_noalloc(
        ctx, ctypes.c_void_p(dev.data_ptr()), dev.numel(), tt.ptr, tt.n, dtype_code, ctypes.c_void_p(out.data_ptr()),
        fo.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)), ctypes.c_void_p(stream.cuda_stream))
    return rc, fo


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_noalloc_equals_extract_chunks_twice_second_smaller(extractor, dtype):
    import torch
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    code = _lib.SFE_F32 if dtype == "f32" else _lib.SFE_BF16
    stream = torch.cuda.current_stream()
    ctx = extractor._handle()
    # first call: a 90 s long-form recording, 7 overlapping chunk tasks
    rec = synth.speech_like(1_440_000, 21)
    big = TaskTable(build_fast_execution_plan(rec.size))
    # second call: 5 ragged clips, fewer tasks and fewer frames than the first
    flat, off = synth.ragged_batch(5, 22)
    small = TaskTable([ChunkTask(int(off[i]), int(off[i + 1]), int(off[i]), 0) for i in range(5)])
    for name, x, tt in (("long form 90 s", rec, big), ("5 ragged clips", flat, small)):
        _flush(f"case: noalloc {dtype} {name} ({tt.n} tasks)")
        dev = torch.from_numpy(x).cuda()
        want, wfo = extractor.extract_chunks(dev, tt, dtype=dtype, stream=stream)
        got = torch.full_like(want, float("nan"))
        rc, fo = _noalloc(ctx, dev, tt, got, code, stream)
        assert rc == _lib.SFE_OK, _lib.last_error()
        torch.cuda.synchronize()
        assert np.array_equal(fo, wfo)
        assert torch.equal(got, want), name
    assert big.n > small.n and int(big.frame_offsets[-1]) > int(small.frame_offsets[-1])


def test_noalloc_rejects_calls_past_its_limits(extractor):
    import torch
    _flush("case: noalloc limits")
    stream = torch.cuda.current_stream()
    ctx = extractor._handle()
    # 30 min of audio in 15 s chunks needs more raw scratch than the 64 MiB array
    n = 28_800_000
    dev = torch.zeros(n, dtype=torch.float32, device="cuda")
    tt = TaskTable(build_fast_execution_plan(n))
    out = torch.empty(int(tt.frame_offsets[-1]) * 128, dtype=torch.float32, device="cuda")
    rc, _ = _noalloc(ctx, dev, tt, out, _lib.SFE_F32, stream)
    assert rc == _lib.SFE_INVALID_ARG and "scratch" in _lib.last_error()
    # more tasks than its item table holds
    many = TaskTable(np.array([[i, i + 160, i, 0] for i in range(4097)], np.int64))
    rc, _ = _noalloc(ctx, dev, many, out, _lib.SFE_F32, stream)
    assert rc == _lib.SFE_INVALID_ARG and "4096" in _lib.last_error()
    torch.cuda.synchronize()


def test_noalloc_shared_plan_at_its_raw_limit(extractor):
    """1024 heavily overlapping tasks (starts 5 hops apart, 126 frames each):
    their own regions fill the 64 MiB raw array exactly, and with sharing on
    the plan has about 3 log-mel entries per task.  Both plans must give
    sfe_extract_chunks' output bit for bit."""
    import torch
    stream = torch.cuda.current_stream()
    ctx = extractor._handle()
    n_tasks, step, length = 1024, 800, 20_000
    rec = synth.speech_like((n_tasks - 1) * step + length, 31)
    tt = TaskTable(np.array([[i * step, i * step + length, i * step, 0] for i in range(n_tasks)], np.int64))
    dev = torch.from_numpy(rec).cuda()
    outs = []
    try:
        for share in (True, False):
            _flush(f"case: noalloc 1024 overlapping tasks, sharing {share}")
            extractor.set_frame_sharing(share)
            want, wfo = extractor.extract_chunks(dev, tt, dtype="f32", stream=stream)
            got = torch.full_like(want, float("nan"))
            rc, fo = _noalloc(ctx, dev, tt, got, _lib.SFE_F32, stream)
            assert rc == _lib.SFE_OK, _lib.last_error()
            torch.cuda.synchronize()
            assert np.array_equal(fo, wfo)
            assert torch.equal(got, want), share
            outs.append(got)
    finally:
        extractor.set_frame_sharing(True)
    assert torch.equal(outs[0], outs[1])


def test_noalloc_allocates_nothing_on_a_fresh_context():
    """The contract itself: after sfe_create, calls of the allocation-free
    entry point make no device or pinned host allocation (the library counts
    every hipMalloc and hipHostMalloc it makes), on a fresh context, over
    calls of different sizes."""
    import torch
    from scriptrs_amd import ParakeetFeatureExtractor
    _flush("case: noalloc allocation count on a fresh context")
    L = _lib.lib()
    stream = torch.cuda.current_stream()
    rec = synth.speech_like(1_440_000, 41)
    big = TaskTable(build_fast_execution_plan(rec.size))
    small = TaskTable([ChunkTask(0, 300_000, 0, 0), ChunkTask(1000, 2000, 1000, 0)])
    dev = torch.from_numpy(rec).cuda()
    out = torch.empty(int(big.frame_offsets[-1]) * 128, dtype=torch.float32, device="cuda")
    ext = ParakeetFeatureExtractor()
    try:
        ctx = ext._handle()
        before = L.sfe_debug_allocation_count()
        for tt in (big, small, big):
            rc, _ = _noalloc(ctx, dev, tt, out, _lib.SFE_F32, stream)
            assert rc == _lib.SFE_OK, _lib.last_error()
        torch.cuda.synchronize()
        assert L.sfe_debug_allocation_count() == before
        # the counter does count: a resident call on the same fresh context
        # grows its item table and raw scratch
        ext.extract_chunks(dev, big, stream=stream, out=out)
        torch.cuda.synchronize()
        assert L.sfe_debug_allocation_count() > before
    finally:
        ext.close()


def test_noalloc_rejects_graph_capture(extractor):
    """Its pinned item table is rewritten by every call, so a captured upload
    would replay another call's table: under capture it returns
    SFE_INVALID_ARG and enqueues nothing."""
    import torch
    _flush("case: noalloc under stream capture")
    ctx = extractor._handle()
    rec = synth.speech_like(240_000, 42)
    tt = TaskTable([ChunkTask(0, rec.size, 0, 0)])
    dev = torch.from_numpy(rec).cuda()
    out = torch.empty(int(tt.frame_offsets[-1]) * 128, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        g.capture_begin(capture_error_mode="relaxed")
        try:
            rc, _ = _noalloc(ctx, dev, tt, out, _lib.SFE_F32, s)
        finally:
            g.capture_end()
    assert rc == _lib.SFE_INVALID_ARG and "captured" in _lib.last_error()
    torch.cuda.synchronize()


def test_noalloc_calls_from_two_contexts_on_two_streams_do_not_race(extractor):
    """Two contexts share the device's static scratch; calls issued back to
    back on two streams, with no host synchronisation between them, must
    each give sfe_extract_chunks' output bit for bit."""
    import torch
    from scriptrs_amd import ParakeetFeatureExtractor
    _flush("case: noalloc two contexts, two streams")
    recs = [synth.speech_like(1_440_000, 51), synth.speech_like(960_000, 52)]
    tts = [TaskTable(build_fast_execution_plan(r.size)) for r in recs]
    devs = [torch.from_numpy(r).cuda() for r in recs]
    wants = [extractor.extract_chunks(d, t, dtype="f32")[0] for d, t in zip(devs, tts)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    exts = [ParakeetFeatureExtractor(), ParakeetFeatureExtractor()]
    try:
        outs = [[torch.full_like(w, float("nan")) for _ in range(3)] for w in wants]
        for rep in range(3):
            for k in (0, 1):
                rc, _ = _noalloc(exts[k]._handle(), devs[k], tts[k], outs[k][rep], _lib.SFE_F32, streams[k])
                assert rc == _lib.SFE_OK, _lib.last_error()
        torch.cuda.synchronize()
        for k in (0, 1):
            for rep in range(3):
                assert torch.equal(outs[k][rep], wants[k]), (k, rep)
    finally:
        for e in exts:
            e.close()
