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
