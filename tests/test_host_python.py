"""Python host helpers without a GPU: the task table in the C ABI layout,
the sample-format mapping, and argument checks that run before any device
work."""
import ctypes

import numpy as np
import pytest

from scriptrs_amd import (ChunkTask, InvalidModelOutput, SileroVadFramer, TaskTable, build_fast_execution_plan,
                          vad_num_windows)
from scriptrs_amd import _lib
from scriptrs_amd.frontend import _dtype_code, _pcm_format


def test_task_table_matches_the_c_layout():
    tasks = build_fast_execution_plan(57_600_000)
    tt = TaskTable(tasks)
    assert tt.n == len(tt) == 280
    assert tt.array.dtype == np.int64 and tt.array.shape == (280, 4)
    # same bytes the ctypes struct array would hold
    assert ctypes.sizeof(_lib.SfeChunk) == 32
    first = tt.ptr[0]
    assert (first.audio_start, first.audio_end, first.global_sample_offset, first.context_samples) == \
        (tasks[0].audio_start, tasks[0].audio_end, tasks[0].global_sample_offset, tasks[0].context_samples)
    last = tt.ptr[279]
    assert (last.audio_start, last.audio_end) == (tasks[-1].audio_start, tasks[-1].audio_end)
    assert int(tt.frame_offsets[-1]) == 418_312
    assert np.array_equal(np.diff(tt.frame_offsets), (tt.array[:, 1] - tt.array[:, 0]) // 160 + 1)


def test_task_table_from_array_and_empty():
    a = np.array([[0, 160, 0, 0], [100, 420, 100, 0]], np.int64)
    tt = TaskTable(a)
    assert list(tt.frame_offsets) == [0, 2, 5]  # 160 samples: 2 frames; 320: 3
    tt2 = TaskTable([ChunkTask(0, 160, 0, 0), ChunkTask(100, 420, 100, 0)])
    assert np.array_equal(tt.array, tt2.array)
    with pytest.raises(InvalidModelOutput):
        TaskTable([])


@pytest.mark.parametrize("dtype,bits,want", [("float32", None, (0, 32)), ("int16", None, (1, 16)),
                                             ("int16", 12, (1, 12)), ("int32", None, (2, 32)),
                                             ("int32", 24, (2, 24)), ("torch.int16", None, (1, 16))])
def test_pcm_format(dtype, bits, want):
    assert _pcm_format(dtype, bits) == want


def test_pcm_format_and_dtype_errors():
    with pytest.raises(InvalidModelOutput):
        _pcm_format("float64", None)
    with pytest.raises(InvalidModelOutput):
        _dtype_code("f16")
    assert _dtype_code("f32") == _lib.SFE_F32 and _dtype_code("bf16") == _lib.SFE_BF16


def test_vad_framer_rejects_host_tensors_and_small_outputs():
    import torch
    f = SileroVadFramer()
    with pytest.raises(InvalidModelOutput, match="device tensor"):
        f.model_inputs(torch.zeros(1000))
    with pytest.raises(InvalidModelOutput, match="at least"):
        f.model_inputs(torch.zeros(1000), out=torch.zeros((1, 576)))
    assert vad_num_windows(1000) == 2
    f.close()


class _FakeDeviceTensor:
    """Stands in for a device tensor so the argument checks that run before
    any GPU call can be exercised without a GPU."""

    def __init__(self, numel, dtype):
        self._n, self.dtype, self.is_cuda, self.device = numel, dtype, True, "cuda:0"

    def numel(self):
        return self._n

    def is_contiguous(self):
        return True

    def data_ptr(self):
        return 0


def test_batched_entry_points_validate_buffers_before_the_c_call():
    import torch
    from scriptrs_amd import ParakeetFeatureExtractor
    ext = ParakeetFeatureExtractor()
    f32, i16 = torch.float32, torch.int16
    tasks = [ChunkTask(0, 1600, 0, 0)]  # 11 frames
    good = _FakeDeviceTensor(128 * 11, f32)
    # samples of the wrong dtype would be read as 4-byte samples past their end
    with pytest.raises(InvalidModelOutput, match="samples must be"):
        ext.extract_chunks(_FakeDeviceTensor(1600, i16), tasks, out=good)
    with pytest.raises(InvalidModelOutput, match="samples must be"):
        ext.extract_batch(_FakeDeviceTensor(1600, i16), [0, 1600], out=good)
    with pytest.raises(InvalidModelOutput, match="samples must be"):
        ext.extract_chunks_encoder_input(_FakeDeviceTensor(1600, torch.float64), tasks, out=good)
    # offsets past the buffer (the C ABI has no length to check them against)
    with pytest.raises(InvalidModelOutput, match="past the"):
        ext.extract_batch(_FakeDeviceTensor(1599, f32), [0, 1600], out=good)
    with pytest.raises(InvalidModelOutput, match="non-decreasing"):
        ext.extract_batch(_FakeDeviceTensor(3200, f32), [0, 1600, 800], out=good)
    # a caller-supplied output of the wrong dtype or too small
    with pytest.raises(InvalidModelOutput, match="out must be"):
        ext.extract_chunks(_FakeDeviceTensor(1600, f32), tasks, out=_FakeDeviceTensor(128 * 11, torch.bfloat16))
    with pytest.raises(InvalidModelOutput, match="elements"):
        ext.extract_chunks(_FakeDeviceTensor(1600, f32), tasks, out=_FakeDeviceTensor(128 * 11 - 1, f32))
    with pytest.raises(InvalidModelOutput, match="elements"):
        ext.extract_chunks_pcm(_FakeDeviceTensor(1600, i16), tasks, dtype="bf16",
                               out=_FakeDeviceTensor(128 * 10, torch.bfloat16))
    with pytest.raises(InvalidModelOutput, match="elements"):
        ext.extract_batch(_FakeDeviceTensor(1600, f32), [0, 1600], out=_FakeDeviceTensor(100, f32))
    with pytest.raises(InvalidModelOutput, match="elements"):
        ext.extract_chunks_encoder_input(_FakeDeviceTensor(1600, f32), tasks, target_frames=1501,
                                         out=_FakeDeviceTensor(128 * 1500, f32))
    with pytest.raises(InvalidModelOutput, match="elements"):
        ext.extract_chunks_noalloc(_FakeDeviceTensor(1600, f32), tasks, out=_FakeDeviceTensor(5, f32))
    with pytest.raises(InvalidModelOutput, match="device tensor"):
        ext.extract_chunks(torch.zeros(1600), tasks, out=good)
    assert not ext._ctx  # nothing above reached the GPU


def test_noalloc_limits_checked_before_any_device_work():
    # more tasks than the static item table holds: rejected before the context is touched
    tt = TaskTable(np.array([[i, i + 160, i, 0] for i in range(4097)], np.int64))
    fo = np.zeros(tt.n + 1, np.int64)
    rc = _lib.lib().sfe_extract_chunks_noalloc(None, ctypes.c_void_p(16), 10_000, tt.ptr, tt.n, 0,
                                               ctypes.c_void_p(16), fo.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                                               None)
    assert rc == _lib.SFE_INVALID_ARG and "4096" in _lib.last_error()
    # more raw scratch than the 64 MiB array: 30 min of audio in 15 s chunks
    tt = TaskTable(build_fast_execution_plan(28_800_000))
    fo = np.zeros(tt.n + 1, np.int64)
    rc = _lib.lib().sfe_extract_chunks_noalloc(None, ctypes.c_void_p(16), 28_800_000, tt.ptr, tt.n, 0,
                                               ctypes.c_void_p(16), fo.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                                               None)
    assert rc == _lib.SFE_INVALID_ARG and "scratch" in _lib.last_error()
