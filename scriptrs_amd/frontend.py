"""Host-side mirror of scriptrs' front-end API over the C ABI.

Names, argument meaning and error behaviour follow the reference:
  * ``TranscriptionConfig``       -- src/config.rs:11-53
  * ``TranscriptionError`` family -- src/error.rs:5-40 (the subset on this path)
  * ``ParakeetFeatureExtractor``  -- src/frontend.rs:11-118 (``new``, ``extract``) plus
    the batched entry points that replace per-chunk calls
  * ``ChunkPreparer`` / ``PreparedChunk`` -- src/pipeline.rs:167-216
All compute runs in ``libscriptrs_fe.so`` on the GPU; nothing here computes features.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Sequence

import numpy as np

from . import _lib
from ._lib import SfeChunk, SfeConfig


class TranscriptionError(Exception):
    """Base of the reference's error enum (src/error.rs:5)."""


class EmptyAudio(TranscriptionError):
    """``TranscriptionError::EmptyAudio`` (src/error.rs:7-8)."""

    def __init__(self, msg: str = "audio input was empty"):
        super().__init__(msg)


class AudioTooLong(TranscriptionError):
    """``TranscriptionError::AudioTooLong`` (src/error.rs:10-18)."""

    def __init__(self, max_seconds: float, actual_seconds: float):
        self.max_seconds = max_seconds
        self.actual_seconds = actual_seconds
        super().__init__(f"audio exceeds the single-chunk limit: actual={actual_seconds:.2f}s max={max_seconds:.2f}s")


class InvalidModelOutput(TranscriptionError):
    """``TranscriptionError::InvalidModelOutput`` (src/error.rs:31-33); carries the
    library's message for SFE_INVALID_ARG and SFE_HIP_ERROR."""


def _check(rc: int, *, max_seconds: float = 0.0, actual_seconds: float = 0.0) -> None:
    if rc == _lib.SFE_OK:
        return
    if rc == _lib.SFE_EMPTY_AUDIO:
        raise EmptyAudio()
    if rc == _lib.SFE_AUDIO_TOO_LONG:
        raise AudioTooLong(max_seconds, actual_seconds)
    raise InvalidModelOutput(_lib.last_error())


@dataclass
class TranscriptionConfig:
    """``TranscriptionConfig`` with the defaults of src/config.rs:30-44."""
    sample_rate: int = 16_000
    feature_size: int = 128
    n_fft: int = 512
    win_length: int = 400
    hop_length: int = 160
    preemphasis: float = 0.97
    max_audio_samples: int = 240_000
    samples_per_encoder_frame: int = 1280

    def max_duration_seconds(self) -> float:  # src/config.rs:46-48
        return self.max_audio_samples / self.sample_rate

    def max_feature_frames(self) -> int:  # src/config.rs:50-52
        return self.max_audio_samples // self.hop_length + 1

    def to_c(self) -> SfeConfig:
        return SfeConfig(self.sample_rate, self.feature_size, self.n_fft, self.win_length, self.hop_length,
                         self.preemphasis, self.max_audio_samples, self.samples_per_encoder_frame)


def num_frames(length: int, config: TranscriptionConfig | None = None) -> int:
    """``L / hop + 1`` via the library (src/frontend.rs:124-127)."""
    cfg = (config or TranscriptionConfig()).to_c()
    return int(_lib.lib().sfe_num_frames(ctypes.byref(cfg), int(length)))


def build_tables(config: TranscriptionConfig | None = None):
    """The library's host tables: (hann window [win], mel filterbank [F, n_fft/2+1])."""
    c = config or TranscriptionConfig()
    w = np.empty(c.win_length, np.float32)
    fb = np.empty((c.feature_size, c.n_fft // 2 + 1), np.float32)
    cc = c.to_c()
    _check(_lib.lib().sfe_build_tables(ctypes.byref(cc), _fp(w), _fp(fb)))
    return w, fb


def _fp(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _ip(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))


def _stream_handle(stream) -> ctypes.c_void_p:
    if stream is None:
        import torch
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(int(getattr(stream, "cuda_stream", stream)))


def _dev_ptr(t) -> ctypes.c_void_p:
    if not getattr(t, "is_cuda", False):
        raise InvalidModelOutput("expected a device tensor")
    if not t.is_contiguous():
        raise InvalidModelOutput("expected a contiguous tensor")
    return ctypes.c_void_p(t.data_ptr())


def _torch_dtype(dtype: str):
    import torch
    _dtype_code(dtype)
    return torch.float32 if dtype == "f32" else torch.bfloat16


def _check_samples(t, *dtypes) -> None:
    """The C ABI reads ``numel`` samples of the element size its format
    implies; a tensor of another dtype would be read past its end."""
    _dev_ptr(t)
    if t.dtype not in dtypes:
        raise InvalidModelOutput(f"samples must be {' or '.join(str(d) for d in dtypes)}, got {t.dtype}")


def _check_out(out, dtype: str, numel: int) -> None:
    """A caller-supplied output must have the requested dtype and room for
    every element the kernels write."""
    _dev_ptr(out)
    want = _torch_dtype(dtype)
    if out.dtype != want:
        raise InvalidModelOutput(f"out must be {want} for dtype {dtype!r}, got {out.dtype}")
    if out.numel() < numel:
        raise InvalidModelOutput(f"out holds {out.numel()} elements, {numel} needed")


class ParakeetFeatureExtractor:
    """Mirror of ``ParakeetFeatureExtractor`` (src/frontend.rs:11-118).

    ``ParakeetFeatureExtractor(config)`` is ``new`` (src/frontend.rs:88): it
    builds the tables and uploads them to ``device`` on first use.  One
    instance per host thread, like the reference (``!Sync`` workspace).
    """

    def __init__(self, config: TranscriptionConfig | None = None, device: int = 0):
        self.config = config or TranscriptionConfig()
        self.device = device
        self._ctx = ctypes.c_void_p()

    # -- context ---------------------------------------------------------------
    def _handle(self) -> ctypes.c_void_p:
        if not self._ctx:
            cfg = self.config.to_c()
            _check(_lib.lib().sfe_create(ctypes.byref(cfg), self.device, ctypes.byref(self._ctx)))
        return self._ctx

    def close(self) -> None:
        if self._ctx:
            _lib.lib().sfe_destroy(self._ctx)
            self._ctx = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_frame_sharing(self, enable: bool) -> None:
        """Overlapping chunk tasks of one call compute the frames they share
        once (on by default; the output is bitwise the same either way)."""
        _check(_lib.lib().sfe_set_frame_sharing(self._handle(), 1 if enable else 0))

    def num_frames(self, length: int) -> int:
        return length // self.config.hop_length + 1

    # -- the reference's entry point ---------------------------------------------
    def extract(self, audio) -> np.ndarray:
        """``extract(&self, audio: &[f32]) -> Array2<f32>`` (src/frontend.rs:104-118).

        Returns the logical [T, 128] array, stored feature-major like the
        reference's ``.t().to_owned()`` result (``out.T`` of a [128, T] array).
        Raises ``EmptyAudio`` for empty input before touching the GPU.
        """
        a = np.ascontiguousarray(audio, dtype=np.float32).reshape(-1)
        if a.size == 0:
            raise EmptyAudio()
        T = self.num_frames(a.size)
        out = np.empty((self.config.feature_size, T), np.float32)
        _check(_lib.lib().sfe_extract(self._handle(), _fp(a), a.size, _fp(out), out.size))
        return out.T

    # -- batched entry points (one GPU launch sequence) ---------------------------
    def extract_batch(self, samples, offsets: Sequence[int], dtype: str = "f32", stream=None, out=None):
        """Featurize clips ``samples[offsets[i]:offsets[i+1]]`` of a device tensor.

        Returns ``(out, frame_offsets)``: ``out`` is a flat device tensor of
        ``128 * sum(T_i)`` elements, clip ``i`` at ``out[128*fo[i]:128*fo[i+1]]``
        viewed as [128, T_i].  Each clip matches one ``extract`` call."""
        import torch
        _check_samples(samples, torch.float32)
        off = np.ascontiguousarray(offsets, np.int64).reshape(-1)
        n = off.size - 1
        if n <= 0:
            raise InvalidModelOutput("need at least one clip")
        if off[0] < 0 or np.any(np.diff(off) < 0):
            raise InvalidModelOutput("offsets must be non-negative and non-decreasing")
        if off[-1] > samples.numel():
            raise InvalidModelOutput(f"offsets run to {int(off[-1])}, past the {samples.numel()} samples")
        if np.any(np.diff(off) == 0):
            raise EmptyAudio()
        fo = np.zeros(n + 1, np.int64)
        fo[1:] = np.cumsum(np.diff(off) // self.config.hop_length + 1)
        if out is None:
            out = torch.empty(int(fo[-1]) * self.config.feature_size, dtype=_torch_dtype(dtype), device=samples.device)
        _check_out(out, dtype, int(fo[-1]) * self.config.feature_size)
        rc = _lib.lib().sfe_extract_batch(self._handle(), _dev_ptr(samples), _ip(off), n, _dtype_code(dtype),
                                          _dev_ptr(out), _ip(fo), _stream_handle(stream))
        _check(rc)
        return out, fo

    def extract_chunks(self, recording, tasks, dtype: str = "f32", stream=None, out=None):
        """Featurize long-form chunk tasks over one device recording without
        copying the overlaps (replaces the per-task ``ChunkPreparer::prepare``
        calls of src/long_form.rs:584-592)."""
        import torch
        _check_samples(recording, torch.float32)
        tt = _tasks_array(tasks, self.config.hop_length)
        arr, n = tt.ptr, tt.n
        fo = tt.frame_offsets.copy()
        if out is None:
            out = torch.empty(int(fo[-1]) * self.config.feature_size, dtype=_torch_dtype(dtype), device=recording.device)
        _check_out(out, dtype, int(fo[-1]) * self.config.feature_size)
        rc = _lib.lib().sfe_extract_chunks(self._handle(), _dev_ptr(recording), recording.numel(), arr, n,
                                           _dtype_code(dtype), _dev_ptr(out), _ip(fo), _stream_handle(stream))
        _check(rc)
        return out, fo

    def extract_chunks_noalloc(self, recording, tasks, dtype: str = "f32", stream=None, out=None):
        """``extract_chunks`` through the allocation-free entry point: the
        library keeps its item table and raw log-mel in a static per-GPU
        array (at most 4096 tasks and 64 MiB of raw log-mel per call) and
        allocates nothing.  Calls that overlap on one GPU race on that array.
        ``out`` should be preallocated by callers that cannot allocate."""
        import torch
        _check_samples(recording, torch.float32)
        tt = _tasks_array(tasks, self.config.hop_length)
        fo = tt.frame_offsets.copy()
        if out is None:
            out = torch.empty(int(fo[-1]) * self.config.feature_size, dtype=_torch_dtype(dtype), device=recording.device)
        _check_out(out, dtype, int(fo[-1]) * self.config.feature_size)
        rc = _lib.lib().sfe_extract_chunks_noalloc(self._handle(), _dev_ptr(recording), recording.numel(), tt.ptr,
                                                   tt.n, _dtype_code(dtype), _dev_ptr(out), _ip(fo),
                                                   _stream_handle(stream))
        _check(rc)
        return out, fo

    def extract_chunks_pcm(self, recording, tasks, bits_per_sample: int | None = None, dtype: str = "f32",
                           stream=None, out=None):
        """``extract_chunks`` over a device recording of integer PCM (torch.int16
        or torch.int32), decoded in the kernel as the reference's WAV reader
        does: ``value as f32 / ((1 << (bits - 1)) - 1) as f32``
        (examples/transcribe_wav.rs:342-348).  ``bits_per_sample`` defaults to
        the container width."""
        import torch
        _check_samples(recording, torch.float32, torch.int16, torch.int32)
        pcm, bits = _pcm_format(recording.dtype, bits_per_sample)
        tt = _tasks_array(tasks, self.config.hop_length)
        arr, n = tt.ptr, tt.n
        fo = tt.frame_offsets.copy()
        if out is None:
            out = torch.empty(int(fo[-1]) * self.config.feature_size, dtype=_torch_dtype(dtype), device=recording.device)
        _check_out(out, dtype, int(fo[-1]) * self.config.feature_size)
        rc = _lib.lib().sfe_extract_chunks_pcm(self._handle(), _dev_ptr(recording), pcm, bits, recording.numel(), arr,
                                               n, _dtype_code(dtype), _dev_ptr(out), _ip(fo), _stream_handle(stream))
        _check(rc)
        return out, fo

    def extract_chunks_encoder_input(self, recording, tasks, target_frames: int | None = None, dtype: str = "f32",
                                     stream=None, out=None):
        """Featurize chunk tasks straight into the encoder input layout: a
        device tensor [n, 128, target_frames], feature-major, zero past each
        chunk's frame count -- what ``EncoderInputBuffer::copy_from_features``
        builds on the host (src/model.rs:241-278).  ``target_frames`` defaults
        to ``max_feature_frames()`` (``PreparedChunk::target_frames``,
        src/pipeline.rs:160-163).  Returns ``(out, feature_frames)``."""
        import torch
        _check_samples(recording, torch.float32)
        tt = _tasks_array(tasks, self.config.hop_length)
        arr, n = tt.ptr, tt.n
        tf = int(target_frames or self.config.max_feature_frames())
        ff = np.zeros(n, np.int64)
        if out is None:
            out = torch.empty((n, self.config.feature_size, tf), dtype=_torch_dtype(dtype), device=recording.device)
        _check_out(out, dtype, n * self.config.feature_size * tf)
        rc = _lib.lib().sfe_extract_chunks_padded(self._handle(), _dev_ptr(recording), recording.numel(), arr, n, tf,
                                                  _dtype_code(dtype), _dev_ptr(out), _ip(ff), _stream_handle(stream))
        _check(rc)
        return out, ff

    def extract_chunks_streamed(self, host_recording: np.ndarray, tasks, window_samples: int = 960_000,
                                dtype: str = "f32", out=None, bits_per_sample: int | None = None):
        """Streamed long-form extraction: the recording stays in host memory and
        is copied in double-buffered windows of ``window_samples`` samples.
        float32, int16 or int32 PCM; integer PCM crosses PCIe at its own width
        and is decoded on the GPU (see ``extract_chunks_pcm``)."""
        import torch
        h = np.ascontiguousarray(host_recording)
        if h.dtype not in (np.float32, np.int16, np.int32):
            h = h.astype(np.float32)
        pcm, bits = _pcm_format(h.dtype, bits_per_sample)
        tt = _tasks_array(tasks, self.config.hop_length)
        arr, n = tt.ptr, tt.n
        fo = tt.frame_offsets.copy()
        if out is None:
            out = torch.empty(int(fo[-1]) * self.config.feature_size, dtype=_torch_dtype(dtype),
                              device=f"cuda:{self.device}")
        _check_out(out, dtype, int(fo[-1]) * self.config.feature_size)
        rc = _lib.lib().sfe_extract_chunks_streamed_pcm(self._handle(), h.ctypes.data_as(ctypes.c_void_p), pcm, bits,
                                                        h.size, arr, n, _dtype_code(dtype), _dev_ptr(out), _ip(fo),
                                                        int(window_samples))
        _check(rc)
        return out, fo


def _pcm_format(dtype, bits):
    """(sfe_pcm code, bits_per_sample) for a numpy or torch sample dtype."""
    name = str(dtype).replace("torch.", "")
    if name == "float32":
        return _lib.SFE_PCM_F32, 32
    if name == "int16":
        return _lib.SFE_PCM_I16, int(bits or 16)
    if name == "int32":
        return _lib.SFE_PCM_I32, int(bits or 32)
    raise InvalidModelOutput(f"unsupported sample dtype {name}")


def _dtype_code(dtype: str) -> int:
    if dtype == "f32":
        return _lib.SFE_F32
    if dtype == "bf16":
        return _lib.SFE_BF16
    raise InvalidModelOutput(f"unsupported dtype {dtype!r}")


class TaskTable:
    """Chunk tasks in the C ABI's ``sfe_chunk`` layout (4 x int64 per task:
    audio_start, audio_end, global_sample_offset, context_samples) with their
    frame offsets.  Build it once per plan and pass it to the ``extract_chunks*``
    calls; a plain list of ``ChunkTask`` is converted on every call."""

    def __init__(self, tasks, hop_length: int = 160):
        if isinstance(tasks, np.ndarray):
            a = np.ascontiguousarray(tasks, np.int64).reshape(-1, 4)
        else:
            a = np.array([(t.audio_start, t.audio_end, t.global_sample_offset, t.context_samples) for t in tasks],
                         np.int64).reshape(-1, 4)
        if a.shape[0] == 0:
            raise InvalidModelOutput("no tasks")
        self.array = a
        self.n = int(a.shape[0])
        self.frame_offsets = np.zeros(self.n + 1, np.int64)
        np.cumsum((a[:, 1] - a[:, 0]) // hop_length + 1, out=self.frame_offsets[1:])
        self.ptr = a.ctypes.data_as(ctypes.POINTER(SfeChunk))

    def __len__(self):
        return self.n


def _tasks_array(tasks, hop_length: int = 160) -> TaskTable:
    return tasks if isinstance(tasks, TaskTable) else TaskTable(tasks, hop_length)


@dataclass
class PreparedChunk:
    """``PreparedChunk`` (src/pipeline.rs:167-183)."""
    features: np.ndarray  # logical [T, 128]
    feature_frames: int
    target_frames: int


class ChunkPreparer:
    """``ChunkPreparer`` (src/pipeline.rs:185-216): length checks, then extract."""

    def __init__(self, config: TranscriptionConfig | None = None, device: int = 0):
        self.config = config or TranscriptionConfig()
        self.extractor = ParakeetFeatureExtractor(self.config, device)

    def prepare(self, audio) -> PreparedChunk:
        a = np.ascontiguousarray(audio, dtype=np.float32).reshape(-1)
        if a.size == 0:
            raise EmptyAudio()
        if a.size > self.config.max_audio_samples:
            raise AudioTooLong(self.config.max_duration_seconds(), a.size / self.config.sample_rate)
        feats = self.extractor.extract(a)
        return PreparedChunk(feats, feats.shape[0], self.config.max_feature_frames())
