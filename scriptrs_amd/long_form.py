"""Long-form chunk planning and batched featurization.

Mirrors the parts of scriptrs' long-form path that decide which samples
each chunk gets and featurize them:
  * ``OverlapChunkConfig`` -- src/long_form/planner.rs:83-137.  The integer
    plan itself runs in the library (``sfe_plan_fast``).
  * ``ChunkTask`` / ``build_fast_execution_plan`` -- src/long_form.rs:439-459, :566-582.
  * ``LongFormConfig`` (mode Fast, ``worker_count`` 4) -- src/long_form.rs:57-87.
  * ``featurize_long_form`` replaces the per-worker ``ChunkPreparer::prepare``
    loop (src/long_form.rs:266-314, :584-592) with one batched GPU pass.
    It returns features in task order, as ``consume_prepared_tasks`` reassembles
    them (src/long_form.rs:316-342).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from ._lib import SfeChunk, SfeOverlapConfig
from .frontend import EmptyAudio, InvalidModelOutput, ParakeetFeatureExtractor, TranscriptionConfig


@dataclass(frozen=True)
class SampleRange:
    start: int
    end: int


@dataclass(frozen=True)
class ChunkTask:
    """``ChunkTask`` for an overlap window (src/long_form.rs:566-582)."""
    audio_start: int
    audio_end: int
    global_sample_offset: int
    context_samples: int


@dataclass
class OverlapChunkConfig:
    """``OverlapChunkConfig`` with the defaults of src/long_form/planner.rs:94-102."""
    overlap_seconds: float = 2.0
    context_samples: int = 1280
    max_model_samples: int = 240_000

    def _c(self) -> SfeOverlapConfig:
        return SfeOverlapConfig(self.overlap_seconds, self.context_samples, self.max_model_samples)

    def tasks(self, audio_len: int) -> list[ChunkTask]:
        """``plan`` over [0, audio_len) mapped through ``push_overlap_task``."""
        L = _lib.lib()
        c = self._c()
        n = ctypes.c_int32(0)
        rc = L.sfe_plan_fast(ctypes.byref(c), int(audio_len), None, 0, ctypes.byref(n))
        if n.value == 0:
            return []
        if rc not in (_lib.SFE_OK, _lib.SFE_INVALID_ARG):
            raise InvalidModelOutput(_lib.last_error())
        arr = (SfeChunk * n.value)()
        rc = L.sfe_plan_fast(ctypes.byref(c), int(audio_len), arr, n.value, ctypes.byref(n))
        if rc != _lib.SFE_OK:
            raise InvalidModelOutput(_lib.last_error())
        return [ChunkTask(t.audio_start, t.audio_end, t.global_sample_offset, t.context_samples) for t in arr]

    def plan(self, rng: SampleRange) -> list[SampleRange]:
        """``OverlapChunkConfig::plan`` (src/long_form/planner.rs:124-137) over ``rng``."""
        return [SampleRange(t.global_sample_offset + rng.start, t.audio_end + rng.start)
                for t in self.tasks(rng.end - rng.start)]


@dataclass
class LongFormConfig:
    """``LongFormConfig`` (src/long_form.rs:57-87); only the Fast mode exists here."""
    mode: str = "fast"
    worker_count: int = 4
    transcription: TranscriptionConfig = field(default_factory=TranscriptionConfig)
    overlap: OverlapChunkConfig = field(default_factory=OverlapChunkConfig)


def build_fast_execution_plan(audio_len: int, config: LongFormConfig | None = None) -> list[ChunkTask]:
    """Task list of ``build_fast_execution_plan`` (src/long_form.rs:439-459)."""
    return (config or LongFormConfig()).overlap.tasks(audio_len)


def parallel_worker_count(task_count: int, requested_workers: int) -> int:
    """src/long_form.rs:594-600."""
    if task_count <= 1:
        return 1
    return min(max(requested_workers, 1), task_count)


@dataclass
class LongFormFeatures:
    """Features of every task, in task order.  ``features`` is flat, feature-major
    per task; ``chunk(i)`` gives task i's [128, T_i] view."""
    tasks: list[ChunkTask]
    features: object  # torch tensor on the device
    frame_offsets: np.ndarray
    feature_size: int = 128

    def chunk(self, i: int):
        a, b = int(self.frame_offsets[i]), int(self.frame_offsets[i + 1])
        return self.features[a * self.feature_size:b * self.feature_size].view(self.feature_size, b - a)


def featurize_long_form(extractor: ParakeetFeatureExtractor, recording, config: LongFormConfig | None = None,
                        dtype: str = "f32", stream=None) -> LongFormFeatures:
    """Featurize a device recording the way ``run_fast_long_form`` does
    (src/long_form.rs:218-228), as one batched GPU pass.  Recordings that fit
    one chunk go through the single-chunk path like ``run_with_config``
    (src/long_form.rs:161-163): they become one task covering the whole
    recording."""
    cfg = config or LongFormConfig()
    n = int(recording.numel())
    if n == 0:
        raise EmptyAudio()
    if n <= cfg.transcription.max_audio_samples:
        tasks = [ChunkTask(0, n, 0, 0)]
    else:
        tasks = build_fast_execution_plan(n, cfg)
    out, fo = extractor.extract_chunks(recording, tasks, dtype=dtype, stream=stream)
    return LongFormFeatures(tasks, out, fo, cfg.transcription.feature_size)
