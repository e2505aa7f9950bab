"""Long-form overlap planning restated in pure Python (TEST INFRASTRUCTURE).

Follows ``src/long_form/planner.rs:83-137`` (``OverlapChunkConfig``) and
``src/long_form.rs:439-459,566-582`` (``build_fast_execution_plan`` /
``push_overlap_task``).  All integer arithmetic; ``usize::saturating_sub`` is
written as ``max(a - b, 0)``.  Pinned by the reference's own planner tests
(``src/long_form/planner.rs:376-385``, ``src/long_form.rs:757-769``) and by the
committed chunk-table fixtures.
"""
from __future__ import annotations

from dataclasses import dataclass

SAMPLE_RATE = 16_000                 # src/constants.rs:1
MAX_MODEL_SAMPLES = 240_000          # src/constants.rs:2
MEL_HOP_SAMPLES = 160                # src/constants.rs:3
SAMPLES_PER_ENCODER_FRAME = 1280     # src/constants.rs:4-5 (160 * 8)


@dataclass(frozen=True)
class OverlapChunkConfig:
    overlap_seconds: float = 2.0                         # planner.rs:97
    context_samples: int = SAMPLES_PER_ENCODER_FRAME     # planner.rs:98
    max_model_samples: int = MAX_MODEL_SAMPLES           # planner.rs:99

    def chunk_samples(self) -> int:                      # planner.rs:105-111
        max_actual = max(self.max_model_samples - self.context_samples, 0)
        raw = max(max_actual - MEL_HOP_SAMPLES, 0)
        raw = max(raw, SAMPLES_PER_ENCODER_FRAME)
        return raw // SAMPLES_PER_ENCODER_FRAME * SAMPLES_PER_ENCODER_FRAME

    def overlap_samples(self) -> int:                    # planner.rs:113-117
        requested = int(self.overlap_seconds * SAMPLE_RATE)  # `as usize` truncates (saturating at 0)
        requested = max(requested, 0)
        capped = min(requested, self.chunk_samples() // 2)
        return capped // SAMPLES_PER_ENCODER_FRAME * SAMPLES_PER_ENCODER_FRAME

    def stride_samples(self) -> int:                     # planner.rs:119-122
        raw = max(self.chunk_samples() - self.overlap_samples(), 0)
        return max(raw, SAMPLES_PER_ENCODER_FRAME) // SAMPLES_PER_ENCODER_FRAME * SAMPLES_PER_ENCODER_FRAME

    def plan(self, start: int, end: int):                # planner.rs:124-136
        chunks = []
        s = start
        while s < end:
            e = min(s + self.chunk_samples(), end)
            chunks.append((s, e))
            if e == end:
                break
            s += self.stride_samples()
        return chunks


@dataclass(frozen=True)
class ChunkTask:
    audio_start: int
    audio_end: int
    global_sample_offset: int
    context_samples: int


def build_fast_execution_plan(audio_len: int, cfg: OverlapChunkConfig = OverlapChunkConfig()):
    """``src/long_form.rs:439-459`` + ``push_overlap_task`` (``:566-582``)."""
    tasks = []
    for s, e in cfg.plan(0, audio_len):
        ctx_start = max(s - cfg.context_samples, 0)
        tasks.append(ChunkTask(ctx_start, e, s, s - ctx_start))
    return tasks


def parallel_worker_count(task_count: int, requested: int) -> int:
    """``src/long_form.rs:594-600``."""
    if task_count <= 1:
        return 1
    return min(max(requested, 1), task_count)
