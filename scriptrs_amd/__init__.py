"""MI355X-native log-mel front end of scriptrs (src/frontend.rs), batched over
the chunks of its long-form planner (src/long_form).

All feature computation runs in hand-written gfx950 HIP kernels inside
``libscriptrs_fe.so``, reached through the C ABI in ``include/scriptrs_fe.h``.
"""
from .frontend import (  # noqa: F401
    AudioTooLong, ChunkPreparer, EmptyAudio, InvalidModelOutput, ParakeetFeatureExtractor, PreparedChunk,
    TaskTable, TranscriptionConfig, TranscriptionError, build_tables, num_frames,
)
from .long_form import (  # noqa: F401
    ChunkTask, LongFormConfig, LongFormFeatures, OverlapChunkConfig, SampleRange, build_fast_execution_plan,
    featurize_long_form, parallel_worker_count,
)
from .vad import (  # noqa: F401
    VAD_CONTEXT_SAMPLES, VAD_INPUT_SAMPLES, VAD_WINDOW_SAMPLES, SileroVadFramer, vad_num_windows,
)
