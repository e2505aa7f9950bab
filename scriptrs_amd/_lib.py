"""ctypes binding of ``libscriptrs_fe.so`` (the C ABI in ``include/scriptrs_fe.h``).

The library is required: there is no fallback compute path.  If it has not
been built, importing succeeds but every call raises ``RuntimeError``.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# SFE_LIBRARY selects another build of the same C ABI (the measurement
# build libscriptrs_fe_ts.so, see scriptrs_amd/stamps.py).
LIB_PATH = os.environ.get("SFE_LIBRARY") or os.path.join(_HERE, "libscriptrs_fe.so")

SFE_OK, SFE_EMPTY_AUDIO, SFE_INVALID_ARG, SFE_HIP_ERROR, SFE_AUDIO_TOO_LONG = 0, 1, 2, 3, 4
SFE_F32, SFE_BF16 = 0, 1
SFE_PCM_F32, SFE_PCM_I16, SFE_PCM_I32 = 0, 1, 2

# Every symbol include/scriptrs_fe.h declares.
EXPORTS = (
    "sfe_config_default", "sfe_overlap_config_default", "sfe_num_frames", "sfe_max_feature_frames",
    "sfe_plan_fast", "sfe_build_tables", "sfe_last_error", "sfe_create", "sfe_destroy", "sfe_extract",
    "sfe_prepare_chunk", "sfe_extract_batch", "sfe_extract_chunks", "sfe_extract_chunks_pcm",
    "sfe_extract_chunks_padded", "sfe_extract_chunks_streamed", "sfe_extract_chunks_streamed_pcm",
    "sfe_set_frame_sharing", "sfe_set_timing", "sfe_get_timing", "sfe_vad_num_windows", "sfe_vad_frames", "sfe_extract_chunks_noalloc",
    "sfe_debug_allocation_count", "sfe_debug_mel_schedule", "sfe_debug_stamps",
)


class SfeConfig(ctypes.Structure):
    _fields_ = [
        ("sample_rate", ctypes.c_int32), ("feature_size", ctypes.c_int32), ("n_fft", ctypes.c_int32),
        ("win_length", ctypes.c_int32), ("hop_length", ctypes.c_int32), ("preemphasis", ctypes.c_float),
        ("max_audio_samples", ctypes.c_int64), ("samples_per_encoder_frame", ctypes.c_int32),
    ]


class SfeOverlapConfig(ctypes.Structure):
    _fields_ = [("overlap_seconds", ctypes.c_double), ("context_samples", ctypes.c_int64),
                ("max_model_samples", ctypes.c_int64)]


class SfeChunk(ctypes.Structure):
    _fields_ = [("audio_start", ctypes.c_int64), ("audio_end", ctypes.c_int64),
                ("global_sample_offset", ctypes.c_int64), ("context_samples", ctypes.c_int64)]


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    # torch ships its own libamdhip64 with the same soname (libamdhip64.so.7).
    # Whichever is loaded first serves the whole process, so load torch's
    # first: then this library and torch share one HIP runtime, and device
    # pointers and streams pass freely between them.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
            "(the front end has no CPU fallback)")
    L = ctypes.CDLL(LIB_PATH)
    P = ctypes.POINTER
    i32, i64, vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p
    fp, i64p = P(ctypes.c_float), P(ctypes.c_int64)
    sig = {
        "sfe_config_default": (None, [P(SfeConfig)]),
        "sfe_overlap_config_default": (None, [P(SfeOverlapConfig)]),
        "sfe_num_frames": (i64, [P(SfeConfig), i64]),
        "sfe_max_feature_frames": (i64, [P(SfeConfig)]),
        "sfe_plan_fast": (ctypes.c_int, [P(SfeOverlapConfig), i64, P(SfeChunk), i32, P(i32)]),
        "sfe_build_tables": (ctypes.c_int, [P(SfeConfig), fp, fp]),
        "sfe_last_error": (ctypes.c_char_p, []),
        "sfe_create": (ctypes.c_int, [P(SfeConfig), i32, P(vp)]),
        "sfe_destroy": (None, [vp]),
        "sfe_extract": (ctypes.c_int, [vp, fp, i64, fp, i64]),
        "sfe_prepare_chunk": (ctypes.c_int, [vp, fp, i64, fp, i64, i64p]),
        "sfe_extract_batch": (ctypes.c_int, [vp, vp, i64p, i32, i32, vp, i64p, vp]),
        "sfe_extract_chunks": (ctypes.c_int, [vp, vp, i64, P(SfeChunk), i32, i32, vp, i64p, vp]),
        "sfe_extract_chunks_pcm": (ctypes.c_int, [vp, vp, i32, i32, i64, P(SfeChunk), i32, i32, vp, i64p, vp]),
        "sfe_extract_chunks_streamed_pcm": (ctypes.c_int, [vp, vp, i32, i32, i64, P(SfeChunk), i32, i32, vp, i64p,
                                                           i64]),
        "sfe_extract_chunks_noalloc": (ctypes.c_int, [vp, vp, i64, P(SfeChunk), i32, i32, vp, i64p, vp]),
        "sfe_extract_chunks_padded": (ctypes.c_int, [vp, vp, i64, P(SfeChunk), i32, i32, i32, vp, i64p, vp]),
        "sfe_extract_chunks_streamed": (ctypes.c_int, [vp, fp, i64, P(SfeChunk), i32, i32, vp, i64p, i64]),
        "sfe_vad_num_windows": (i64, [i64]),
        "sfe_vad_frames": (ctypes.c_int, [vp, vp, i32, i32, i64, vp, i64, vp]),
        "sfe_set_frame_sharing": (ctypes.c_int, [vp, i32]),
        "sfe_set_timing": (ctypes.c_int, [vp, i32]),
        "sfe_get_timing": (ctypes.c_int, [vp, P(ctypes.c_double), P(ctypes.c_double), P(i32)]),
        "sfe_debug_allocation_count": (i64, []),
        "sfe_debug_mel_schedule": (ctypes.c_int, [P(SfeConfig)]),
        "sfe_debug_stamps": (ctypes.c_int, [vp, i64]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return _lib


def last_error() -> str:
    return lib().sfe_last_error().decode("utf-8", "replace")
