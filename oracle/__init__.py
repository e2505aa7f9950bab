"""CPU oracle for the scriptrs log-mel front end.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this package, and only as the
checker (or the timed CPU baseline), never as the thing measured or shipped.

Contents:
  * ``sfe_oracle.c`` (built to ``libsfe_oracle.so`` by ``oracle/Makefile``):
    the op-for-op C restatement of ``src/frontend.rs:59-241``.
  * ``planner``: the long-form overlap planner, ``src/long_form/planner.rs:104-137``
    and ``src/long_form.rs:439-459,566-582``, restated in pure Python.

Parity status (what pins each function) is listed in each docstring.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

from . import planner  # noqa: F401

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libsfe_oracle.so")
_lib = None

N_MELS = 128
N_FFT = 512
WIN = 400
HOP = 160
SAMPLE_RATE = 16000


class _Config(ctypes.Structure):
    """``sfo_config`` (sfe_oracle.c), the fields of ``TranscriptionConfig``
    (src/config.rs:11-27) the front end reads."""
    _fields_ = [("sample_rate", ctypes.c_int32), ("feature_size", ctypes.c_int32), ("n_fft", ctypes.c_int32),
                ("win_length", ctypes.c_int32), ("hop_length", ctypes.c_int32), ("preemphasis", ctypes.c_float)]


def build() -> str:
    """Compile the oracle with its Makefile (gcc); returns the .so path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        i64, i32, f32p, i64p = ctypes.c_int64, ctypes.c_int32, ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_int64)
        L.sfo_num_frames.argtypes = [i64, i32]
        L.sfo_num_frames.restype = i64
        L.sfo_hann_window.argtypes = [i32, f32p]
        L.sfo_mel_filterbank.argtypes = [i32, i32, i32, f32p]
        L.sfo_extract.argtypes = [f32p, i64, f32p]
        L.sfo_extract.restype = ctypes.c_int
        L.sfo_stft_power.argtypes = [f32p, i64, f32p]
        L.sfo_stft_power.restype = ctypes.c_int
        L.sfo_extract_spans.argtypes = [f32p, i64p, i64p, i32, f32p, i64p, i32]
        L.sfo_extract_spans.restype = ctypes.c_int
        L.sfo_vad_frames.argtypes = [f32p, i64, f32p]
        L.sfo_vad_frames.restype = i64
        L.sfo_extract_cfg.argtypes = [ctypes.POINTER(_Config), f32p, i64, f32p]
        L.sfo_extract_cfg.restype = ctypes.c_int
        _lib = L
    return _lib


def _fp(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _ip(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))


def num_frames(length: int) -> int:
    """``L / hop + 1`` (``src/frontend.rs:124-127`` with ``padded.len() = L + n_fft``)."""
    return int(lib().sfo_num_frames(int(length), HOP))


def hann_window(win: int = WIN) -> np.ndarray:
    """``src/frontend.rs:161-165`` in f32.  Pinned bit-exactly by an independent
    numpy float32 evaluation of the same expression and by symmetry."""
    out = np.empty(win, np.float32)
    lib().sfo_hann_window(win, _fp(out))
    return out


def mel_filterbank(n_fft: int = N_FFT, n_mels: int = N_MELS, sr: int = SAMPLE_RATE) -> np.ndarray:
    """``src/frontend.rs:188-223`` -> [n_mels, n_fft/2+1] f32.  Pinned by an
    independent numpy Slaney restatement and the Slaney-area invariant."""
    out = np.empty((n_mels, n_fft // 2 + 1), np.float32)
    lib().sfo_mel_filterbank(n_fft, n_mels, sr, _fp(out))
    return out


def stft_power(audio: np.ndarray) -> np.ndarray:
    """``src/frontend.rs:120-147`` -> [257, T] f32 power spectrogram."""
    a = np.ascontiguousarray(audio, np.float32)
    if a.size == 0:
        raise ValueError("EmptyAudio")
    out = np.empty((N_FFT // 2 + 1, num_frames(a.size)), np.float32)
    lib().sfo_stft_power(_fp(a), a.size, _fp(out))
    return out


def extract(audio: np.ndarray) -> np.ndarray:
    """``ParakeetFeatureExtractor::extract`` (``src/frontend.rs:104-118``).

    Returns the feature-major [128, T] f32 array (the memory order of the
    reference's [T, 128] result).  Raises ValueError("EmptyAudio") on empty
    input like ``src/frontend.rs:105-107``."""
    a = np.ascontiguousarray(audio, np.float32)
    if a.size == 0:
        raise ValueError("EmptyAudio")
    out = np.empty((N_MELS, num_frames(a.size)), np.float32)
    rc = lib().sfo_extract(_fp(a), a.size, _fp(out))
    if rc != 0:
        raise ValueError("EmptyAudio")
    return out


def extract_cfg(audio: np.ndarray, sample_rate: int = SAMPLE_RATE, preemphasis: float = 0.97) -> np.ndarray:
    """``extract`` under a ``TranscriptionConfig`` with another sample rate
    (the mel filterbank's band edges, ``src/frontend.rs:188-223``) or
    preemphasis coefficient (``src/frontend.rs:150-163``); the frame shape
    stays n_fft 512, window 400, hop 160, 128 features."""
    a = np.ascontiguousarray(audio, np.float32)
    if a.size == 0:
        raise ValueError("EmptyAudio")
    c = _Config(sample_rate, N_MELS, N_FFT, WIN, HOP, preemphasis)
    out = np.empty((N_MELS, num_frames(a.size)), np.float32)
    if lib().sfo_extract_cfg(ctypes.byref(c), _fp(a), a.size, _fp(out)) != 0:
        raise ValueError("EmptyAudio")
    return out


def extract_spans(samples: np.ndarray, starts, lens, nthreads: int = 4):
    """Featurize independent spans of one buffer on ``nthreads`` CPU workers
    (``src/long_form.rs:266-314``: an atomic task counter over chunk tasks).
    Returns (out [128 * sum T_i] flat, frame_offsets [n+1])."""
    s = np.ascontiguousarray(samples, np.float32)
    st = np.ascontiguousarray(starts, np.int64)
    ln = np.ascontiguousarray(lens, np.int64)
    n = st.size
    fo = np.zeros(n + 1, np.int64)
    fo[1:] = np.cumsum(ln // HOP + 1)
    out = np.empty(N_MELS * int(fo[-1]), np.float32)
    rc = lib().sfo_extract_spans(_fp(s), _ip(st), _ip(ln), n, _fp(out), _ip(fo), nthreads)
    if rc != 0:
        raise ValueError("EmptyAudio")
    return out, fo


def vad_frames(audio: np.ndarray) -> np.ndarray:
    """Silero VAD model inputs, [ceil(len/512), 576] float32: the reference's
    window/context loop (``src/long_form/vad.rs:62-99``) restated in C."""
    a = np.ascontiguousarray(audio, np.float32).reshape(-1)
    n = (a.size + 511) // 512
    out = np.empty((n, 576), np.float32)
    rows = lib().sfo_vad_frames(_fp(a), a.size, _fp(out))
    assert rows == n
    return out
