"""VAD model-input framing (src/long_form/vad.rs:62-99) without a GPU.

The oracle restates the reference's stateful loop: copy the window, pad a
short one with its last sample, emit [context | window], keep the last 64
samples as the next context.  It is pinned here against the closed form
that loop reduces to (every window but the last is full), built with numpy
indexing, not a loop:

    out[w][p] = x(512 w - 64 + p),  x(i) = 0 if i < 0 else a[min(i, len - 1)],

and against hand-written rows for lengths around the window boundaries.  A
context taken from the wrong window, a zero- instead of last-sample pad, or
a context that is not reset would each fail one of them.
"""
import ctypes

import numpy as np
import pytest

import oracle
from scriptrs_amd import _lib
from scriptrs_amd.vad import VAD_INPUT_SAMPLES, vad_num_windows


def closed_form(a: np.ndarray) -> np.ndarray:
    n = (a.size + 511) // 512
    idx = 512 * np.arange(n, dtype=np.int64)[:, None] - 64 + np.arange(576, dtype=np.int64)[None, :]
    out = a[np.clip(idx, 0, a.size - 1)] if a.size else np.zeros((0, 576), np.float32)
    return np.where(idx < 0, np.float32(0), out).astype(np.float32)


@pytest.mark.parametrize("n", [0, 1, 2, 63, 64, 65, 448, 511, 512, 513, 575, 576, 1023, 1024, 1025, 16_000,
                               160_000, 240_001])
def test_oracle_matches_closed_form(n):
    a = np.random.default_rng(n).standard_normal(n).astype(np.float32)
    got = oracle.vad_frames(a)
    assert got.shape == (vad_num_windows(n), 576)
    assert np.array_equal(got, closed_form(a))


def test_hand_rows():
    a = np.arange(1, 1100, dtype=np.float32)  # 1099 samples: two full windows and one of 75
    got = oracle.vad_frames(a)
    assert got.shape == (3, 576)
    assert np.array_equal(got[0, :64], np.zeros(64, np.float32))
    assert np.array_equal(got[0, 64:], a[:512])
    assert np.array_equal(got[1, :64], a[448:512])
    assert np.array_equal(got[1, 64:], a[512:1024])
    assert np.array_equal(got[2, :64], a[960:1024])
    assert np.array_equal(got[2, 64:64 + 75], a[1024:])
    assert np.all(got[2, 64 + 75:] == a[-1])


def test_single_sample_repeats():
    got = oracle.vad_frames(np.array([0.25], np.float32))
    assert got.shape == (1, 576)
    assert np.all(got[0, :64] == 0) and np.all(got[0, 64:] == np.float32(0.25))


@pytest.mark.parametrize("n,w", [(0, 0), (1, 1), (511, 1), (512, 1), (513, 2), (57_600_000, 112_500),
                                 (460_800_000, 900_000), (-5, 0)])
def test_num_windows(n, w):
    assert vad_num_windows(n) == w
    assert VAD_INPUT_SAMPLES == 576


def test_vad_argument_errors_before_device():
    L = _lib.lib()
    buf = (ctypes.c_int16 * 1024)()
    out = (ctypes.c_float * (2 * 576 + 4))()
    vp = lambda b: ctypes.cast(b, ctypes.c_void_p)  # noqa: E731
    # bad pcm formats and widths
    for fmt, bits in ((1, 1), (1, 17), (2, 33), (7, 16)):
        assert L.sfe_vad_frames(None, vp(buf), fmt, bits, 1024, vp(out), 2, None) == _lib.SFE_INVALID_ARG
    # output too small: 1025 samples need 3 windows
    assert L.sfe_vad_frames(None, vp(buf), 1, 16, 1025, vp(out), 2, None) == _lib.SFE_INVALID_ARG
    assert "windows" in _lib.last_error()
    # negative length
    assert L.sfe_vad_frames(None, vp(buf), 1, 16, -1, vp(out), 2, None) == _lib.SFE_INVALID_ARG
    # misaligned output
    mis = ctypes.c_void_p(ctypes.addressof(out) + 4 if ctypes.addressof(out) % 16 == 0 else ctypes.addressof(out))
    if mis.value % 16:
        assert L.sfe_vad_frames(None, vp(buf), 1, 16, 1024, mis, 2, None) == _lib.SFE_INVALID_ARG
    # empty audio: nothing to do, like the reference's empty probability list
    assert L.sfe_vad_frames(None, None, 0, 32, 0, None, 0, None) == _lib.SFE_OK
