"""Independent float64 numpy restatement of the log-mel front end.

Written from the mathematics of src/frontend.rs:104-241 rather than from the
C oracle: vectorised framing, ``numpy.fft.rfft`` (a library FFT) and a dense
matmul, all in float64.  Used to pin the oracle (and the GPU path) against a
third implementation whose rounding error is ~1e-13.
"""
from __future__ import annotations

import numpy as np

N_FFT, WIN, HOP, N_MELS, SR = 512, 400, 160, 128, 16000


def hann_window_f32(win: int = WIN) -> np.ndarray:
    """The reference's window with float32 operations.  The cosine is the C
    library's cosf, which is what Rust's f32::cos calls on Linux (glibc's
    cosf is not correctly rounded everywhere; numpy's float32 cos differs
    from it by an ulp at a few taps)."""
    import ctypes
    import ctypes.util
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.cosf.argtypes = [ctypes.c_float]
    libm.cosf.restype = ctypes.c_float
    n = np.arange(win, dtype=np.float32)
    arg = (np.float32(2.0) * np.float32(np.pi)) * n / (np.float32(win) - np.float32(1.0))
    c = np.array([libm.cosf(float(v)) for v in arg], np.float32)
    return (np.float32(0.5) - np.float32(0.5) * c).astype(np.float32)


def slaney_mel_filterbank(n_fft: int = N_FFT, n_mels: int = N_MELS, sr: int = SR) -> np.ndarray:
    """librosa-style Slaney filterbank (norm='slaney', htk=False), float64."""
    f_sp = 200.0 / 3.0
    min_log_hz, logstep = 1000.0, np.log(6.4) / 27.0
    min_log_mel = min_log_hz / f_sp

    def hz2mel(f):
        f = np.asarray(f, np.float64)
        return np.where(f >= min_log_hz, min_log_mel + np.log(np.maximum(f, 1e-300) / min_log_hz) / logstep, f / f_sp)

    def mel2hz(m):
        m = np.asarray(m, np.float64)
        return np.where(m >= min_log_mel, min_log_hz * np.exp(logstep * (m - min_log_mel)), f_sp * m)

    fftfreqs = np.linspace(0, sr / 2, n_fft // 2 + 1)
    mel_f = mel2hz(np.linspace(hz2mel(0.0), hz2mel(sr / 2.0), n_mels + 2))
    fdiff = np.diff(mel_f)
    ramps = mel_f[:, None] - fftfreqs[None, :]
    lower = -ramps[:-2] / fdiff[:-1, None]
    upper = ramps[2:] / fdiff[1:, None]
    w = np.maximum(0.0, np.minimum(lower, upper))
    return w * (2.0 / (mel_f[2:n_mels + 2] - mel_f[:n_mels]))[:, None]


def logmel_raw(audio: np.ndarray, window=None, fb=None, sr: int = SR, preemph: float = 0.97) -> np.ndarray:
    """ln(mel + 2^-24), [128, T] float64, before normalisation (sample rate
    sr sets the filterbank's band edges; preemph the preemphasis
    coefficient, an f32 value as in the reference's config)."""
    x = np.asarray(audio, np.float64)
    if x.size == 0:
        raise ValueError("EmptyAudio")
    w = (hann_window_f32() if window is None else window).astype(np.float64)
    fb = slaney_mel_filterbank(sr=sr) if fb is None else np.asarray(fb, np.float64)
    y = np.empty_like(x)
    y[0] = x[0]
    y[1:] = x[1:] - np.float64(np.float32(preemph)) * x[:-1]
    padded = np.concatenate([np.zeros(N_FFT // 2), y, np.zeros(N_FFT // 2)])
    T = x.size // HOP + 1
    idx = np.arange(T)[:, None] * HOP + np.arange(WIN)[None, :]
    frames = padded[idx] * w[None, :]
    spec = np.abs(np.fft.rfft(frames, n=N_FFT, axis=1)) ** 2      # [T, 257]
    mel = spec @ fb.T                                             # [T, 128]
    return np.log(mel + 2.0 ** -24).T


def normalize(raw: np.ndarray) -> np.ndarray:
    """Per-feature (x - mean) / (std + 1e-5), variance over T - 1."""
    T = raw.shape[1]
    mean = raw.mean(axis=1, keepdims=True)
    var = ((raw - mean) ** 2).sum(axis=1, keepdims=True) / (T - 1) if T > 1 else np.full((raw.shape[0], 1), np.nan)
    return (raw - mean) / (np.sqrt(var) + 1e-5)


def extract(audio: np.ndarray, sr: int = SR, preemph: float = 0.97) -> np.ndarray:
    """Feature-major [128, T] float64 normalised log-mel."""
    return normalize(logmel_raw(audio, sr=sr, preemph=preemph))


# An element is near the noise floor when its float64 mel energy is at most
# this fraction of its frame's energy (sum of |X_k|^2).  f32 FFT rounding is
# of order u log2(N) ||frame|| per bin, so only such elements can move by
# more than the 1e-4 / 1e-3 bar (observed: at most 1.6e-8 of the frame
# energy on the speech-like workloads).
NEAR_GUARD_RATIO = 1e-6
# The envelope never widens an element by more than this (normalised units;
# observed maximum 3.4e-3).
ENV_CAP = 5e-3


def _frames_f64(audio: np.ndarray, preemph: float = 0.97):
    x = np.asarray(audio, np.float64)
    w = hann_window_f32().astype(np.float64)
    y = np.empty_like(x)
    y[0] = x[0]
    y[1:] = x[1:] - np.float64(np.float32(preemph)) * x[:-1]
    padded = np.concatenate([np.zeros(N_FFT // 2), y, np.zeros(N_FFT // 2)])
    T = x.size // HOP + 1
    idx = np.arange(T)[:, None] * HOP + np.arange(WIN)[None, :]
    return padded[idx] * w[None, :]


def near_guard(audio: np.ndarray, sr: int = SR, preemph: float = 0.97) -> np.ndarray:
    """[128, T] bool: elements whose float64 mel energy is at most
    NEAR_GUARD_RATIO of their frame's energy (frames of zero energy are
    exact in every implementation and are not near-guard)."""
    frames = _frames_f64(audio, preemph)
    P = np.abs(np.fft.rfft(frames, n=N_FFT, axis=1)) ** 2
    mel = P @ slaney_mel_filterbank(sr=sr).T
    E = P.sum(1, keepdims=True)
    return ((mel <= NEAR_GUARD_RATIO * E) & (E > 0)).T


def f32_noise_envelope(audio: np.ndarray, parts: bool = False, sr: int = SR, preemph: float = 0.97):
    """Per-element scale of the rounding noise any f32 FFT-based implementation
    of the front end carries, in normalised units, [128, T].

    A radix-2/4 f32 FFT of a frame r has per-bin absolute error of order
    u * log2(N) * ||r||_2 (u = 2^-24), independent of the bin.  That moves
    |X_k|^2 by about 2|X_k| dX + dX^2, the mel value by the filter-weighted
    sum of that, the log by dmel / (mel + 2^-24), and the normalised output
    by that divided by the row's std.  A floor of 4u*|raw| covers the f32 log
    and elementwise rounding.  This element term is zero except on near-guard
    elements (near_guard) and at most ENV_CAP.

    The row term: a row's mean and std are taken over its near-guard
    elements too, so their noise dx (the element term in raw units) shifts
    every normalised value z of the row by up to (mean(dx) + |z| *
    mean(|x - mean| dx) / std) / std (first order in dx: out = (x - mean) /
    std).  It is zero in rows without near-guard elements and at most
    ENV_CAP.  Only elements with a non-zero envelope may be widened past the
    flat bar.  Returns elem + row, or (elem, row) with parts."""
    frames = _frames_f64(audio, preemph)
    fb = slaney_mel_filterbank(sr=sr)
    T = frames.shape[0]
    X = np.abs(np.fft.rfft(frames, n=N_FFT, axis=1))
    u = 2.0 ** -24
    dX = u * np.log2(N_FFT) * np.sqrt((frames ** 2).sum(1, keepdims=True))
    dP = 2.0 * X * dX + dX ** 2
    mel = (X ** 2) @ fb.T
    raw = np.log(mel + 2.0 ** -24)
    d_raw = (dP @ fb.T) / (mel + 2.0 ** -24) + 4 * u * np.abs(raw)
    std = raw.std(axis=0, ddof=1, keepdims=True) if T > 1 else np.ones((1, raw.shape[1]))
    E = (X ** 2).sum(1, keepdims=True)
    near = (mel <= NEAR_GUARD_RATIO * E) & (E > 0)
    with np.errstate(divide="ignore", invalid="ignore"):
        elem = np.where(near, np.minimum(d_raw / std, ENV_CAP), 0.0)
        row = np.zeros_like(elem)
        if T > 1:
            dx = elem * std  # raw units
            dev = np.abs(raw - raw.mean(axis=0, keepdims=True))
            dm = dx.mean(axis=0, keepdims=True)
            ds = (dev * dx).mean(axis=0, keepdims=True) / std
            row = np.where(dx.any(axis=0, keepdims=True), np.minimum((dm + dev / std * ds) / std, ENV_CAP), 0.0)
    elem = np.nan_to_num(elem, nan=0.0)
    row = np.nan_to_num(row, nan=0.0)
    return (elem.T, row.T) if parts else (elem + row).T
