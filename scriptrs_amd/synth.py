"""Seeded synthetic audio for the five benchmark workloads.

Generators (numpy PCG64, so the same seed gives the same samples on any host):
  * ``sinusoids``  -- 3 sinusoids, f ~ U(100, 4000) Hz, a ~ U(0.1, 0.3),
    plus N(0, 0.05^2) noise, clipped to [-1, 1]          (configs 1, 2, 4)
  * ``speech_like`` -- 200 ms bursts of 300-3400 Hz band-limited noise,
    4 Hz amplitude modulation, 30% of the bursts replaced by digital silence
    (configs 3, 5)
"""
from __future__ import annotations

import numpy as np

SR = 16_000


def sinusoids(n: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    f = rng.uniform(100.0, 4000.0, 3)
    a = rng.uniform(0.1, 0.3, 3)
    t = np.arange(n, dtype=np.float64) / SR
    x = (a[:, None] * np.sin(2.0 * np.pi * f[:, None] * t[None, :])).sum(0)
    x += rng.normal(0.0, 0.05, n)
    return np.clip(x, -1.0, 1.0).astype(np.float32)


def dense_batch(batch: int, n: int, seed: int) -> np.ndarray:
    """[batch, n] of ``sinusoids`` with per-clip seed ``seed + i``."""
    return np.stack([sinusoids(n, seed + i) for i in range(batch)])


def ragged_lengths(count: int, seed: int, lo: int = 16_000, hi: int = 320_000) -> np.ndarray:
    """Clip lengths uniform on [lo, hi] samples (1-20 s)."""
    return np.random.default_rng(seed).integers(lo, hi + 1, count).astype(np.int64)


def ragged_batch(count: int, seed: int):
    """Flat buffer + offsets[count+1] of ``sinusoids`` clips with seeded lengths."""
    lens = ragged_lengths(count, seed)
    off = np.zeros(count + 1, np.int64)
    off[1:] = np.cumsum(lens)
    flat = np.empty(int(off[-1]), np.float32)
    for i in range(count):
        flat[off[i]:off[i + 1]] = sinusoids(int(lens[i]), seed + 1 + i)
    return flat, off


_BURST = SR // 5  # 200 ms


def _bandpass_bank(rng: np.random.Generator, nbursts: int) -> np.ndarray:
    """nbursts x 200 ms of white noise band-limited to 300-3400 Hz by an FFT mask
    with 50 Hz raised-cosine skirts (so leakage stays above the log guard)."""
    noise = rng.standard_normal((nbursts, _BURST))
    spec = np.fft.rfft(noise, axis=1)
    f = np.fft.rfftfreq(_BURST, 1.0 / SR)
    mask = np.clip((f - 250.0) / 100.0, 0.0, 1.0) * np.clip((3450.0 - f) / 100.0, 0.0, 1.0)
    mask = 0.5 - 0.5 * np.cos(np.pi * mask)
    out = np.fft.irfft(spec * mask, n=_BURST, axis=1)
    out /= out.std(axis=1, keepdims=True) + 1e-12
    return out


def speech_like(n: int, seed: int, block_bursts: int = 4096) -> np.ndarray:
    """Speech-like recording of n samples (float32), generated blockwise."""
    rng = np.random.default_rng(seed)
    out = np.empty(n, np.float32)
    env_t = np.arange(_BURST, dtype=np.float64) / SR
    env = 0.5 - 0.5 * np.cos(2.0 * np.pi * 4.0 * env_t)  # 4 Hz AM, zero at burst edges
    pos = 0
    while pos < n:
        nb = min(block_bursts, (n - pos + _BURST - 1) // _BURST)
        bursts = _bandpass_bank(rng, nb) * env[None, :]
        gain = rng.uniform(0.05, 0.3, nb)
        silent = rng.random(nb) < 0.3
        gain[silent] = 0.0
        block = (bursts * gain[:, None]).reshape(-1)
        take = min(block.size, n - pos)
        out[pos:pos + take] = block[:take]
        pos += take
    return out
