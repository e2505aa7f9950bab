"""Silero VAD model-input framing on the GPU.

Mirrors the framing half of the reference's VAD loop
(``process_coreml_vad``, src/long_form/vad.rs:62-99; constants
src/constants.rs:6-11): one model input of ``VAD_CONTEXT_SAMPLES +
VAD_WINDOW_SAMPLES`` = 576 samples per 512-sample window,
``[64 context | 512 window]``.  The model itself (CoreML) is outside this
library; ``SileroVadFramer.model_inputs`` returns the tensor the model's
per-window calls consume, in window order.
"""
from __future__ import annotations

import ctypes

from . import _lib
from .frontend import (InvalidModelOutput, ParakeetFeatureExtractor, _check, _dev_ptr, _pcm_format,
                       _stream_handle)

VAD_WINDOW_SAMPLES = 512
VAD_CONTEXT_SAMPLES = 64
VAD_INPUT_SAMPLES = VAD_WINDOW_SAMPLES + VAD_CONTEXT_SAMPLES


def vad_num_windows(length: int) -> int:
    """Windows the VAD loop runs for ``length`` samples:
    ``(0..len).step_by(512)`` (src/long_form/vad.rs:78), i.e. ceil(len / 512)."""
    return int(_lib.lib().sfe_vad_num_windows(int(length)))


class SileroVadFramer:
    """Builds the VAD model inputs of a device recording on ``device``.

    One instance per host thread, like the feature extractor (it owns an
    ``sfe_ctx``; calls on it are ordered after each other).
    """

    def __init__(self, device: int = 0):
        self._fe = ParakeetFeatureExtractor(device=device)
        self.device = device

    def close(self) -> None:
        self._fe.close()

    def model_inputs(self, recording, bits_per_sample: int | None = None, stream=None, out=None):
        """``[n_windows, 576]`` float32 device tensor of model inputs for a
        contiguous device recording (torch.float32, or integer PCM in
        torch.int16 / torch.int32 decoded as the WAV reader does,
        examples/transcribe_wav.rs:342-348).  Empty audio gives an empty
        tensor, as the reference returns no probabilities
        (src/long_form/vad.rs:67-69)."""
        import torch
        pcm, bits = _pcm_format(recording.dtype, bits_per_sample)
        n = vad_num_windows(recording.numel())
        if out is None:
            out = torch.empty((n, VAD_INPUT_SAMPLES), dtype=torch.float32, device=recording.device)
        elif out.dtype != torch.float32 or out.numel() < n * VAD_INPUT_SAMPLES:
            raise InvalidModelOutput("out must be a float32 tensor of at least n_windows x 576 elements")
        if n == 0:
            return out
        rec_ptr, out_ptr = _dev_ptr(recording), _dev_ptr(out)  # checked before any device work
        rc = _lib.lib().sfe_vad_frames(self._fe._handle(), rec_ptr, pcm, bits, recording.numel(), out_ptr,
                                       out.numel() // VAD_INPUT_SAMPLES, _stream_handle(stream))
        _check(rc)
        return out
