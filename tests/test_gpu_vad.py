"""GPU parity of the VAD model-input framing kernel against the CPU oracle
(the reference's loop, src/long_form/vad.rs:62-99).  The framing is pure
data movement plus the PCM decode, so the bar is bit-exact."""
import numpy as np
import pytest

import oracle
from scriptrs_amd import SileroVadFramer, synth

pytestmark = pytest.mark.gpu


def _flush(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def framer():
    f = SileroVadFramer()
    yield f
    f.close()


@pytest.mark.parametrize("n", [1, 3, 63, 64, 511, 512, 513, 1025, 8192, 160_000, 240_001])
def test_f32_lengths(framer, n):
    import torch
    _flush(f"case: vad f32 length {n}")
    a = synth.sinusoids(n, 500 + n)
    got = framer.model_inputs(torch.from_numpy(a).cuda())
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), oracle.vad_frames(a))


def test_f32_recording_at_4_byte_offset(framer):
    """A recording that starts 4 bytes past a 16-byte boundary (a slice)."""
    import torch
    _flush("case: vad f32 offset slice")
    a = synth.speech_like(100_003, 5)
    dev = torch.from_numpy(a).cuda()[1:]
    assert dev.data_ptr() % 16 == 4
    got = framer.model_inputs(dev)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), oracle.vad_frames(a[1:]))


def test_empty_audio(framer):
    import torch
    _flush("case: vad empty")
    got = framer.model_inputs(torch.empty(0, dtype=torch.float32, device="cuda"))
    assert tuple(got.shape) == (0, 576)


def test_pcm16_equals_f32_of_decoded(framer):
    import torch
    _flush("case: vad pcm16")
    x = synth.speech_like(1_500_017, 41)
    pcm = np.clip(np.round(x * 32767.0), -32768, 32767).astype(np.int16)
    dec = pcm.astype(np.float32) / np.float32(32767.0)
    got = framer.model_inputs(torch.from_numpy(pcm).cuda())
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), oracle.vad_frames(dec))


def test_pcm12_in_int16_equals_f32_of_decoded(framer):
    """12-bit samples in int16 containers (scale 2047), including values
    outside the 12-bit range, which the reference's formula also divides."""
    import torch
    _flush("case: vad pcm12 in int16")
    pcm = np.random.default_rng(44).integers(-32768, 32768, 300_001).astype(np.int16)
    dec = pcm.astype(np.float32) / np.float32(2047.0)
    got = framer.model_inputs(torch.from_numpy(pcm).cuda(), bits_per_sample=12)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), oracle.vad_frames(dec))


def test_pcm24_in_int32_equals_f32_of_decoded(framer):
    import torch
    _flush("case: vad pcm24 in int32")
    x = synth.speech_like(700_001, 43)
    pcm = np.clip(np.round(x * 8388607.0), -8388608, 8388607).astype(np.int32)
    dec = pcm.astype(np.float32) / np.float32(8388607.0)
    got = framer.model_inputs(torch.from_numpy(pcm).cuda(), bits_per_sample=24)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), oracle.vad_frames(dec))


def test_reused_output_then_smaller_input(framer):
    """A second, shorter call into the same buffer writes exactly its rows."""
    import torch
    _flush("case: vad reused output")
    a = synth.sinusoids(300_000, 9)
    b = synth.sinusoids(70_001, 10)
    out = torch.full((600, 576), 7.0, dtype=torch.float32, device="cuda")
    framer.model_inputs(torch.from_numpy(a).cuda(), out=out)
    framer.model_inputs(torch.from_numpy(b).cuda(), out=out)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    nb = (b.size + 511) // 512
    assert np.array_equal(o[:nb], oracle.vad_frames(b))
    assert np.array_equal(o[nb:586], oracle.vad_frames(a)[nb:])
    assert np.all(o[586:] == 7.0)


def test_one_hour_full_size(framer):
    """The 1 h long-form recording (57.6 M samples, 112,500 windows)."""
    import torch
    _flush("case: vad 1 h full size")
    a = synth.speech_like(57_600_000, 3)
    got = framer.model_inputs(torch.from_numpy(a).cuda())
    torch.cuda.synchronize()
    assert tuple(got.shape) == (112_500, 576)
    assert np.array_equal(got.cpu().numpy(), oracle.vad_frames(a))
