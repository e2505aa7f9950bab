"""C-ABI host logic without a GPU: symbols, planner, tables, error mapping."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle
from oracle import planner
from scriptrs_amd import (AudioTooLong, ChunkPreparer, EmptyAudio, InvalidModelOutput, OverlapChunkConfig,
                          ParakeetFeatureExtractor, SampleRange, TranscriptionConfig, build_fast_execution_plan,
                          build_tables, num_frames, parallel_worker_count)
from scriptrs_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "scriptrs_fe.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sfe_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = header_functions()
    assert len(names) >= 16
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(_lib.EXPORTS)


def test_product_library_has_no_stamps():
    """sfe_debug_stamps is only live in the measurement build; the product
    library refuses it without touching the device."""
    L = _lib.lib()
    assert L.sfe_debug_stamps(None, 0) == _lib.SFE_INVALID_ARG
    assert "SFE_TIMESTAMPS" in _lib.last_error()


def test_measurement_build_exports_the_same_abi():
    from scriptrs_amd import stamps
    if not os.path.exists(stamps.TS_LIB):
        pytest.skip("measurement build not present")
    T = ctypes.CDLL(stamps.TS_LIB)
    for n in header_functions():
        assert hasattr(T, n), n


def test_config_defaults_match_reference():
    c = _lib.SfeConfig()
    _lib.lib().sfe_config_default(ctypes.byref(c))
    py = TranscriptionConfig()
    assert (c.sample_rate, c.feature_size, c.n_fft, c.win_length, c.hop_length, c.max_audio_samples,
            c.samples_per_encoder_frame) == (16000, 128, 512, 400, 160, 240000, 1280)
    assert abs(c.preemphasis - 0.97) < 1e-7
    assert py.max_feature_frames() == 1501 and py.max_duration_seconds() == 15.0
    o = _lib.SfeOverlapConfig()
    _lib.lib().sfe_overlap_config_default(ctypes.byref(o))
    assert (o.overlap_seconds, o.context_samples, o.max_model_samples) == (2.0, 1280, 240000)


@pytest.mark.parametrize("n", [1, 159, 160, 161, 16000, 240000, 57_600_000])
def test_num_frames(n):
    assert num_frames(n) == n // 160 + 1 == oracle.num_frames(n)


def test_tables_bit_exact_with_oracle():
    w, fb = build_tables()
    assert np.array_equal(w, oracle.hann_window())
    assert np.array_equal(fb, oracle.mel_filterbank())
    w2, fb2 = build_tables(TranscriptionConfig(sample_rate=22050))
    assert np.array_equal(fb2, oracle.mel_filterbank(512, 128, 22050))


def test_mel_schedule_by_sample_rate():
    """The mel contraction schedule sfe_create takes for each sample rate:
    the default one at 16, 22.05 and 24 kHz (and some rates near them); the
    wider one (50% more matrix steps) at 8, 11.025, 32, 44.1, 48 and 96 kHz;
    one or the other for every rate from 3.5 to 107 kHz tried here; none
    (SFE_INVALID_ARG) where no schedule fits the Slaney filterbank, and for
    another shape."""
    import ctypes
    from scriptrs_amd import _lib

    def schedule(**kw):
        c = TranscriptionConfig(**kw).to_c()
        return _lib.lib().sfe_debug_mel_schedule(ctypes.byref(c))

    assert [schedule(sample_rate=sr) for sr in (16000, 22050, 24000)] == [0, 0, 0]
    assert [schedule(sample_rate=sr) for sr in (8000, 11025, 32000, 44100, 48000, 96000)] == [1] * 6
    rates = list(range(3500, 8000, 500)) + list(range(8000, 107001, 1000)) + [11025, 44100, 88200]
    assert all(schedule(sample_rate=sr) in (0, 1) for sr in rates)
    for sr in (2500, 3000, 108000):
        assert schedule(sample_rate=sr) == -1
        assert "band table" in _lib.last_error()
    assert schedule(n_fft=1024) == -1 and "unsupported frontend shape" in _lib.last_error()


LENGTHS = [0, 1, 1279, 1280, 95_999, 96_000, 238_079, 238_080, 238_081, 240_000, 240_001, 444_160,
           444_161, 650_240, 1_000_003, 57_600_000, 460_800_000]


@pytest.mark.parametrize("n", LENGTHS)
def test_library_planner_matches_oracle_planner(n):
    got = build_fast_execution_plan(n)
    want = planner.build_fast_execution_plan(n)
    assert [(t.audio_start, t.audio_end, t.global_sample_offset, t.context_samples) for t in got] == \
        [(t.audio_start, t.audio_end, t.global_sample_offset, t.context_samples) for t in want]


@pytest.mark.parametrize("cfg", [(2.0, 1280, 240000), (0.5, 0, 100000), (30.0, 1280, 240000), (1.0, 5000, 48000),
                                 (0.0, 1280, 2000), (-1.0, 1280, 240000)])
def test_planner_configs(cfg):
    c = OverlapChunkConfig(*cfg)
    o = planner.OverlapChunkConfig(*cfg)
    for n in (0, 1, 5000, 123_457, 2_000_000):
        got = c.tasks(n)
        want = [t for t in _oracle_tasks(o, n)]
        assert [(t.audio_start, t.audio_end, t.global_sample_offset, t.context_samples) for t in got] == want


def test_planner_random_configs_match_oracle():
    """Property test over random planner configs (overlap seconds, context
    and model-sample limits, including the saturating and degenerate ends)
    and recording lengths: the library's task table equals the restated
    planner's (src/long_form/planner.rs:94-137, src/long_form.rs:566-582)."""
    from hypothesis import given, settings, strategies as st

    @settings(max_examples=300, deadline=None, derandomize=True)
    @given(ov=st.floats(-10.0, 100.0, allow_nan=False), ctx=st.integers(0, 60_000),
           mx=st.integers(0, 1_500_000), n=st.integers(0, 20_000_000))
    def check(ov, ctx, mx, n):
        got = OverlapChunkConfig(ov, ctx, mx).tasks(n)
        want = _oracle_tasks(planner.OverlapChunkConfig(ov, ctx, mx), n)
        assert [(t.audio_start, t.audio_end, t.global_sample_offset, t.context_samples) for t in got] == want

    check()


def _oracle_tasks(o, n):
    out = []
    for s, e in o.plan(0, n):
        cs = max(s - o.context_samples, 0)
        out.append((cs, e, s, s - cs))
    return out


def test_plan_sample_range():
    got = OverlapChunkConfig().plan(SampleRange(0, 600_000))
    assert len(got) > 1 and got[1].start < got[0].end  # src/long_form/planner.rs:376-385


def test_worker_count():
    assert [parallel_worker_count(*a) for a in [(0, 4), (1, 4), (3, 0), (3, 2), (3, 8)]] == [1, 1, 1, 2, 3]


def test_plan_buffer_too_small_reports_count():
    c = OverlapChunkConfig()._c()
    n = ctypes.c_int32(0)
    arr = (_lib.SfeChunk * 2)()
    rc = _lib.lib().sfe_plan_fast(ctypes.byref(c), 57_600_000, arr, 2, ctypes.byref(n))
    assert rc == _lib.SFE_INVALID_ARG and n.value == 280
    assert arr[0].audio_end == 238_080 and arr[1].audio_start == 206_080 - 1280
    assert "too small" in _lib.last_error()


# ---- errors map onto the reference's TranscriptionError without touching a GPU ----

def test_empty_audio():
    with pytest.raises(EmptyAudio):
        ParakeetFeatureExtractor().extract(np.zeros(0, np.float32))
    with pytest.raises(EmptyAudio):
        ChunkPreparer().prepare([])


def test_audio_too_long():
    with pytest.raises(AudioTooLong) as e:
        ChunkPreparer().prepare(np.zeros(240_001, np.float32))
    assert e.value.max_seconds == 15.0 and abs(e.value.actual_seconds - 15.0000625) < 1e-9
    assert "actual=15.00s max=15.00s" in str(e.value)


def test_c_abi_argument_errors():
    L = _lib.lib()
    assert L.sfe_extract(None, None, 0, None, 0) == _lib.SFE_EMPTY_AUDIO
    assert L.sfe_extract(None, (ctypes.c_float * 4)(), 4, (ctypes.c_float * 512)(), 512) == _lib.SFE_INVALID_ARG
    assert "null context" in _lib.last_error()
    fo = (ctypes.c_int64 * 3)()
    off = (ctypes.c_int64 * 3)(0, 10, 5)
    assert L.sfe_extract_batch(None, ctypes.c_void_p(16), off, 2, 0, ctypes.c_void_p(16), fo, None) == \
        _lib.SFE_INVALID_ARG
    assert "non-decreasing" in _lib.last_error()
    bad = _lib.SfeConfig()
    L.sfe_config_default(ctypes.byref(bad))
    bad.n_fft = 1024
    ctx = ctypes.c_void_p()
    assert L.sfe_create(ctypes.byref(bad), 0, ctypes.byref(ctx)) == _lib.SFE_INVALID_ARG
    assert "specialised" in _lib.last_error()


def test_unsupported_dtype_rejected_before_device():
    with pytest.raises(InvalidModelOutput):
        from scriptrs_amd.frontend import _dtype_code
        _dtype_code("f16")


def _rn32(x):
    """Exact rounding of a rational to float32 (nearest, ties to even)."""
    from fractions import Fraction
    c = np.float32(float(x))
    best = None
    for v in (np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))):
        key = (abs(Fraction(float(v)) - x), int(np.float32(v).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, np.float32(v))
    return best[1]


def _residual_div(v, scale, recip):
    """The kernel's PCM decode: q = RN(v r); RN(q + r RN(v - scale q)) with
    both steps fused multiply-adds (exact products, one rounding each)."""
    from fractions import Fraction
    a, s, r = np.float32(v), np.float32(scale), np.float32(recip)
    q = np.float32(a * r)
    e = _rn32(Fraction(float(a)) - Fraction(float(s)) * Fraction(float(q)))
    return _rn32(Fraction(float(q)) + Fraction(float(e)) * Fraction(float(r)))


def test_pcm_decode_is_correctly_rounded_for_every_int32_holding_16_bits():
    """The int32-container decode (Markstein residual step) equals the
    reference's f32 division value as f32 / 32767.0
    (examples/transcribe_wav.rs:342-348) for all 65536 16-bit inputs."""
    scale = np.float32(32767.0)
    recip = np.float32(1.0) / scale
    v = np.arange(-32768, 32768, dtype=np.float32)
    want = v / scale  # numpy's f32 division is correctly rounded
    q = v * recip
    # fast exact screen: where q already equals the quotient nothing can go wrong
    todo = np.nonzero(q != want)[0]
    for i in todo:
        assert _residual_div(v[i], scale, recip) == want[i], int(v[i])


@pytest.mark.parametrize("bits", range(2, 17))
def test_int16_decode_is_correctly_rounded_for_every_value(bits):
    """The int16-container decode RN_f32(RN_f64(v * RN_f64(1 / scale))) equals
    correctly rounded f32 division for every int16 value at every width (a
    plain f32 multiply by RN_f32(1 / scale) would not: it is wrong for
    thousands of values at most widths)."""
    scale = np.float32((1 << (bits - 1)) - 1)
    v = np.arange(-32768, 32768, dtype=np.int64)
    want = v.astype(np.float32) / scale
    got = (v.astype(np.float64) * (1.0 / np.float64(scale))).astype(np.float32)
    assert np.array_equal(got, want)
    if bits > 2:
        assert np.count_nonzero(v.astype(np.float32) * (np.float32(1.0) / scale) != want) > 0


def test_pcm_decode_24_bit_sample():
    rng = np.random.default_rng(5)
    scale = np.float32(float((1 << 23) - 1))
    recip = np.float32(1.0) / scale
    vals = rng.integers(-(1 << 23), 1 << 23, 4000).astype(np.float32)
    for v in vals:
        assert _residual_div(v, scale, recip) == np.float32(v) / scale, v


def test_pcm_argument_errors_before_device():
    from scriptrs_amd._lib import SfeChunk
    L = _lib.lib()
    t = (SfeChunk * 1)(SfeChunk(0, 1000, 0, 0))
    fo = (ctypes.c_int64 * 2)()
    buf = (ctypes.c_int16 * 1000)()
    for fmt, bits in ((1, 1), (1, 17), (2, 33), (7, 16)):
        rc = L.sfe_extract_chunks_pcm(None, ctypes.cast(buf, ctypes.c_void_p), fmt, bits, 1000, t, 1, 0,
                                      ctypes.cast(buf, ctypes.c_void_p), fo, None)
        assert rc == _lib.SFE_INVALID_ARG, (fmt, bits)


def test_build_rejects_mfma_destination_overlapping_its_operands():
    from scriptrs_amd.build import mfma_operand_overlaps
    asm = ("\tv_mfma_f32_4x4x1_16b_f32 v[46:49], v49, v57, v[62:65]\n"   # dst holds its own A operand
           "\tv_mfma_f32_4x4x1_16b_f32 v[50:53], v1, v51, v[50:53]\n"    # dst holds its own B operand
           "\tv_mfma_f32_4x4x1_16b_f32 v[46:49], v50, v57, v[46:49]\n"   # in-place accumulate: fine
           "\tv_mfma_f32_4x4x1_16b_f32 a[0:3], v2, v3, a[0:3]\n")        # AGPR accumulator: fine
    bad = mfma_operand_overlaps(asm)
    assert len(bad) == 2 and "v49" in bad[0] and "v51" in bad[1]


def test_build_reads_spill_counts_from_kernel_metadata():
    from scriptrs_amd.build import vgpr_spills
    meta = ("    .name:           _ZN3sfe4kernAEv\n    .sgpr_count:     66\n    .vgpr_count:     168\n"
            "    .vgpr_spill_count: 7\n  - .args:\n    .name:           _ZN3sfe4kernBEv\n"
            "    .vgpr_count:     88\n    .vgpr_spill_count: 0\n")
    assert vgpr_spills(meta) == {"_ZN3sfe4kernAEv": 7, "_ZN3sfe4kernBEv": 0}


def test_build_counts_lane_masked_loops_per_kernel():
    from scriptrs_amd.build import lane_masked_loops
    asm = ("_ZN3sfe4kernAEv:\n\ts_andn2_b64 exec, exec, s[4:5]\n\ts_cbranch_execnz .LBB0_1\n"
           "\ts_andn2_b64 exec, exec, s[8:9]\n.Lfunc_end0:\n"
           "_ZN3sfe4kernBEv:\n\ts_cbranch_scc1 .LBB1_1\n.Lfunc_end1:\n")
    assert lane_masked_loops(asm, "kernA") == 2
    assert lane_masked_loops(asm, "kernB") == 0
    with pytest.raises(RuntimeError):
        lane_masked_loops(asm, "kernC")


def _closed_form_plan(n, chunk=238_080, stride=206_080, ctx=1280, hop=160):
    """Count, sum of task lengths and sum of frame counts of the fast plan,
    in closed form: task i covers [max(i*stride - ctx, 0), min(i*stride +
    chunk, n)) and the plan ends with the first task that reaches n, so
    count = ceil((n - chunk) / stride) + 1 (1 when n <= chunk).  Lengths:
    the first task has no context; middle tasks are chunk + ctx; the last
    runs to n (src/long_form/planner.rs:124-137, src/long_form.rs:566-582)."""
    if n <= 0:
        return 0, 0, 0
    count = 1 if n <= chunk else -(-(n - chunk) // stride) + 1
    lens = []
    for i in range(count):
        lo, hi = max(i * stride - ctx, 0), min(i * stride + chunk, n)
        lens.append(hi - lo)
    return count, sum(lens), sum(L // hop + 1 for L in lens)


@pytest.mark.parametrize("n", [1, 238_080, 238_081, 444_160, 444_161, 1_000_003, 28_800_000, 57_600_000,
                               460_800_000])
def test_planner_matches_closed_form(n):
    """The library's plan against the closed form above, without the
    restated planner.  The constants follow from the reference's defaults:
    chunk = (240000 - 1280 - 160) // 1280 * 1280 = 238080, overlap =
    min(32000, 119040) // 1280 * 1280 = 32000, stride = 206080."""
    assert (240_000 - 1280 - 160) // 1280 * 1280 == 238_080
    assert min(2 * 16_000, 238_080 // 2) // 1280 * 1280 == 32_000 and 238_080 - 32_000 == 206_080
    t = build_fast_execution_plan(n)
    got = (len(t), sum(x.audio_end - x.audio_start for x in t), sum((x.audio_end - x.audio_start) // 160 + 1 for x in t))
    assert got == _closed_form_plan(n)
    if n == 57_600_000:
        assert got == (280, 66_885_120, 418_312)
    if n == 460_800_000:
        assert got == (2236, 535_180_800, 3_347_116)
    # every task starts on the stride grid and the last one ends at n
    assert [x.global_sample_offset for x in t] == [i * 206_080 for i in range(len(t))]
    assert t[-1].audio_end == n and all(x.context_samples == x.global_sample_offset - x.audio_start for x in t)


def _markstein_f64(v32, scale, recip):
    """Vectorised kernel decode for f32 inputs: q = RN32(v r); e = RN32(v -
    scale q) (scale q is exact in f64 and v - scale q is exact by Sterbenz);
    RN32(q + e r) with e r exact in f64.  The sum q + e r is rounded twice (f64
    then f32), so values whose f64 sum lies within an f64 ulp of an f32
    rounding midpoint are returned in `hard` for an exact check."""
    q = (v32 * recip).astype(np.float32)
    e = (v32.astype(np.float64) - np.float64(scale) * q.astype(np.float64)).astype(np.float32)
    s64 = q.astype(np.float64) + e.astype(np.float64) * np.float64(recip)
    out = s64.astype(np.float32)
    # f32 midpoints around the result
    up = np.nextafter(out, np.float32(np.inf)).astype(np.float64)
    dn = np.nextafter(out, np.float32(-np.inf)).astype(np.float64)
    o64 = out.astype(np.float64)
    mids = np.stack([(o64 + up) / 2, (o64 + dn) / 2])
    near = (np.abs(mids - s64[None]) <= np.spacing(np.abs(s64))[None] * 2).any(0)
    return out, np.nonzero(near)[0]


def test_pcm_decode_is_correctly_rounded_for_every_24_bit_value():
    """The int32-container decode at 24 bits, for all 2^24 values, equals the
    reference's f32 division value as f32 / 8388607.0
    (examples/transcribe_wav.rs:342-348)."""
    scale = np.float32((1 << 23) - 1)
    recip = np.float32(1.0) / scale
    v = np.arange(-(1 << 23), 1 << 23, dtype=np.int64).astype(np.float32)
    want = v / scale
    got, hard = _markstein_f64(v, scale, recip)
    for i in hard:
        got[i] = _residual_div(v[i], scale, recip)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("bits", range(25, 33))
def test_pcm_decode_edge_values_at_widths_25_to_32(bits):
    """Widths past 24 bits: the divisor ((1 << (bits-1)) - 1) as f32 and the
    sample value as f32 are both rounded first, as the reference computes
    them; the decode equals correctly rounded f32 division at the edges."""
    scale = np.float32(float((1 << (bits - 1)) - 1))
    recip = np.float32(1.0) / scale
    top = (1 << (bits - 1)) - 1
    ints = [-(1 << (bits - 1)), -top, -(1 << 24) - 1, -(1 << 24), -1, 0, 1, (1 << 24) - 1, 1 << 24, (1 << 24) + 1,
            top - 1, top]
    rng = np.random.default_rng(bits)
    ints += rng.integers(-(1 << (bits - 1)), 1 << (bits - 1), 200).tolist()
    for iv in ints:
        v = np.float32(iv)
        assert _residual_div(v, scale, recip) == v / scale, (bits, iv)


def test_max_feature_frames_null_and_zero_hop():
    L = _lib.lib()
    assert L.sfe_max_feature_frames(None) == 1501
    c = _lib.SfeConfig()
    L.sfe_config_default(ctypes.byref(c))
    c.hop_length = 0
    assert L.sfe_max_feature_frames(ctypes.byref(c)) == 240_000 // 160 + 1


def test_tuning_calls_reject_null_context():
    L = _lib.lib()
    assert L.sfe_set_frame_sharing(None, 1) == _lib.SFE_INVALID_ARG
    assert L.sfe_set_timing(None, 1) == _lib.SFE_INVALID_ARG
