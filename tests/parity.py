"""The GPU-vs-oracle parity criterion, shared by the tests (through
conftest.py) and __graft_entry__.smoke()."""

# Parity bar for normalised log-mel (north_star): 1e-4 absolute + 1e-3 relative.
ATOL = 1e-4
RTOL = 1e-3
# Largest allowed widening past the flat bar against the oracle, in
# normalised units: both f32 implementations carry the noise envelope, whose
# element and row terms are each capped at ENV_CAP (5e-3,
# tests/np_reference.py), so two of them differ by at most 2 * (2 * ENV_CAP).
MAX_WIDENING = 4 * 5e-3

# One record per assert_parity call: (test, what, elements, widened, largest
# widening).  conftest.py prints them per test at the end of the run.
RECORDS = []
CURRENT_TEST = [""]


def assert_close(got, want, atol=ATOL, rtol=RTOL, what=""):
    import numpy as np
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    nan_g, nan_w = np.isnan(got), np.isnan(want)
    assert np.array_equal(nan_g, nan_w), f"{what}: NaN pattern differs"
    g, w = got[~nan_g], want[~nan_w]
    err = np.abs(g - w)
    bad = err > atol + rtol * np.abs(w)
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} outside tol, max abs err {err.max():.3e}"
    return float(err.max()) if err.size else 0.0


def assert_parity(got, oracle_out, ref64, env, atol=ATOL, rtol=RTOL, what=""):
    """GPU vs oracle at the north-star bar, widened only by the f32 noise envelope.

    The oracle and the reference both compute in f32.  Where a mel bin's
    energy sits near the 2^-24 guard, f32 FFT rounding moves the normalised
    value by up to ~1e-3, so no two f32 implementations agree to 1e-4 there.
    ``env`` (tests/np_reference.py:f32_noise_envelope) is the analytic scale
    of that noise per element: zero except on near-guard elements (float64
    mel energy at most 1e-6 of the frame's energy) and, through the row's
    mean and std, on the other elements of rows that hold them; each term at
    most 5e-3.
    Checks, per element:
      |got - ref64| <= atol + rtol*|ref64| + env         (GPU within f32 noise of exact)
    and either
      |got - oracle| <= atol + rtol*|oracle| + 2*env     (two f32 implementations agree)
    or |got - ref64| <= |oracle - ref64|                 (GPU closer to exact than the
                                                          oracle's radix-2 f32 FFT)
    and every element outside the flat bar against the oracle has env > 0
    (a near-guard element or a row holding one), and none is further past
    the flat bar than MAX_WIDENING.  Returns (max |got-oracle|, number of such widened
    elements)."""
    import numpy as np
    g = np.asarray(got, np.float64)
    o = np.asarray(oracle_out, np.float64)
    r = np.asarray(ref64, np.float64)
    n = np.asarray(env, np.float64)
    assert g.shape == o.shape == r.shape == n.shape, (g.shape, o.shape, r.shape, n.shape)
    nan = np.isnan(o)
    assert np.array_equal(np.isnan(g), nan), f"{what}: NaN pattern differs"
    g, o, r, n = g[~nan], o[~nan], r[~nan], n[~nan]
    base = atol + rtol * np.abs(o)
    b1 = (np.abs(g - o) > base + 2 * n) & (np.abs(g - r) > np.abs(o - r))
    b2 = np.abs(g - r) > atol + rtol * np.abs(r) + n
    assert not b1.any(), f"{what}: {b1.sum()} of {b1.size} outside oracle bound, max {np.abs(g - o).max():.3e}"
    assert not b2.any(), f"{what}: {b2.sum()} of {b2.size} outside f64 bound, max {np.abs(g - r).max():.3e}"
    wide = np.abs(g - o) > base
    assert not (wide & (n <= 0)).any(), \
        f"{what}: {(wide & (n <= 0)).sum()} elements outside the flat bar have no envelope"
    widened = int(wide.sum())
    widening = float((np.abs(g - o) - base).max()) if widened else 0.0
    RECORDS.append((CURRENT_TEST[0], what, int(g.size), widened, widening))
    assert widening <= MAX_WIDENING, f"{what}: widened {widening:.3e} past the flat bar, bound {MAX_WIDENING:.0e}"
    return float(np.abs(g - o).max()) if g.size else 0.0, widened
