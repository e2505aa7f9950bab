import os
import sys

import pytest

import parity
from parity import ATOL, RTOL, assert_close, assert_parity  # noqa: F401

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def extractor():
    from scriptrs_amd import ParakeetFeatureExtractor
    ext = ParakeetFeatureExtractor()
    yield ext
    ext.close()


@pytest.fixture(autouse=True)
def _parity_test_name(request):
    parity.CURRENT_TEST[0] = request.node.name
    yield
    parity.CURRENT_TEST[0] = ""


def pytest_terminal_summary(terminalreporter):
    """Per test: elements compared against the oracle, how many of them the
    f32 noise envelope widened past the flat 1e-4 + 1e-3 bar, and the
    largest widening (normalised units), against the bound."""
    if not parity.RECORDS:
        return
    per = {}
    for test, _, n, w, mx in parity.RECORDS:
        a = per.setdefault(test, [0, 0, 0.0, 0])
        a[0] += n
        a[1] += w
        a[2] = max(a[2], mx)
        a[3] += 1
    tr = terminalreporter
    tr.write_line(f"parity vs oracle: widened elements past the flat bar, largest widening (bound "
                  f"{parity.MAX_WIDENING:.0e})")
    for test, (n, w, mx, calls) in per.items():
        if w:
            tr.write_line(f"  {test}: {w} of {n} widened, largest {mx:.2e} ({calls} comparisons)")
    n = sum(a[0] for a in per.values())
    w = sum(a[1] for a in per.values())
    mx = max(a[2] for a in per.values())
    quiet = sum(1 for a in per.values() if not a[1])
    tr.write_line(f"  all {len(per)} tests: {w} of {n} widened, largest {mx:.2e}; {quiet} tests widened none")
