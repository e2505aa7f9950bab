import os
import sys

import pytest

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
