import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def f16(rng, *shape):
    """N(0,1) draws rounded to f16 (the synthetic inputs of every config)."""
    return rng.standard_normal(shape, dtype=np.float32).astype(np.float16)


@pytest.fixture
def rng():
    return np.random.default_rng(1234)
