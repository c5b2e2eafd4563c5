import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "ppdoclayout-ggml_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI)")


def normwise(y, ref):
    """max|y - ref| / max|ref|: the per-op parity metric (tolerance 2e-5)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.abs(ref).max()
    return float(np.abs(y - ref).max() / (den if den > 0 else 1.0))


def rel1(y, ref):
    """max|y - ref| / (|ref| + 1): elementwise companion metric."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float((np.abs(y - ref) / (np.abs(ref) + 1.0)).max())


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def hip():
    import ppdl_hip

    ppdl_hip.lib()
    return ppdl_hip
