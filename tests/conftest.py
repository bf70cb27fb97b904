import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def parity_err(got, ref):
    """max_i |got_i - ref_i| / max(|ref_i|, 1e-3 * ||ref||_inf) — the per-element
    relative error with a floor for entries near zero (the 1e-3 bar)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    floor = 1e-3 * np.abs(ref).max() if ref.size else 0.0
    den = np.maximum(np.abs(ref), max(floor, 1e-30))
    return float((np.abs(got - ref) / den).max()) if ref.size else 0.0


def inf_rel(got, ref):
    """||got - ref||_inf / ||ref||_inf."""
    ref = np.asarray(ref, np.float64)
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))


@pytest.fixture(scope="session")
def gpu():
    import fomoe_amd
    g = fomoe_amd.Gpu()
    yield g
    g.close()
