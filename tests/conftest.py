"""Shared test setup: import paths, the `gpu` marker, common fixtures.

CPU tests (`-m "not gpu"`) check the oracle against the reference's golden
vectors and closed forms, the synthetic generators and the C-ABI library's
exports. GPU tests (`-m gpu`) call the HIP path through the C ABI and compare
it with the oracle.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "strata-rs_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

# torch bundles its own HIP runtime with the same soname (libamdhip64.so.7)
# as the system one libstrata_hip links against; whichever is loaded first
# serves the whole process, and torch only works with its own. Importing
# torch before the library is loaded keeps one runtime for every test (the
# benchmark imports torch first for the same reason).
try:
    import torch  # noqa: F401
except ImportError:  # pragma: no cover - torch is part of the image
    torch = None


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path)")


@pytest.fixture(scope="session")
def oracle():
    import oracle as O
    if not os.path.exists(O.LIB_PATH):
        O.build()
    return O


@pytest.fixture(scope="session")
def backend():
    """One HIP context for the GPU tests (fails loudly without a device)."""
    import strata_hip as H
    be = H.HipBackend(0, 8 << 30)
    yield be
    be.close()


def rel_err(got, want):
    """max|got - want| / max|want| (the normwise parity metric)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    denom = np.abs(want).max()
    return float(np.abs(got - want).max() / (denom if denom > 0 else 1.0))


def elem_rel_err(got, want, floor=1e-3):
    """max_i |got_i - want_i| / max(|want_i|, floor * rms(want))."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    rms = float(np.sqrt(np.mean(want * want))) if want.size else 0.0
    den = np.maximum(np.abs(want), floor * rms if rms > 0 else 1.0)
    return float((np.abs(got - want) / den).max()) if want.size else 0.0
