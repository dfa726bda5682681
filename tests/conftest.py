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
    """max_i |got_i - want_i| / max(|want_i|, floor * rms(want)) (the
    per-element parity metric; the floor keeps near-zero outputs from
    dominating)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    rms = float(np.sqrt(np.mean(want * want))) if want.size else 0.0
    den = np.maximum(np.abs(want), floor * rms if rms > 0 else 1.0)
    return float((np.abs(got - want) / den).max()) if want.size else 0.0


# The parity bars of the matvec, expert and MoE outputs against the oracle:
#   normwise  max|got - want| / max|want|                          <= 1e-3
#   strict    max_i |got_i - want_i| / max(|want_i|, 1e-3 rms)      <= 2e-3
# The strict bound sits at about three times what f32 arithmetic itself
# scores at these widths: for a Q4_K matrix with 12288 inputs, a plain f32
# BLAS product of the same dequantized operands scores 5.9e-4, and x held as
# 24-bit limbs with exact sums 4.8e-4 (measured on the device: 3.5e-4 to
# 7.5e-4 across the decode shapes). A dropped term, a wrong index or a wrong
# scale scores O(1).
NORM_TOL = 1e-3
STRICT_TOL = 2e-3
METRICS = []  # (test, label, normwise, strict, strict asserted) of every check_parity call


def check_parity(got, want, label="", norm_tol=NORM_TOL, strict_tol=STRICT_TOL):
    """Asserts both parity metrics and records them for the session report."""
    n = rel_err(got, want)
    st = elem_rel_err(got, want)
    test = os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0]
    METRICS.append((test, label, n, st, strict_tol is not None))
    assert n <= norm_tol, f"{label}: normwise error {n:.3e} > {norm_tol:g}"
    if strict_tol is not None:  # None: recorded only (operands rounded on purpose, e.g. bf16)
        assert st <= strict_tol, f"{label}: per-element error {st:.3e} > {strict_tol:g}"


def pytest_terminal_summary(terminalreporter):
    """The worst parity metrics per test file (and a JSON record of every
    check in the file STRATA_PARITY_JSON names, when it is set)."""
    if not METRICS:
        return
    worst = {}
    for test, _label, n, st, asserted in METRICS:
        f = test.split("::")[0]
        a, b, r, c = worst.get(f, (0.0, 0.0, None, 0))
        if asserted:
            b = max(b, st)
        else:  # operands rounded on purpose (bf16, Q8): the per-element figure is recorded, not held to the bar
            r = max(r or 0.0, st)
        worst[f] = (max(a, n), b, r, c + 1)
    terminalreporter.write_sep("-", "parity metrics (worst per file: normwise, per-element with 1e-3 rms floor)")
    for f, (n, st, r, c) in sorted(worst.items()):
        extra = "" if r is None else f"; per-element of the checks against unrounded f32 (not asserted) {r:.2e}"
        terminalreporter.write_line(f"{f}: {c} checks, normwise {n:.2e}, per-element {st:.2e}{extra}")
    out = os.environ.get("STRATA_PARITY_JSON")
    if out:
        import json
        with open(out, "w") as fh:
            json.dump([{"test": t, "label": l, "normwise": n, "per_element": st, "per_element_asserted": a}
                       for t, l, n, st, a in METRICS], fh)
