import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def device():
    from enargeia_amd.kernels import Device

    dev = Device(0)
    yield dev
    dev.close()


def compare(actual: np.ndarray, expected: np.ndarray, atol: float, rtol: float):
    """test/reference/matmul.ts:56-81: per element |a - e| <= atol + rtol*|e|; returns the
    worst ratio (1.0 = exactly at tolerance), its index, max abs and max rel error."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, f"length mismatch: {a.shape} vs {e.shape}"
    err = np.abs(a - e)
    mag = np.abs(e)
    ratio = err / (atol + rtol * mag)
    worst = int(np.argmax(ratio)) if ratio.size else -1
    rel = np.where(mag > 1e-6, err / np.maximum(mag, 1e-30), 0.0)
    return (float(ratio[worst]) if ratio.size else 0.0, worst, float(err.max(initial=0.0)),
            float(rel.max(initial=0.0)))


def assert_close(actual, expected, atol, rtol, label=""):
    worst, idx, max_abs, max_rel = compare(actual, expected, atol, rtol)
    assert worst <= 1.0, (f"{label}: worst element {idx} at {worst * 100:.1f}% of tolerance "
                          f"(abs {max_abs:.2e}, rel {max_rel:.2e}; got {np.asarray(actual).ravel()[idx]!r} "
                          f"expected {np.asarray(expected).ravel()[idx]!r})")
    return worst


FP32_TOLERANCE = (1e-4, 1e-4)   # test/reference/matmul.ts:88
Q4_TOLERANCE = (5e-2, 8e-2)     # test/reference/matmul.ts:97


def gemv_tolerance(expected: np.ndarray):
    """BASELINE's fp32 GEMV bar: 1e-3 relative, with an absolute floor of 1e-5 x the output's
    RMS so that outputs that happen to sit near zero are judged against the row scale."""
    rms = float(np.sqrt(np.mean(np.asarray(expected, dtype=np.float64) ** 2))) if np.size(expected) else 0.0
    return (1e-5 * rms, 1e-3)
