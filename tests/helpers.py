"""Comparison helpers shared by the tests."""

import numpy as np


def rms(a):
    a = np.asarray(a, dtype=np.float64)
    return float(np.sqrt(np.mean(a * a))) if a.size else 0.0


def assert_close_rms(actual, expected, rtol, what=""):
    """Element-wise ``|a - e| <= rtol*|e| + rtol*RMS(e)`` (the atol convention
    for the bf16/fp8 configurations), plus relative Frobenius error <= rtol."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, (a.shape, e.shape)
    atol = rtol * rms(e)
    np.testing.assert_allclose(a, e, rtol=rtol, atol=atol, err_msg=what)
    den = np.linalg.norm(e)
    if den > 0:
        rel = np.linalg.norm(a - e) / den
        assert rel <= rtol, f"{what}: relative Frobenius error {rel:.3e} > {rtol}"


def assert_close(actual, expected, rtol=1e-5, atol=1e-6):
    """The reference's comparison (tests/utils.py:244-251)."""
    np.testing.assert_allclose(np.asarray(actual), np.asarray(expected), rtol=rtol, atol=atol)
