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


def assert_close_requantized(actual, expected, rtol, frob, max_frac, max_rms, what=""):
    """For results computed from re-quantised intermediates (e4m3 SwiGLU rows):
    an intermediate that the kernel and the oracle round one bf16 ulp apart
    next to an e4m3 rounding boundary gets codes one e4m3 ulp apart, which
    moves that row's outputs by more than the bf16 tolerance.  So: relative
    Frobenius error <= frob, at most a fraction max_frac of the elements
    outside ``rtol*|e| + rtol*RMS(e)``, and none beyond ``max_rms*RMS(e)``."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, (a.shape, e.shape)
    r = rms(e)
    err = np.abs(a - e)
    rel = np.linalg.norm(a - e) / np.linalg.norm(e)
    frac = float(np.mean(err > rtol * np.abs(e) + rtol * r))
    worst = float(err.max() / r)
    msg = f"{what}: rel Frobenius {rel:.2e}, {frac:.2e} of elements outside rtol {rtol}, max |err| {worst:.3f} RMS"
    assert np.all(np.isfinite(a)), msg
    assert rel <= frob and frac <= max_frac and worst <= max_rms, msg
    return rel, frac, worst


def assert_close(actual, expected, rtol=1e-5, atol=1e-6):
    """The reference's comparison (tests/utils.py:244-251)."""
    np.testing.assert_allclose(np.asarray(actual), np.asarray(expected), rtol=rtol, atol=atol)


def packed_index(n_out, n_in, n_expert, dtype):
    """Flat element offset of every weight (e, n, k) in the packed buffer,
    shape [E, n_out, n_in]: the WF_MFMA16 block layout (16 rows x 32 inputs
    per 1 KiB block for bf16, 16 x 64 for fp8, 64 lanes x 16 bytes, lane l =
    row l%16, inputs 8*(l//16)..+8 of each 32-input step) when the shape
    allows it, else row-major [E][n_out][n_in]."""
    e, n, k = np.meshgrid(np.arange(n_expert), np.arange(n_out), np.arange(n_in), indexing="ij")
    if dtype == "bf16" and n_out % 16 == 0 and n_in % 32 == 0:
        blk = (e * (n_out // 16) + n // 16) * (n_in // 32) + k // 32
        lane = n % 16 + 16 * ((k % 32) // 8)
        return blk * 512 + lane * 8 + k % 8
    if dtype == "fp8" and n_out % 16 == 0 and n_in % 64 == 0:
        blk = (e * (n_out // 16) + n // 16) * (n_in // 64) + k // 64
        kk = k % 64
        q = kk % 32
        lane = n % 16 + 16 * (q // 8)
        return blk * 1024 + lane * 16 + (kk // 32) * 8 + q % 8
    return (e * n_out + n) * n_in + k
