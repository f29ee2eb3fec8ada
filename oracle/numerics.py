"""Number-format closed forms used by the oracle (test infrastructure only).

The reference computes in fp32 only; the bf16 and fp8-e4m3 paths are
extensions whose oracle is the fp32 formula on rounded / dequantised inputs.
These are written from the format definitions:

* bfloat16: the top 16 bits of an IEEE binary32, rounded to nearest even.
* OCP FP8 E4M3 ("e4m3fn"): 1 sign, 4 exponent (bias 7), 3 mantissa bits;
  no infinities; NaN = S.1111.111; largest finite 448 = 1.75 * 2**8;
  subnormals m/8 * 2**-6.
"""

from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round binary32 values to the nearest bfloat16 (ties to even) and return
    them widened back to float32."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    bits = a.view(np.uint32).astype(np.uint64)
    lsb = (bits >> np.uint64(16)) & np.uint64(1)
    r = ((bits + np.uint64(0x7FFF) + lsb) >> np.uint64(16)) << np.uint64(16)
    out = (r & np.uint64(0xFFFFFFFF)).astype(np.uint32).view(np.float32).reshape(a.shape)
    out = np.where(np.isnan(a), np.float32(np.nan), out)
    return out


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """The bfloat16 bit pattern (uint16) of ``bf16_round(x)``."""
    return (bf16_round(x).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def _e4m3fn_table() -> np.ndarray:
    codes = np.arange(256, dtype=np.uint32)
    s = (codes >> 7) & 1
    e = (codes >> 3) & 0xF
    m = codes & 7
    mag = np.where(e == 0, m / 8.0 * 2.0**-6, (1 + m / 8.0) * 2.0 ** (e.astype(np.float64) - 7))
    val = np.where(s == 1, -mag, mag)
    val[(e == 15) & (m == 7)] = np.nan
    return val


E4M3FN_VALUES = _e4m3fn_table()  # float64 value of every code


def e4m3fn_decode(codes: np.ndarray) -> np.ndarray:
    """Code (uint8) -> float32 value."""
    return E4M3FN_VALUES[np.asarray(codes, dtype=np.uint8)].astype(np.float32)


def e4m3fn_encode(x: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn code (uint8): round to nearest, ties to the even code,
    finite values beyond 448 saturate to +-448, NaN -> 0x7F."""
    a = np.asarray(x, dtype=np.float32).astype(np.float64)
    mag = np.abs(a)
    pos = E4M3FN_VALUES[:127]  # codes 0x00..0x7E, increasing, 0 .. 448
    hi = np.clip(np.searchsorted(pos, mag, side="left"), 0, 126)
    lo = np.clip(hi - 1, 0, 126)
    d_lo = mag - pos[lo]
    d_hi = pos[hi] - mag
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo)
    code = np.where(mag >= E4M3_MAX, 126, code)
    code = code.astype(np.uint32) | (np.signbit(a).astype(np.uint32) << 7)
    code = np.where(np.isnan(a), 0x7F, code)
    return code.astype(np.uint8)


def quantize_per_channel_e4m3fn(w: np.ndarray):
    """Per-output-channel absmax quantisation of expert weights in the
    reference layout ``[n_out, n_in, E]``.

    ``scale[n, e] = max_i |w[n, i, e]| / 448`` (float32; an all-zero channel
    gets scale 1), ``q = e4m3fn_encode(w / scale)``.  Returns
    ``(q [n_out, n_in, E] uint8, scale [n_out, E] float32)``; the dequantised
    weights are ``e4m3fn_decode(q) * scale[:, None, :]``.
    """
    w32 = np.asarray(w, dtype=np.float32)
    amax = np.abs(w32).max(axis=1)  # [n_out, E]
    scale = (amax / np.float32(E4M3_MAX)).astype(np.float32)
    scale = np.where(amax > 0, scale, np.float32(1.0)).astype(np.float32)
    q = e4m3fn_encode(w32 / scale[:, None, :])
    return q, scale


def dequantize_e4m3fn(q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """``decode(q) * scale`` for the ``[n_out, n_in, E]`` / ``[n_out, E]`` pair."""
    return (e4m3fn_decode(q) * np.asarray(scale, np.float32)[:, None, :]).astype(np.float32)


def quantize_rows_e4m3fn(a: np.ndarray):
    """Per-row e4m3fn quantisation of activations (the fp8-activation GEMMs'
    operand): ``scale[r] = 2**e``, the smallest power of two with
    ``max_i |a[r, i]| / 2**e <= 448`` (``e`` clamped to [-126, 126]; 1 for an
    all-zero row), ``q = e4m3fn_encode(a * 2**-e)``.  The scaling is exact, so
    each value's rounding depends only on the value and its binade, not on the
    row maximum.  Returns ``(q uint8, scale float32)``; the row's largest
    magnitude lands in (224, 448]."""
    a32 = np.asarray(a, dtype=np.float32)
    amax = np.abs(a32).max(axis=1).astype(np.float32)
    bits = amax.view(np.uint32).astype(np.int64)
    # 448 = 1.75 * 2**8: amax = m * 2**E needs e = E - 8, or E - 7 when m > 1.75
    e = (bits >> 23) - 127 - 8 + ((bits & 0x7FFFFF) > 0x600000)
    e = np.clip(e, -126, 126)
    scale = np.where(amax > 0, np.ldexp(np.float32(1.0), e).astype(np.float32), np.float32(1.0)).astype(np.float32)
    q = e4m3fn_encode((a32 / scale[:, None]).astype(np.float32))
    return q, scale


def fake_quantize_rows_e4m3fn(a: np.ndarray) -> np.ndarray:
    """``decode(q) * scale`` of ``quantize_rows_e4m3fn(a)`` (float32)."""
    q, scale = quantize_rows_e4m3fn(a)
    return (e4m3fn_decode(q) * scale[:, None]).astype(np.float32)


def quantize_rows_e4m3fn_x2(a: np.ndarray):
    """Two-term per-row e4m3fn quantisation (the FMOE_F8E4M3FN_A8X2 GEMM
    operand; no counterpart in the reference): the row scale of
    ``quantize_rows_e4m3fn``, ``hi = e4m3fn_encode(a / scale)`` (its codes),
    and ``lo = e4m3fn_encode(a / scale - decode(hi))``, the rounding
    remainder as a second code under the same scale.  Returns
    ``(hi uint8, lo uint8, scale float32)``; the represented value is
    ``(decode(hi) + decode(lo)) * scale``."""
    hi, scale = quantize_rows_e4m3fn(a)
    v = (np.asarray(a, dtype=np.float32) / scale[:, None]).astype(np.float32)
    lo = e4m3fn_encode((v - e4m3fn_decode(hi)).astype(np.float32))
    return hi, lo, scale


def fake_quantize_rows_e4m3fn_x2(a: np.ndarray) -> np.ndarray:
    """``(decode(hi) + decode(lo)) * scale`` of ``quantize_rows_e4m3fn_x2(a)``
    (float32)."""
    hi, lo, scale = quantize_rows_e4m3fn_x2(a)
    return ((e4m3fn_decode(hi) + e4m3fn_decode(lo)) * scale[:, None]).astype(np.float32)
