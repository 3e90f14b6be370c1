"""OCP 8-bit E4M3 ("float8_e4m3fn") decode and encode, built from the format definition,
and the per-tensor quantisation of tasks/fp8_linear/reference.py:15-18.  Test
infrastructure only (see oracle/__init__.py).

Layout s.eeee.mmm, exponent bias 7, no infinities; exponent field 0 is subnormal
(value m * 2^-9); S.1111.111 is NaN; the largest finite magnitude is 448 (0x7E).
encode() is pinned against torch's float8_e4m3fn cast and quantize() against the
golden-pinned input quantisation (tests/test_quantize.py).
"""
from __future__ import annotations

import numpy as np


def _decode(byte: int) -> float:
    s = -1.0 if byte & 0x80 else 1.0
    e = (byte >> 3) & 0xF
    m = byte & 0x7
    if e == 0xF and m == 0x7:
        return float("nan")
    if e == 0:
        return s * m * 2.0 ** -9
    return s * (1.0 + m / 8.0) * 2.0 ** (e - 7)


TABLE = np.array([_decode(b) for b in range(256)], dtype=np.float64)


def decode(raw: np.ndarray) -> np.ndarray:
    """uint8 array of e4m3 bit patterns -> float64 values."""
    return TABLE[np.asarray(raw, dtype=np.uint8)]


# Non-negative finite codes 0x00..0x7E in increasing value (their values increase with the
# code), for nearest-value search.
_POS = TABLE[:0x7F]


def encode(v: np.ndarray) -> np.ndarray:
    """float array -> e4m3 bit patterns, round to nearest with ties to the even code (the
    even mantissa), the sign bit kept for -0.0, NaN -> 0x7F | sign.  Restates the cast
    torch.Tensor.to(torch.float8_e4m3fn) for inputs already clamped to [-448, 448], which is
    how tasks/fp8_linear/reference.py:15-18 uses it; larger magnitudes are not handled."""
    v = np.asarray(v, dtype=np.float64)
    sign = np.signbit(v).astype(np.uint8) << 7
    a = np.abs(v)
    if np.any(a[~np.isnan(a)] > 448.0):
        raise ValueError("encode() takes |v| <= 448")
    hi = np.clip(np.searchsorted(_POS, a, side="left"), 0, 0x7E)   # first code with value >= a
    lo = np.clip(hi - 1, 0, 0x7E)
    dlo, dhi = a - _POS[lo], _POS[hi] - a
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    code = np.where(np.isnan(a), np.uint8(0x7F), code)
    return (code | sign).astype(np.uint8)


def quantize(x: np.ndarray) -> tuple[np.ndarray, np.float32]:
    """Per-tensor max-abs quantisation of a non-empty fp32 array, as
    tasks/fp8_linear/reference.py:15-18: scale = fp32(448 / max(amax, 1e-9)) with the
    quotient in fp64 (Python max keeps a NaN amax), q = e4m3(clamp(x * scale, +-448)) with
    the product in fp32."""
    x = np.asarray(x, dtype=np.float32)
    amax = float(np.abs(x).max())           # NaN if x holds one
    den = amax if amax != amax else max(amax, 1e-9)
    scale = np.float32(448.0 / den)
    with np.errstate(invalid="ignore", over="ignore"):
        s = (x * scale).astype(np.float32)
        s = np.where(s < -448.0, np.float32(-448.0), np.where(s > 448.0, np.float32(448.0), s))
    return encode(s), scale


def same_codes(a: np.ndarray, b: np.ndarray) -> bool:
    """Byte arrays equal, except that any two NaN codes (0x7F, 0xFF) match: the sign of a
    NaN produced by arithmetic is unspecified (IEEE 754), and torch on x86 gives -NaN
    where numpy gives +NaN, as the grader's compare rule lets NaN match NaN."""
    a, b = np.asarray(a, dtype=np.uint8), np.asarray(b, dtype=np.uint8)
    nan_a, nan_b = (a & 0x7F) == 0x7F, (b & 0x7F) == 0x7F
    return a.shape == b.shape and bool(np.all((a == b) | (nan_a & nan_b)))
