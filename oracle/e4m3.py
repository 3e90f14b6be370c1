"""OCP 8-bit E4M3 ("float8_e4m3fn") decode, built from the format definition.

Layout s.eeee.mmm, exponent bias 7, no infinities; exponent field 0 is subnormal
(value m * 2^-9); S.1111.111 is NaN; the largest finite magnitude is 448 (0x7E).
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
