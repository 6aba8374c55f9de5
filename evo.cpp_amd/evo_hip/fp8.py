"""Vectorised E4M3FN (OCP ``float8_e4m3fn``) codec used by the artifact writer.

Encoding is round-to-nearest-even with saturation to +-448 for finite
overflow and infinities, NaN -> 0x7f|sign, and a negative sign kept on values
that round to zero -- the semantics of evo.cpp `src/fp8.cpp:26-58`.
"""
from __future__ import annotations

import numpy as np


def _positive_table() -> np.ndarray:
    codes = np.arange(0x7F, dtype=np.uint32)  # 0x00..0x7e
    exponent = (codes >> 3) & 0xF
    mantissa = (codes & 7).astype(np.float64)
    normal = (1.0 + mantissa / 8.0) * np.exp2(exponent.astype(np.float64) - 7)
    subnormal = mantissa * 2.0 ** -9
    return np.where(exponent == 0, subnormal, normal).astype(np.float32)


_TABLE = _positive_table()


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    codes = np.asarray(codes, dtype=np.uint8)
    magnitude = codes & np.uint8(0x7F)
    values = _TABLE[np.minimum(magnitude, 0x7E)].astype(np.float32)
    values = np.where(magnitude == 0x7F, np.float32(np.nan), values)
    return np.where(codes & 0x80, -values, values).astype(np.float32)


def e4m3_encode(values: np.ndarray) -> np.ndarray:
    x = np.asarray(values, dtype=np.float32)
    sign = np.where(np.signbit(x), np.uint8(0x80), np.uint8(0))
    magnitude = np.abs(x)
    # index of the largest code not above the magnitude
    low = np.searchsorted(_TABLE, magnitude, side="right") - 1
    low = np.clip(low, 0, 0x7E)
    high = np.minimum(low + 1, 0x7E)
    below = magnitude - _TABLE[low]
    above = _TABLE[high] - magnitude
    choose_high = (above < below) | ((above == below) & ((high & 1) == 0))
    code = np.where(choose_high & (high != low), high, low).astype(np.uint8)
    code = np.where(magnitude >= np.float32(448.0), np.uint8(0x7E), code)
    code = np.where(np.isnan(x), np.uint8(0x7F), code)
    return (code | sign).astype(np.uint8)
