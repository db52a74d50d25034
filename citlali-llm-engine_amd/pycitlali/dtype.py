"""Host fp16 conversion with the reference's rounding rule, vectorised.

float_to_half_bits follows dtype.cpp:136-176 of the reference: round to
nearest with ties away from zero (only the most significant dropped bit is
looked at), overflow and NaN to signed infinity, magnitudes below 2^-25 to
signed zero.  half_bits_to_float is the exact widening of dtype.cpp:76-133.
"""
from __future__ import annotations

import numpy as np


def float_to_half_bits(values) -> np.ndarray:
    f = np.ascontiguousarray(values, dtype=np.float32)
    u = f.view(np.uint32).astype(np.int64)
    sign = (u >> 16) & 0x8000
    e16 = ((u >> 23) & 0xFF) - 112
    frac = u & 0x7FFFFF
    out = np.zeros(u.shape, dtype=np.int64)
    normal = (e16 > 0) & (e16 < 31)
    out = np.where(normal, ((e16 << 10) | (frac >> 13)) + ((frac >> 12) & 1), out)
    out = np.where(e16 >= 31, 0x7C00, out)
    sub = (e16 <= 0) & (e16 >= -10)
    sig = frac | 0x800000
    sh = np.clip(14 - e16, 14, 24)
    out = np.where(sub, (sig >> sh) + ((sig >> (sh - 1)) & 1), out)
    return (sign | out).astype(np.uint16)


def half_bits_to_float(bits) -> np.ndarray:
    return np.ascontiguousarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)
