"""Exact IEEE binary32 arithmetic for spec restatements in tests.

numpy float32 `+ - * /` are single correctly rounded operations; fma is
not available, so fma32 rounds the exact rational a*b + c once (round to
nearest, ties to even).
"""
from fractions import Fraction

import numpy as np

F32 = np.float32


def round_f32(x: Fraction) -> np.float32:
    c = F32(float(x))
    if not np.isfinite(c):
        return c
    best = None
    for cand in (np.nextafter(c, F32(-np.inf)), c, np.nextafter(c, F32(np.inf))):
        d = abs(Fraction(float(cand)) - x)
        key = (d, int(np.asarray(cand).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, cand)
    return F32(best[1])


def fma32(a, b, c) -> np.float32:
    return round_f32(Fraction(float(F32(a))) * Fraction(float(F32(b))) + Fraction(float(F32(c))))


def f16_to_f32(bits) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)
