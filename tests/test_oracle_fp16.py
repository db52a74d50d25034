"""Pins the oracle's fp16 conversions (dtype.cpp:76-176).

f2h (ties away): golden vectors from the compiled reference, an independent
closed-form statement of "nearest, ties away from zero" in float64, known
answers, and (when oracle/_ref is built) every one of the 2^32 inputs.
h2f: all 65536 patterns against the golden file and numpy's exact widening.
f2h_rne: numpy's float32 -> float16 cast (IEEE nearest-even).
"""
from __future__ import annotations

import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def spec_ties_away(f: np.ndarray) -> np.ndarray:
    """Closed form, not the bit algorithm: |x| rounded to the fp16 grid with
    halves rounded up in magnitude; |x| >= 65520 -> Inf; NaN -> Inf; results
    below the smallest subnormal flush per the grid rounding."""
    x = f.astype(np.float64)
    a = np.abs(x)
    sign = np.signbit(x).astype(np.uint16) << 15
    with np.errstate(divide="ignore", invalid="ignore"):
        e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    e = np.clip(e, -14, 15)
    ulp = np.exp2(e - 10)
    q = np.floor(a / ulp + 0.5) * ulp          # ties go up in magnitude
    q = np.where(np.isnan(x) | (a >= 65520.0), np.inf, q)
    out = q.astype(np.float16).view(np.uint16)  # q is on the grid: the cast is exact
    return (out & 0x7FFF) | sign


def test_f2h_known_answers(orc):
    cases = [(1.0, 0x3C00), (1.0 + 2 ** -11, 0x3C01), (1.0 + 3 * 2 ** -11, 0x3C02), (-(1.0 + 2 ** -11), 0xBC01),
             (65504.0, 0x7BFF), (65519.0, 0x7BFF), (65520.0, 0x7C00), (float("inf"), 0x7C00),
             (float("nan"), 0x7C00), (2 ** -24, 0x0001), (2 ** -25, 0x0001), (2 ** -26, 0x0000),
             (0.0, 0x0000), (-0.0, 0x8000)]
    for v, h in cases:
        assert int(orc.f2h(np.array([v], np.float32))[0]) == h, v
    # NaN keeps its sign: -NaN -> -Inf
    neg_nan = np.array([0xFFC00000], np.uint32).view(np.float32)
    assert int(orc.f2h(neg_nan)[0]) == 0xFC00


def test_f2h_matches_reference_golden(orc):
    g = np.load(os.path.join(GOLDEN, "f2h.npz"), allow_pickle=False)
    x = g["f32_bits"].view(np.float32)
    np.testing.assert_array_equal(orc.f2h(x), g["fp16"])


def test_f2h_matches_closed_form_spec(orc):
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2 ** 32, 2_000_000, dtype=np.uint64).astype(np.uint32)
    # concentrate on the fp16 range and on exact ties
    mag = rng.uniform(-30, 17, 1_000_000)
    x = np.concatenate([bits.view(np.float32), np.exp2(mag).astype(np.float32),
                        -np.exp2(mag[:300000]).astype(np.float32)])
    h = np.arange(0, 0x7BFF, dtype=np.uint16).view(np.float16).astype(np.float64)
    ties = ((h[:-1] + h[1:]) / 2).astype(np.float32)
    x = np.concatenate([x, ties, -ties])
    x = x[~np.isnan(x) | (rng.random(x.size) < 0.01)]
    np.testing.assert_array_equal(orc.f2h(x), spec_ties_away(x))


def test_f2h_rne_matches_ieee_cast(orc):
    rng = np.random.default_rng(8)
    x = np.concatenate([rng.integers(0, 2 ** 32, 2_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32),
                        np.exp2(rng.uniform(-30, 17, 500000)).astype(np.float32)])
    h = np.arange(0, 0x7BFF, dtype=np.uint16).view(np.float16).astype(np.float64)
    x = np.concatenate([x, ((h[:-1] + h[1:]) / 2).astype(np.float32)])
    x = x[~np.isnan(x)]
    with np.errstate(over="ignore"):
        expect = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(orc.f2h_rne(x), expect)


def test_h2f_all_patterns(orc):
    h = np.arange(65536, dtype=np.uint16)
    got = orc.h2f(h)
    g = np.load(os.path.join(GOLDEN, "h2f.npz"), allow_pickle=False)
    np.testing.assert_array_equal(got.view(np.uint32), g["f32_bits"])
    finite = (h & 0x7C00) != 0x7C00
    np.testing.assert_array_equal(got[finite], h[finite].view(np.float16).astype(np.float32))


def test_f2h_exhaustive_against_compiled_reference(orc, ref):
    """All 2^32 float32 inputs through the reference's float_to_half_bits."""
    chunk = 1 << 24
    for c in range(256):
        f = (np.arange(chunk, dtype=np.uint64) + np.uint64(c * chunk)).astype(np.uint32).view(np.float32)
        a, b = orc.f2h(f), ref.f2h(f)
        if not np.array_equal(a, b):
            i = int(np.flatnonzero(a != b)[0])
            pytest.fail(f"mismatch at bits {f.view(np.uint32)[i]:#010x}: {a[i]:#06x} vs {b[i]:#06x}")


def test_product_host_conversion_matches_oracle(orc):
    """pycitlali.dtype.float_to_half_bits (used to make inputs) == oracle."""
    from pycitlali.dtype import float_to_half_bits
    rng = np.random.default_rng(9)
    x = np.concatenate([rng.integers(0, 2 ** 32, 3_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32),
                        np.exp2(rng.uniform(-30, 17, 500000)).astype(np.float32)])
    np.testing.assert_array_equal(float_to_half_bits(x), orc.f2h(x))
