"""The backward triangular solve's division step (lusolve.hip, lu_trsv_kernel):
with ur = 1/u (IEEE FP32 division), q = v ur, then q + ur (v - u q) through two
FMAs, is v / u correctly rounded (Markstein's correction).  Checked here with
exact rational arithmetic for the FMAs against NumPy's IEEE FP32 division, on
random quotients over a wide exponent range and on divisors with mantissas
near 2, where the reciprocal is hardest to round."""

from fractions import Fraction

import numpy as np


def round32(x):
    """An exact rational rounded to the nearest FP32 value (ties to even)."""
    f = np.float32(float(x))
    cands = [f, np.nextafter(f, np.float32(np.inf)), np.nextafter(f, np.float32(-np.inf))]
    return min(cands, key=lambda y: (abs(Fraction(float(y)) - x),
                                     int(np.float32(y).view(np.uint32)) & 1))


def fma32(a, b, c):
    return round32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def test_reciprocal_correction_is_correctly_rounded():
    rng = np.random.default_rng(1)
    n = 30000
    v = (rng.standard_normal(n) * np.exp2(rng.integers(-20, 20, n))).astype(np.float32)
    u = (rng.standard_normal(n) * np.exp2(rng.integers(-20, 20, n))).astype(np.float32)
    u[:6000] = (np.float32(1.9999999) * np.exp2(rng.integers(-5, 5, 6000))).astype(np.float32)
    u[6000:6100] = np.float32(1.0)
    for a, b in zip(v, u):
        ur = np.float32(1) / b
        q = a * ur
        got = fma32(fma32(-b, q, a), ur, q)
        assert got == a / b, (a, b, got, a / b)


def test_plain_reciprocal_product_is_not():
    """The correction is needed: v * (1/u) alone misses correct rounding on
    some random quotients, so the test above would catch its omission."""
    rng = np.random.default_rng(2)
    v = rng.standard_normal(2000).astype(np.float32)
    u = rng.standard_normal(2000).astype(np.float32)
    assert np.any(v * (np.float32(1) / u) != v / u)
