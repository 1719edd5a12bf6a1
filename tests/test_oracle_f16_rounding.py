"""float64 -> float16 rounding of the rotated float16 activations (oracle/convrot.py
round_f64_to_f16) and the device's route to it (act_rot.h f64_to_f16_bits: round-to-odd to
float32, then round-to-nearest-even to float16), both against exact rational rounding.

Cases: the midpoint between every pair of adjacent positive float16 values (an exact tie: the
even neighbour wins), the midpoint moved by one float64 ulp either way (the nearer side wins,
which a plain float32 round trip gets wrong wherever the float32 rounding lands on the
midpoint), subnormal and overflow boundaries, and random float64 values. A planted mistake (the
plain float32 round trip, rounded twice) must fail.
"""

from fractions import Fraction

import numpy as np

from oracle import convrot as cr


def _exact_rne_f16(x: float) -> int:
    """float16 bits of x by exact rational round-to-nearest-even (finite x)."""
    if x == 0.0:
        return 0x8000 if np.signbit(x) else 0
    sign = 0x8000 if x < 0 else 0
    ax = Fraction(abs(x))
    lo, hi = 0, 0x7C00  # search the positive float16 magnitudes (0x7C00 = +inf as the top)
    vals = np.arange(0, 0x7C01, dtype=np.uint16).view(np.float16).astype(np.float64)
    # largest magnitude <= ax
    i = int(np.searchsorted(vals, float(ax), side="right")) - 1
    while i + 1 <= 0x7BFF and Fraction(vals[i + 1]) <= ax:
        i += 1
    while i > 0 and Fraction(vals[i]) > ax:
        i -= 1
    if i >= 0x7BFF:  # at or above the largest finite value: overflow boundary 65520
        return sign | (0x7C00 if ax >= Fraction(65520) else 0x7BFF)
    a, b = Fraction(vals[i]), Fraction(vals[i + 1])
    if ax - a < b - ax:
        return sign | i
    if ax - a > b - ax:
        return sign | (i + 1)
    return sign | (i if i % 2 == 0 else i + 1)


def _device_route(x: np.ndarray) -> np.ndarray:
    """The device's f64_to_f16_bits restated: float32 by round-to-odd, then RNE to float16."""
    x = np.asarray(x, dtype=np.float64)
    f = x.astype(np.float32)
    u = f.view(np.uint32).copy()
    inexact = f.astype(np.float64) != x
    away = np.abs(f.astype(np.float64)) > np.abs(x)
    u = np.where(inexact & away, u - 1, u)
    u = np.where(inexact, u | 1, u).astype(np.uint32)
    with np.errstate(over="ignore"):
        return u.view(np.float32).astype(np.float16).view(np.uint16)


def _cases() -> np.ndarray:
    pos = np.arange(1, 0x7BFF, dtype=np.uint16).view(np.float16).astype(np.float64)
    nxt = np.arange(2, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mid = (pos + nxt) / 2  # exact in float64
    up = np.nextafter(mid, np.inf)
    down = np.nextafter(mid, 0.0)
    rng = np.random.default_rng(5)
    rnd = rng.standard_normal(4000) * np.exp2(rng.integers(-26, 16, 4000))
    edges = np.array([2.0 ** -25, np.nextafter(2.0 ** -25, 1.0), 2.0 ** -24 * 1.5, 65504.0, 65519.99, 65520.0])
    sample = np.concatenate([mid[::7], up[::7], down[::7], rnd, edges])
    return np.concatenate([sample, -sample])


def test_oracle_and_device_route_round_once():
    x = _cases()
    exact = np.array([_exact_rne_f16(float(v)) for v in x], dtype=np.uint16)
    oracle = cr.round_f64_to_f16(x).view(np.uint16)
    assert np.array_equal(oracle, exact)
    assert np.array_equal(_device_route(x), exact)


def test_planted_double_rounding_is_caught():
    x = _cases()
    exact = np.array([_exact_rne_f16(float(v)) for v in x], dtype=np.uint16)
    with np.errstate(over="ignore"):
        twice = x.astype(np.float32).astype(np.float16).view(np.uint16)
    assert not np.array_equal(twice, exact)
