"""The decode prologue's RMSNorm mean decision, pinned with exact rationals.

The kernel sums the squares of a row in a tree, T, and decides the mean
(float)(ss / H) of the reference's in-order double sum ss
(kernel/qwen35_decoder.cpp:137-138) from an error bound E >= |ss - T|: when
every ss in [T - E, T + E] gives the same float, that float is the mean.
norm_mean_from_bound_r (csrc/qmm_common.h) brackets ss / H with a
reciprocal rH = RN(1 / H) instead of two divisions,
q = RN(T rH), D = (E rH + 2^-50 q)(1 + 2^-10), and decides when
(float)RN(q - D) == (float)RN(q + D).  The checks below evaluate both ends
T -/+ E exactly (Fractions: the quotient by H correctly rounded to double,
then to float) and require any decided mean to equal both, on random sums
over the whole range of float squares and on sums placed within a few
double ulps of a float rounding boundary of the mean.  A version without
the 2^-50 q term (the reciprocal's own error) must fail there.
"""
from fractions import Fraction

import numpy as np
import pytest

F64 = np.float64


def _decide(T, H, per=0, recip_term=True):
    """The decision rule of norm_mean_from_bound_r, step by step in IEEE
    binary64 (numpy scalars: every operation rounded, none fused)."""
    T = F64(T)
    E = F64(H + per + 24) * F64(2.0 ** -53) * T * F64(1.0 + 2.0 ** -10)
    rH = F64(1.0) / F64(H)
    q = T * rH
    D = E * rH
    if recip_term:
        D = D + q * F64(2.0 ** -50)
    D = D * F64(1.0 + 2.0 ** -10)
    with np.errstate(over="ignore"):  # means past FLT_MAX are inf, as in the reference
        lo, hi = np.float32(q - D), np.float32(q + D)
    return bool(lo == hi), lo, E


def _mean_exact(x, H):
    """(float)(x / H) for an exact rational x: the quotient correctly rounded
    to double (Python's int division), then to float."""
    with np.errstate(over="ignore"):
        return np.float32(float(Fraction(x) / H))


def _sound(T, H, recip_term=True):
    ok, lo, E = _decide(T, H, recip_term=recip_term)
    if not ok:
        return True, False
    t, e = Fraction(float(T)), Fraction(float(E))
    return bool(_mean_exact(t - e, H) == lo and _mean_exact(t + e, H) == lo), True


def _boundary_sums(H, rng, n):
    """Sums T that put a float rounding boundary b of the mean (the midpoint
    of two adjacent floats) within a few double ulps of either end of the
    decision interval: T / H = b (1 -/+ c) with c = E / T, the relative
    half-width (about H ulps), shifted by -24..24 ulps; and T / H = b itself."""
    c = Fraction(H + 24, 2 ** 53) * (1 + Fraction(1, 2 ** 10))
    out = []
    for _ in range(n):
        m = np.float32(rng.uniform(0.5, 2.0) * 2.0 ** int(rng.integers(-90, 90)))
        up = np.nextafter(m, np.float32(np.inf))
        mid = (Fraction(float(m)) + Fraction(float(up))) / 2  # the rounding boundary
        out.append(float(mid * H))
        for sgn in (-1, 1):
            for k in range(-24, 25, 2):
                out.append(float(mid * H * (1 + sgn * c + Fraction(k, 2 ** 53))))
    return out


@pytest.mark.parametrize("H", [64, 1920, 3072, 4096, 5120, 12288])
def test_decided_means_are_exact_near_rounding_boundaries(H):
    rng = np.random.default_rng(H)
    sums = _boundary_sums(H, rng, 40)
    decided = 0
    for T in sums:
        sound, d = _sound(T, H)
        assert sound, (H, T)
        decided += d
    # Sums just inside an end go to the in-order sum, those just outside
    # are decided: both kinds occur.
    assert 0 < decided < len(sums)


@pytest.mark.parametrize("H", [64, 3072, 5120, 12288])
def test_random_sums_are_decided_and_exact(H):
    rng = np.random.default_rng(7 * H)
    n, decided = 3000, 0
    for _ in range(n):
        # From one denormal float square (2^-298) to squares of huge floats.
        T = float(rng.uniform(1.0, 2.0) * 2.0 ** int(rng.integers(-298, 250)))
        sound, d = _sound(T, H)
        assert sound, (H, T)
        decided += d
    assert decided >= n - 3  # a boundary within 5 ulps of the mean is rare


def test_zero_sum_is_decided_as_zero():
    ok, lo, _ = _decide(0.0, 5120)
    assert ok and lo == 0.0


def test_without_the_reciprocal_term_a_decision_goes_wrong():
    # The reciprocal's own rounding (up to ~2 ulps of the quotient) is what
    # the 2^-50 q term covers; without it some boundary sum is decided to
    # the wrong float.
    bad = 0
    for H in (3, 7, 1920, 3072, 5120, 12288):
        rng = np.random.default_rng(H + 1)
        for T in _boundary_sums(H, rng, 60):
            sound, _ = _sound(T, H, recip_term=False)
            bad += not sound
    assert bad > 0
