"""The oracle's RMSNorm (kernel/qwen35_decoder.cpp:134-140), pinned.

The reference sums the squares in double one element after the other, so
the sum carries that order's roundings.  The crafted rows below have sums
fixed by IEEE round-to-nearest-even alone, worked out with exact rationals:
an exact (or pairwise, or compensated) sum gives a different double, and so
does a tie rounded the wrong way.
"""
from fractions import Fraction

import numpy as np
import pytest

from conftest import bits_equal

F = np.float32


def _round_double(v, u):
    """Fraction v rounded to a multiple of u, ties to even (IEEE binary64
    within one binade, u its unit in the last place)."""
    q, r = divmod(v, u)
    if r * 2 > u or (r * 2 == u and q % 2 == 1):
        q += 1
    return q * u


def test_tie_rounds_to_even_and_keeps_the_sum(orc):
    # 1.5^2 = 2.25 lies in [2, 4) where u = 2^-51; 2.25/u = 9*2^49 is even.
    # Each (2^-26)^2 = 2^-52 = u/2 is an exact tie and rounds back to 2.25.
    x = np.array([1.5] + [2.0 ** -26] * 100, F)
    assert orc.sumsq(x[None, :])[0] == 2.25
    # The exact sum is 2.25 + 100 * 2^-52, a double itself.
    assert float(np.sum(x.astype(np.float64) ** 2)) != 2.25


def test_tie_after_an_odd_partial_sum_rounds_up(orc):
    # t1 = ((2^23 + 5) * 2^-28)^2 / u = 2^41 + 5*2^19 + 25/32: it rounds up
    # to an odd multiple of u, so the following tie rounds up by one u.
    u = Fraction(1, 2 ** 51)
    x1 = F((2 ** 23 + 5) * 2.0 ** -28)
    t1 = Fraction(float(x1)) ** 2
    s1 = _round_double(Fraction(9, 4) + t1, u)
    assert (s1 / u) % 2 == 1
    s2 = _round_double(s1 + Fraction(1, 2 ** 52), u)
    assert s2 == s1 + u
    x = np.array([1.5, x1, 2.0 ** -26], F)
    assert Fraction(orc.sumsq(x[None, :])[0]) == s2


def test_vanishing_terms_leave_the_sum_unchanged(orc):
    # After s = 1 (u = 2^-52), each 2^-60 rounds away.
    x = np.full(5120, 2.0 ** -30, F)
    x[0] = 1.0
    assert orc.sumsq(x[None, :])[0] == 1.0
    # The same terms first, then 1: they add up exactly before the 1 arrives.
    y = np.concatenate([x[1:], x[:1]])
    assert orc.sumsq(y[None, :])[0] == 1.0 + 5119 * 2.0 ** -60


def test_closed_form_outputs(orc):
    H, eps = 512, F(1e-6)
    w = np.linspace(-2, 2, H, dtype=F)
    out = orc.rmsnorm(np.ones((1, H), F), w, eps)[0]
    inv = F(1) / np.sqrt(F(1) + eps)  # ss / H = 1 exactly
    assert bits_equal(out, (F(1) * inv) * w)
    # Zero row: inv = 1/sqrt(eps), out = 0 * inv * w (signed zeros kept).
    z = orc.rmsnorm(np.zeros((1, H), F), w, eps)[0]
    assert bits_equal(z, (F(0) * (F(1) / np.sqrt(eps))) * w)


@pytest.mark.parametrize("H", [1, 3, 64, 257])
def test_oracle_matches_a_sequential_double_sum(orc, H):
    rng = np.random.default_rng(H)
    x = (rng.standard_normal((4, H)) * np.exp(rng.uniform(-8, 8, (4, H)))).astype(F)
    w = rng.standard_normal(H).astype(F)
    eps = F(1e-6)
    got = orc.rmsnorm(x, w, eps)
    for i in range(4):
        ss = 0.0
        for v in x[i]:
            ss += float(v) * float(v)
        inv = F(1) / np.sqrt(F(ss / H) + eps)
        assert bits_equal(got[i], (x[i] * inv) * w)


def test_non_finite_rows(orc):
    H, eps = 64, F(1e-6)
    w = np.ones(H, F)
    x = np.ones((3, H), F)
    x[0, 5] = np.inf
    x[1, 7] = np.nan
    x[2, 9] = np.inf
    x[2, 11] = np.nan
    out = orc.rmsnorm(x, w, eps)
    # inf: inv = 1/inf = 0, finite entries 0, the inf one inf*0 = NaN.
    assert np.all(out[0][np.isfinite(x[0])] == 0) and np.isnan(out[0, 5])
    assert np.all(np.isnan(out[1])) and np.all(np.isnan(out[2]))
