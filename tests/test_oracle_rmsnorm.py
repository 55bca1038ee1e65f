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


def _kernel_tree_sum(x):
    """The double sum of squares in the order of the GPU RMSNorm's shortcut:
    thread t of 1024 sums the terms t, t + 1024, ... in order, a 64-lane
    butterfly (lane l adds lane l ^ d for d = 32, 16, .., 1) gives each
    wave's total, and the 16 wave totals are added in order."""
    H = len(x)
    per = -(-H // 1024)
    t = np.zeros(1024 * per)
    t[:H] = x.astype(np.float64) ** 2
    runs = t.reshape(per, 1024)
    loc = np.zeros(1024)
    for i in range(per):  # each thread's run, in order
        loc = loc + runs[i]
    total = 0.0
    lanes = np.arange(64)
    for w in range(16):
        v = loc[64 * w:64 * (w + 1)].copy()
        for d in (32, 16, 8, 4, 2, 1):
            v = v + v[lanes ^ d]
        total = total + float(v[0])
    return total, per


def _bound_rows(rng, H):
    rows = [rng.standard_normal(H).astype(F), np.ones(H, F),
            (rng.standard_normal(H) * np.exp(rng.uniform(-40, 40, H))).astype(F)]
    r = np.full(H, 2.0 ** -30, F)
    r[0] = 1.0
    rows.append(r)  # every term after the 1 rounds away in order, not in the tree
    ties = np.where(rng.random(H) < 0.5, F(2.0 ** -26), F(3 * 2.0 ** -26)).astype(F)
    ties[0] = 1.5
    rows.append(ties)
    r = rng.standard_normal(H).astype(F)
    r[H // 2] = 1e18
    rows.append(r)
    return rows


@pytest.mark.parametrize("H", [1, 7, 1000, 1025, 5120, 8192])
def test_tree_sum_bound_holds_and_decides_the_mean(orc, H):
    """The GPU RMSNorm's shortcut: with T its tree sum, the reference's
    in-order sum ss lies within E = (H + per + 24) 2^-53 T (1 + 2^-10) of T,
    so when (float)((T - E)/H) == (float)((T + E)/H), that is
    (float)(ss / H).  Checked against the oracle's in-order sum; the row of
    terms that round away in order (but add up in the tree) needs the H
    term of E: a bound of the tree's own depth alone is too small there."""
    rng = np.random.default_rng(H)
    for i, x in enumerate(_bound_rows(rng, H)):
        ss = float(orc.sumsq(x[None, :])[0])
        T, per = _kernel_tree_sum(x)
        E = (H + per + 24) * 2.0 ** -53 * T * (1 + 2.0 ** -10)
        assert abs(T - ss) <= E, (H, i, T, ss)
        lo, hi = np.float32((T - E) / H), np.float32((T + E) / H)
        if lo == hi:
            assert lo == np.float32(ss / H), (H, i)
        if i == 3 and H in (5120, 8192):
            assert abs(T - ss) > (per + 24) * 2.0 ** -53 * T, (H, T, ss)
