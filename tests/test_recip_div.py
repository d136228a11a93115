"""CPU check of the quantizers' division through the reciprocal (rt4_dev.h
div_by_recip): y = RN(1/s), t = RN(x*y), q = RN(t + RN(x - t*s)*y) with both
inner steps fused multiply-adds.  The quantizers take this form instead of the
IEEE quotient RN(x/s) that the reference's kernels compute (quant_act,
kernels/gemv_w4a8_core.h:34-66; quant_rows_a8_k, src/k_new.hip:268-301), so the
codes are bit-identical only where q == RN(x/s).

The fp32 sequence is emulated exactly on the CPU: products of two binary32 values
are exact in binary64, x - t*s is exact in binary64 (t is within a few ulp of
x/s), and the final rounding of t + r*y is resolved exactly with an error-free
two-sum in binary64 plus a rational tie-break.  The reference RN(x/s) is the
binary64 quotient rounded to binary32, with the rare cases where binary64's own
rounding could move it across a binary32 rounding boundary decided in exact
rational arithmetic.

Inputs target the places where a reciprocal-based quotient can go wrong:
quotients within a few ulp of every half-integer of the code range (where lrintf's
result changes), of every power of two (where t's ulp changes), scales with
all-ones significands, and the quantizers' own distributions (s = amax/127 and
amax/119 with x up to amax).  Every input lies in the range where the kernels use
this form (s in [2^-96, 2^100]).
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np

F32 = np.float32


def _rn32_of_f64_exact(a: np.ndarray, err: np.ndarray) -> np.ndarray:
    """RN to binary32 of the exact value a + err (a binary64, |err| <= ulp64(a)/2)."""
    f = a.astype(F32)
    # a binary32 midpoint is exactly representable in binary64; only a value of `a`
    # sitting exactly on one can round differently from a + err
    lo = np.nextafter(f, F32(-np.inf)).astype(np.float64)
    hi = np.nextafter(f, F32(np.inf)).astype(np.float64)
    f64 = f.astype(np.float64)
    mid_up = (f64 + hi) / 2
    mid_dn = (f64 + lo) / 2
    on_up = (a == mid_up) & (err > 0)    # a rounded down to f by the tie rule, value above the tie
    on_dn = (a == mid_dn) & (err < 0)
    out = f.copy()
    out[on_up] = hi[on_up].astype(F32)
    out[on_dn] = lo[on_dn].astype(F32)
    # a tie broken to even by astype but with err of the other sign is handled above;
    # a tie with err == 0 stays ties-to-even, as IEEE rounding does
    return out


def div_by_recip(x: np.ndarray, s: np.ndarray) -> np.ndarray:
    y = (F32(1) / s).astype(F32)                    # hipcc's division: correctly rounded
    t = (x * y).astype(F32)                          # RN(x*y)
    r64 = x.astype(np.float64) - t.astype(np.float64) * s.astype(np.float64)   # exact
    r = r64.astype(F32)                              # fma(-t, s, x): one rounding of the exact value
    ry = r.astype(np.float64) * y.astype(np.float64)  # exact
    t64 = t.astype(np.float64)
    a = t64 + ry                                     # two-sum: a + e == t + r*y exactly
    bb = a - t64
    e = (t64 - (a - bb)) + (ry - bb)
    return _rn32_of_f64_exact(a, e)


def exact_quotient(x: np.ndarray, s: np.ndarray) -> np.ndarray:
    """RN(x/s) to binary32 (ties to even), exactly."""
    q64 = x.astype(np.float64) / s.astype(np.float64)
    q = q64.astype(F32)
    # binary64's error is below 2^-53 relative; re-decide exactly wherever q64 lies
    # within 2^-40 (relative) of a binary32 rounding boundary
    f = q.astype(np.float64)
    hi = np.nextafter(q, F32(np.inf)).astype(np.float64)
    lo = np.nextafter(q, F32(-np.inf)).astype(np.float64)
    near = (np.abs(q64 - (f + hi) / 2) <= np.abs(q64) * 2.0 ** -40) | \
           (np.abs(q64 - (f + lo) / 2) <= np.abs(q64) * 2.0 ** -40)
    for i in np.nonzero(near)[0]:
        fr = Fraction(float(x[i])) / Fraction(float(s[i]))
        cands = [float(np.nextafter(q[i], F32(-np.inf))), float(q[i]), float(np.nextafter(q[i], F32(np.inf)))]
        best = min(cands, key=lambda c: (abs(Fraction(c) - fr), int(np.float32(c).view(np.uint32)) & 1))
        q[i] = F32(best)
    return q


def _ulps(v: np.ndarray, n: int) -> np.ndarray:
    """v and its n binary32 neighbours on each side, flattened."""
    out = [v]
    a = b = v
    for _ in range(n):
        a = np.nextafter(a, F32(np.inf))
        b = np.nextafter(b, F32(-np.inf))
        out += [a, b]
    return np.concatenate(out)


def _check(x, s):
    assert np.all((s >= 2.0 ** -96) & (s <= 2.0 ** 100)), "outside the reciprocal form's range"
    got = div_by_recip(x, s)
    want = exact_quotient(x, s)
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, (f"{bad.size} of {x.size} differ, e.g. x={x[bad[0]]!r} s={s[bad[0]]!r} "
                           f"got {got[bad[0]]!r} want {want[bad[0]]!r}")
    return x.size


def test_emulation_matches_ieee_for_random_operands():
    """The emulation itself against exact rational arithmetic on a few thousand cases."""
    rng = np.random.default_rng(0)
    x = rng.standard_normal(4000).astype(F32)
    s = (np.abs(rng.standard_normal(4000)) / 100 + 1e-3).astype(F32)
    got = div_by_recip(x, s)
    for i in range(0, 4000, 7):
        fr = Fraction(float(x[i])) / Fraction(float(s[i]))
        # the result is within one ulp of the exact quotient (faithful at worst)
        assert abs(Fraction(float(got[i])) - fr) <= Fraction(float(np.spacing(np.abs(got[i]))))
        # and exact_quotient is the correctly rounded quotient
        q = exact_quotient(x[i:i + 1], s[i:i + 1])[0]
        for c in (np.nextafter(q, F32(np.inf)), np.nextafter(q, F32(-np.inf))):
            assert abs(Fraction(float(q)) - fr) <= abs(Fraction(float(c)) - fr)


def test_quotients_near_half_integers_of_the_code_range():
    """x/s within +-8 ulp of k + 1/2 for every k in [-130, 129], across scales."""
    rng = np.random.default_rng(1)
    n = 0
    for scale_exp in (-90, -20, -7, 0, 5, 60, 95):
        s = (rng.uniform(1, 2, 40) * 2.0 ** scale_exp).astype(F32)
        k = np.arange(-130, 130) + 0.5
        S = np.repeat(s, k.size)
        Q = np.tile(k, s.size)
        x0 = (Q * S.astype(np.float64)).astype(F32)
        X = _ulps(x0, 8)
        n += _check(X, np.tile(S, 17))
    assert n > 500_000


def test_quotients_near_powers_of_two():
    """x/s within +-8 ulp of 2^j (where the ulp of the quotient changes)."""
    rng = np.random.default_rng(2)
    s = np.concatenate([(rng.uniform(1, 2, 400) * 2.0 ** rng.integers(-80, 80, 400)).astype(F32),
                        np.array([1.0, 1.5, np.nextafter(F32(2), F32(0))], F32)])
    j = np.arange(-12, 8)
    S = np.repeat(s, j.size)
    Q = np.tile(2.0 ** j, s.size) * np.sign(np.tile(rng.standard_normal(j.size), s.size))
    x0 = (Q * S.astype(np.float64)).astype(F32)
    _check(_ulps(x0, 8), np.tile(S, 17))


def test_scales_with_all_ones_significands():
    """s = (2^24 - 1) * 2^e and its neighbours, with quotients across the code range."""
    rng = np.random.default_rng(3)
    base = np.array([(2 ** 24 - 1) * 2.0 ** e for e in range(-100, 60, 7)], np.float64).astype(F32)
    s = _ulps(base, 2)
    S = np.repeat(s, 600)
    Q = np.tile(rng.uniform(-128, 128, 600), s.size)
    x = (Q * S.astype(np.float64)).astype(F32)
    _check(_ulps(x, 2), np.tile(S, 5))


def test_quantizer_distributions():
    """The quantizers' own inputs: s = amax/127 (decode) and amax/119 (prefill), x in
    [-amax, amax], including the element that is the max itself (quotient +-127/119)."""
    rng = np.random.default_rng(4)
    for div in (F32(127), F32(119)):
        amax = np.abs(rng.standard_normal(20000) * np.exp2(rng.integers(-30, 30, 20000))).astype(F32)
        amax = amax[amax > 0]
        s = (amax / div).astype(F32)
        xs = [(amax * rng.uniform(-1, 1, amax.size)).astype(F32), amax, -amax]
        for x in xs:
            _check(x, s)


def test_faithfulness_counterexample_still_rounds_correctly():
    """x/s just below a power of two, where t = RN(x*RN(1/s)) is more than one ulp from
    x/s (so the textbook premise of Markstein's theorem fails): the corrected
    quotient still equals RN(x/s)."""
    x = np.array([0.12499404698610306], F32)
    s = np.array([0.01562426146119833], F32)
    y = (F32(1) / s).astype(F32)
    t = (x * y).astype(F32)
    q = exact_quotient(x, s)
    assert abs(int(t.view(np.int32)[0]) - int(q.view(np.int32)[0])) >= 1
    _check(_ulps(x, 64), np.repeat(s, 129))


def test_planted_mistake_is_caught():
    """Without the correction step (q = t) the targeted inputs expose the error: the
    checks above are not vacuous."""
    rng = np.random.default_rng(5)
    s = (rng.uniform(1, 2, 200) * 2.0 ** rng.integers(-20, 20, 200)).astype(F32)
    k = np.arange(-128, 128) + 0.5
    S = np.repeat(s, k.size)
    x = _ulps((np.tile(k, s.size) * S.astype(np.float64)).astype(F32), 2)
    S = np.tile(S, 5)
    t = (x * (F32(1) / S).astype(F32)).astype(F32)
    assert np.count_nonzero(t.view(np.uint32) != exact_quotient(x, S).view(np.uint32)) > 1000
