"""CPU: the FP8 quantizers' quotient (``div_by`` in csrc/afd_common.h) against IEEE division.

The kernels compute v / s for every value of a 1x128 group as y = 1 / s (an IEEE division,
once per group), q0 = RN(v y), t = fma(q0, s, -v), q = fma(-t, y, q0). Here fma is
evaluated exactly (rationals) and rounded once to float32, and q is compared bit for bit with
numpy's float32 division (IEEE round-to-nearest-even) on random operands, operands whose
quotient lies next to a float32 rounding midpoint, the FP8 quantizers' extreme scales, and
zeros of both signs. The GPU build was also checked on every pair of fp32 significands."""

from fractions import Fraction

import numpy as np

F32_MIN_NORMAL = Fraction(2) ** -126


def rn32(v: Fraction) -> np.float32:
    """The float32 nearest to the rational v, ties to even (normal range)."""
    f = np.float32(float(v))  # within one float32 step of the answer
    best = None
    for c in (np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))):
        d = abs(Fraction(float(c)) - v)
        if best is None or d < best[0] or (d == best[0] and (int(c.view(np.uint32)) & 1) == 0):
            best = (d, c)
    return np.float32(best[1])


def fma(a, b, c) -> np.float32:
    """RN(a b + c) of float32 operands. An exact zero is -0 only when a b and c are both
    zeros of negative sign (IEEE 754: an exact zero sum of opposite signs is +0 under
    round-to-nearest, and x + x keeps the sign of x)."""
    exact = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
    if exact == 0:
        prod_is_neg_zero = (a == 0 or b == 0) and bool(np.signbit(a)) != bool(np.signbit(b))
        return np.float32(-0.0) if prod_is_neg_zero and c == 0 and np.signbit(c) else np.float32(0.0)
    return rn32(exact)


def div_by(v: np.float32, s: np.float32, y: np.float32) -> np.float32:
    q0 = np.float32(v * y)
    t = fma(q0, s, -v)
    return fma(-t, y, q0)


def check(vs, ss):
    bad = []
    for v, s in zip(vs, ss):
        v, s = np.float32(v), np.float32(s)
        y = np.float32(np.float32(1.0) / s)
        got, want = div_by(v, s, y), np.float32(v / s)
        if got.view(np.uint32) != want.view(np.uint32):
            bad.append((float(v), float(s), float(got), float(want)))
    return bad


def test_rn32_rounds_to_nearest_even():
    one = Fraction(1)
    ulp = Fraction(2) ** -23
    assert rn32(one + ulp / 2) == np.float32(1.0)  # tie -> even
    assert rn32(one + 3 * ulp / 2) == np.float32(1.0 + 2 * float(ulp))
    assert rn32(one + ulp / 2 + Fraction(1, 2**60)) == np.float32(1.0 + float(ulp))


def test_fma_model_signed_zeros():
    f32 = np.float32
    assert np.signbit(fma(f32(-0.0), f32(2.0), f32(-0.0)))  # -0 + -0
    assert not np.signbit(fma(f32(0.0), f32(2.0), f32(-0.0)))  # +0 + -0
    assert not np.signbit(fma(f32(-0.0), f32(-2.0), f32(-0.0)))  # +0 + -0
    assert not np.signbit(fma(f32(1.5), f32(2.0), f32(-3.0)))  # exact cancellation
    assert not np.signbit(fma(f32(-1.5), f32(2.0), f32(3.0)))
    assert fma(f32(3.0), f32(1.0 / 3.0), f32(-1.0)) == f32(2.0**-25)  # unrounded product


def test_random_operands_of_fp8_groups():
    rng = np.random.default_rng(5)
    amax = np.exp2(rng.uniform(-20, 20, 3000)).astype(np.float32)
    s = (np.maximum(amax, np.float32(1e-10)) / np.float32(448.0)).astype(np.float32)
    v = (amax * rng.uniform(-1, 1, 3000)).astype(np.float32)
    assert not check(v, s)


def test_quotients_next_to_rounding_midpoints():
    rng = np.random.default_rng(6)
    vs, ss = [], []
    for _ in range(1500):
        s = np.float32(rng.uniform(1, 2))
        q = np.float32(rng.uniform(1, 2))
        mid = (Fraction(float(q)) + Fraction(float(np.nextafter(q, np.float32(3))))) / 2
        for t in (-2, -1, 0, 1, 2):  # v whose exact quotient is at or beside the midpoint
            v = rn32(mid * Fraction(float(s))) if t == 0 else np.float32(
                float(rn32(mid * Fraction(float(s)))) * (1 + t * 2.0**-24))
            vs.append(v)
            ss.append(s)
    assert not check(vs, ss)


def test_extreme_scales_and_zeros():
    s_min = np.float32(np.float32(1e-10) / np.float32(448.0))
    cases = [(0.0, 1.0), (-0.0, 1.0), (0.0, float(s_min)), (-0.0, 3.5), (448.0, 1.0),
             (-448.0, 1.0), (float(s_min) * 448, float(s_min)), (1e-30, float(s_min)),
             (3.0e38, 1.0e30), (-1.5, 1.3333334)]
    bad = check([c[0] for c in cases], [c[1] for c in cases])
    assert not bad, bad
    z = div_by(np.float32(-0.0), np.float32(2.0), np.float32(0.5))
    assert z == 0 and np.signbit(z)
    z = div_by(np.float32(0.0), np.float32(2.0), np.float32(0.5))
    assert z == 0 and not np.signbit(z)


def test_quotients_stay_below_the_e4m3_rounding_limit():
    """The FP8 gate_up epilogue converts v / s to e4m3 without a clamp: with s = RN(max(amax,
    1e-10) / 448) every |v| <= amax gives |v / s| <= 448 (1 + 2^-23), and round to nearest
    even takes all of (448, 464) to 448 (the codes of both conversions compared bit for bit on
    the GPU's layer cases)."""
    rng = np.random.default_rng(7)
    amax = np.concatenate([np.exp2(rng.uniform(-40, 40, 200000)),
                           np.float32(448.0) * np.exp2(rng.integers(-30, 30, 2000)).astype(np.float64)])
    amax = amax.astype(np.float32)
    s = (np.maximum(amax, np.float32(1e-10)) / np.float32(448.0)).astype(np.float32)
    q = (amax / s).astype(np.float32)  # numpy float32 division: IEEE round to nearest even
    limit = np.float32(448.0) * (1 + np.float32(2.0**-23))
    assert q.max() <= limit < 464
    assert (q > 448).any()  # the overshoot does occur: the conversion must round it to 448
