"""Pin the declared arithmetic of the oracle against exact rational arithmetic."""

import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import numerics as nm
from loopspec_amd import philox


def exact_rne_f32(x: Fraction) -> np.float32:
    """Round an exact rational to binary32, ties to even (normal range)."""
    if x == 0:
        return np.float32(0.0)
    sign = -1 if x < 0 else 1
    x = abs(x)
    e = math.floor(math.log2(x.numerator) - math.log2(x.denominator))
    while Fraction(2) ** e > x:
        e -= 1
    while Fraction(2) ** (e + 1) <= x:
        e += 1
    ulp = Fraction(2) ** (e - 23)
    q, r = divmod(x, ulp)
    q = int(q)
    if r > ulp / 2 or (r == ulp / 2 and q % 2 == 1):
        q += 1
    return np.float32(sign * float(q * ulp))


def test_fma32_random_against_exact():
    rng = np.random.default_rng(0)
    a = (rng.standard_normal(3000) * 4).astype(np.float32)
    b = (rng.standard_normal(3000) * 4).astype(np.float32)
    c = (rng.standard_normal(3000) * 4).astype(np.float32)
    got = nm.fma32(a, b, c)
    for i in range(3000):
        want = exact_rne_f32(Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i])))
        assert got[i] == want, (a[i], b[i], c[i])


def test_fma32_midpoint_cases():
    # a*b = 1 + 2^-11 + 2^-24 is exactly halfway between two binary32 values.
    a = np.float32(1 + 2 ** -12)
    for c, want in [(0.0, 1 + 2 ** -11), (2.0 ** -60, 1 + 2 ** -11 + 2 ** -23), (-(2.0 ** -60), 1 + 2 ** -11)]:
        exact = Fraction(float(a)) ** 2 + Fraction(c)
        assert exact_rne_f32(exact) == np.float32(want)
        assert nm.fma32(a, a, np.float32(c)) == np.float32(want), c
    # a separate double-rounding trap: naive float64 then float32 gets this wrong
    naive = np.float32(np.float64(a) * np.float64(a) + np.float64(np.float32(2.0 ** -60)))
    assert naive != np.float32(1 + 2 ** -11 + 2 ** -23)


def test_exp2_accuracy_and_special_points():
    rng = np.random.default_rng(1)
    t = np.concatenate([
        -rng.random(200000).astype(np.float32) * 126,
        -rng.random(50000).astype(np.float32) * 2,
        np.float32([0.0, -0.0, -1e-30, -0.5, -1.5, -2.5, -0.49999997, -125.5, -126.0]),
    ]).astype(np.float32)
    e, k = nm.exp2q_k(t)
    ref = np.exp2(t.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    err = np.abs(e.astype(np.float64) - ref) / ulp
    assert err.max() <= 4.0, err.max()
    # k is the rounded argument (half to even) and e / 2^k is the polynomial's range
    assert np.array_equal(k, np.rint(t).astype(np.int32))
    scaled = np.ldexp(e.astype(np.float64), -k)
    assert scaled.min() >= 2 ** -0.5 * (1 - 1e-6) and scaled.max() <= nm.EXP2_POLY_MAX
    # integers are exact powers of two; the floor, -inf and NaN give 0
    ints = -np.arange(0, 127, dtype=np.float32)
    assert np.array_equal(nm.exp2q(ints), np.ldexp(np.float32(1), ints.astype(np.int32)).astype(np.float32))
    assert (nm.exp2q(np.float32([-200.0, -1e30, -np.inf, np.nan])) == 0).all()
    assert nm.exp2q(np.float32([-149.0]))[0] == np.float32(2.0 ** -149)  # denormals keep their exact value
    # e^(x/T) = 2^(c x): the temperature scale agrees with the natural exponential
    x = (rng.standard_normal(10000) * 3).astype(np.float32)
    c = np.float32(nm.LOG2E * (np.float32(1) / np.float32(0.7)))
    got = nm.exp2q(nm.fma32(x, c, np.float32(0)))
    want = np.exp(x.astype(np.float64) / 0.7)
    assert np.max(np.abs(got / want - 1)) < 3e-6


def test_tree_sum_order():
    rng = np.random.default_rng(5)

    def pairwise(v):
        if len(v) == 1:
            return np.float32(v[0])
        h = len(v) // 2
        return np.float32(pairwise(v[:h]) + pairwise(v[h:]))

    for n in (1, 2, 8, 32, 256):
        a = (rng.random(n) * 10.0 ** rng.integers(-8, 3, n)).astype(np.float32)
        assert nm.tree_sum_f32(a) == pairwise(list(a))
    # the order is observable: 1 + 2^-24 + 2^-24 depends on the grouping
    tiny = np.float32(2.0 ** -24)
    assert nm.tree_sum_f32(np.float32([1, tiny, tiny, 0])) == np.float32(1)
    assert nm.tree_sum_f32(np.float32([1, 0, tiny, tiny])) == np.float32(1 + 2.0 ** -23)


def test_fixed_point_and_conversions():
    rng = np.random.default_rng(2)
    w = np.concatenate([rng.random(2000).astype(np.float32), np.float32([0, 1, 2 ** -46, 2 ** -47, 1e-20])])
    fx = nm.fx46(w)
    for i in range(len(w)):
        assert int(fx[i]) == math.floor(Fraction(float(w[i])) * 2 ** 46)
    for x in list(rng.integers(0, 2 ** 63, 2000)) + [2 ** 24 + 1, 2 ** 24 + 3, 2 ** 25 + 2, 2 ** 63 - 1, 1, 0]:
        assert nm.u64_to_f32(int(x)) == exact_rne_f32(Fraction(int(x))) if x else nm.u64_to_f32(0) == 0
    for u in list(rng.random(500).astype(np.float32)) + [np.float32(0.0), np.float32(1 - 2 ** -24), np.float32(1e-40)]:
        total = int(rng.integers(1, 2 ** 63))
        assert nm.floor_u_times(u, total) == math.floor(Fraction(float(u)) * total)


def test_philox_known_answers():
    # Known-answer vectors of Philox4x32-10 (Salmon et al., Random123 distribution).
    cases = [
        ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
        ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
        ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
         (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
    ]
    for ctr, key, want in cases:
        got = philox.philox4x32(np.array([ctr], dtype=np.uint32), np.array(key, dtype=np.uint32))[0]
        assert tuple(int(x) for x in got) == want
    u = philox.uniforms((1000,), seed=5)
    assert u.dtype == np.float32 and (u >= 0).all() and (u < 1).all()
    assert np.array_equal(philox.uniforms((10,), seed=5, offset=3), u[3:13])


def test_exp2_polynomial_bound_for_candidate_scale():
    """The chunk kernel keeps every e >= 1.41422 * 2^-K as a candidate and
    relies on e < 1.41422 * 2^k whenever exp2q scaled by 2^k: the polynomial
    must stay below 1.41422 on [-1/2, 1/2]. Exhaustive over the binary32
    arguments of [1/4, 1/2] (where the maximum lies), sampled below."""
    top = np.arange(np.float32(0.25).view(np.uint32), np.float32(0.5).view(np.uint32) + 1,
                    dtype=np.uint32).view(np.float32)
    low = np.linspace(-0.5, 0.25, 200001, dtype=np.float64).astype(np.float32)
    for r in (top, low):
        p = np.full_like(r, nm.EXP2_COEFFS[5])
        for coef in nm.EXP2_COEFFS[4::-1]:
            p = nm.fma32(p, r, coef)
        assert float(p.max()) < 1.41422
