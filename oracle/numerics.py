"""Declared arithmetic of the sampling path (numpy restatement; test infrastructure).

The reference's sampler results depend on float rounding inside torch softmax,
torch CUDA cumsum and Triton tl.sum trees, none of which can be reproduced on
another machine. The kernels and this oracle therefore share one declared
arithmetic, made of operations that are exactly reproducible on both sides:

* IEEE binary32 +, -, *, / and sqrt with round-to-nearest-even, and fused
  multiply-add with a single rounding (``fma32`` emulates it exactly here);
* ``ls_exp``: an exponential built only from those operations (Cody-Waite
  range reduction, a degree-6 polynomial for e^r, exact scaling by 2^k);
* masses as exact integers: a weight w in [0, 1] contributes
  ``fx46(w) = floor(w * 2^46)``; sums of these are exact, so every reduction
  order gives the same result, and comparisons with u * total are exact;
* ``u64_to_f32``: round-to-nearest-even conversion of an exact integer mass.

Pinned by: tests/test_oracle_numerics.py (fma32 against exact rationals on
random and constructed midpoint cases; ls_exp within 2 ulp of math.exp over its
whole domain; fx46 and u64_to_f32 against Fraction arithmetic).
"""

from __future__ import annotations

import numpy as np

F32 = np.float32
F64 = np.float64

FX_BITS = 46
FX_ONE = 1 << FX_BITS

# ls_exp constants (binary32). LN2_HI has 16 significant bits so k*LN2_HI is
# exact for |k| <= 256; LN2_LO = ln 2 - LN2_HI rounded to binary32.
LOG2E = F32(1.44269504)
LN2_HI = F32(0.693145752)
LN2_LO = F32(1.42860677e-06)
EXP_MIN = F32(-87.0)
# e^r on [-0.35, 0.35], relative-error fit, coefficients rounded to binary32.
EXP_COEFFS = tuple(F32(c) for c in (
    1.0, 1.0, 0.4999999403953552, 0.1666642129421234,
    0.041668057441711426, 0.00837495643645525, 0.0013842721236869693,
))


def f32(x) -> np.ndarray:
    return np.asarray(x, dtype=F32)


def fma32(a, b, c) -> np.ndarray:
    """Binary32 fused multiply-add with one rounding, elementwise.

    The product a*b of two binary32 values is exact in binary64. The sum is
    formed in binary64 together with its exact error (TwoSum); the binary64
    sum can only round to a different binary32 value than the exact sum when
    it lands exactly on a binary32 midpoint, which is then decided by the sign
    of the error term.
    """
    a, b, c = (np.asarray(v, dtype=F32) for v in (a, b, c))
    a, b, c = np.broadcast_arrays(a, b, c)
    p = a.astype(F64) * b.astype(F64)
    cc = c.astype(F64)
    with np.errstate(over="ignore", invalid="ignore"):
        s = p + cc
        bp = s - p
        err = (p - (s - bp)) + (cc - bp)
        r = s.astype(F32)
        toward = np.where(s > r.astype(F64), F32(np.inf), F32(-np.inf)).astype(F32)
        nb = np.nextafter(r, toward)
        mid = (r.astype(F64) + nb.astype(F64)) * 0.5
        on_mid = (s == mid) & (s != r.astype(F64)) & np.isfinite(s)
        move = on_mid & (np.sign(err) == np.sign(s - r.astype(F64))) & (err != 0)
    return np.where(move, nb, r).astype(F32)


def ls_exp_k(t):
    """Return (e, k) where e = ls_exp(t) and k the binary exponent used in scaling.

    t is binary32 (normally t = x - max(x) <= 0). k = rint(t * LOG2E) with the
    product rounded to binary32 first; r = t - k*ln2 in two fused steps;
    e = P(r) * 2^k. Inputs below EXP_MIN (and NaN) give exactly 0.
    """
    t = np.asarray(t, dtype=F32)
    with np.errstate(invalid="ignore", over="ignore"):
        kf = np.rint((t * LOG2E).astype(F32)).astype(F32)
        kf_safe = np.where(np.isfinite(kf), kf, F32(0)).astype(F32)
        r = fma32(kf_safe, -LN2_HI, t)
        r = fma32(kf_safe, -LN2_LO, r)
        p = np.full_like(t, EXP_COEFFS[6])
        for coef in EXP_COEFFS[5::-1]:
            p = fma32(p, r, coef)
        e = np.ldexp(p, kf_safe.astype(np.int32)).astype(F32)
        keep = t >= EXP_MIN
    return np.where(keep, e, F32(0)).astype(F32), np.where(keep, kf_safe, F32(0)).astype(F32)


def ls_exp(t) -> np.ndarray:
    return ls_exp_k(t)[0]


def fx46(w) -> np.ndarray:
    """floor(w * 2^46) as uint64 for binary32 w in [0, 1] (exact)."""
    w = np.asarray(w, dtype=F32).astype(F64)
    return np.floor(w * float(FX_ONE)).astype(np.uint64)


def u64_to_f32(x: int) -> np.float32:
    """Round-to-nearest-even conversion of a non-negative integer to binary32."""
    x = int(x)
    if x < 0:
        raise ValueError("negative mass")
    if x == 0:
        return F32(0.0)
    nbits = x.bit_length()
    if nbits <= 24:
        return F32(float(x))
    shift = nbits - 24
    mant = x >> shift
    rem = x & ((1 << shift) - 1)
    half = 1 << (shift - 1)
    if rem > half or (rem == half and (mant & 1)):
        mant += 1
        if mant == (1 << 24):
            mant >>= 1
            shift += 1
    return F32(np.ldexp(F64(mant), shift))


def mass_to_f32(mass_fx: int) -> np.float32:
    """Binary32 value of an exact 2^-46 fixed-point mass (exact scaling)."""
    return F32(np.ldexp(F64(u64_to_f32(mass_fx)), -FX_BITS))


def floor_u_times(u: np.float32, total: int) -> int:
    """floor(u * total) exactly, for binary32 u in [0, 1) and an integer total."""
    u = F32(u)
    if u <= 0:
        return 0
    m, e = np.frexp(F64(u))  # u = m * 2^e, 0.5 <= m < 1
    mi = int(np.ldexp(m, 24))  # 24-bit integer mantissa
    shift = 24 - int(e)
    return (mi * int(total)) >> shift
