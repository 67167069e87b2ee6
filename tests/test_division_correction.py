"""The softmax kernels' quotient (csrc/hipo_common.h, div_rn): with
inv = RN(1/sum), q = RN(e * inv) and one FMA step with the exact remainder,
q' = RN(q + RN(e - q * sum) * inv), is the IEEE fp32 quotient RN(e / sum).

Checked with exact rational arithmetic (fractions.Fraction; RN = round to
nearest fp32, ties to even, and FMA = one rounding of the exact a * b + c)
over the softmax domain: e in (0, 1] -- uniform, and e^-u for u up to 80
(tiny exp values) -- and sum in [1, 2048], uniform and of the form
(1 + k 2^-23) 2^j (every significand pattern).  A planted mistake (dropping
the correction, or using the hardware-style reciprocal without the exact
remainder) must fail the same check."""
from __future__ import annotations

import math
import random
from fractions import Fraction

import numpy as np


def rn32(x: Fraction) -> np.float32:
    """Round an exact rational to the nearest fp32 (ties to even); normal range."""
    if x == 0:
        return np.float32(0.0)
    f = np.float32(float(x))  # within one fp32 ulp of x; fix it exactly
    cands = {float(f), float(np.nextafter(f, np.float32(np.inf))),
             float(np.nextafter(f, np.float32(-np.inf)))}
    best = min(cands, key=lambda c: (abs(Fraction(c) - x),
                                     int(np.float32(c).view(np.uint32)) & 1))
    return np.float32(best)


def fma(a, b, c) -> np.float32:
    return rn32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def div_rn(e, s):
    inv = rn32(Fraction(1) / Fraction(float(s)))
    q = rn32(Fraction(float(e)) * Fraction(float(inv)))
    return fma(fma(-q, s, e), inv, q)


def mul_only(e, s):
    inv = rn32(Fraction(1) / Fraction(float(s)))
    return rn32(Fraction(float(e)) * Fraction(float(inv)))


def samples(n: int, seed: int = 7):
    rng = random.Random(seed)
    for i in range(n):
        if i % 3:
            s = np.float32(rng.uniform(1.0, 2048.0))
        else:
            s = np.float32((1 + rng.randrange(1 << 23) / 2.0 ** 23) * 2.0 ** rng.randrange(11))
        e = np.float32(rng.random()) if i % 5 else np.float32(math.exp(-rng.uniform(0, 80)))
        if e > 0:
            yield e, s


def test_one_fma_correction_is_the_ieee_quotient():
    n = 0
    for e, s in samples(20000):
        want = rn32(Fraction(float(e)) / Fraction(float(s)))
        assert div_rn(e, s) == want, (float(e), float(s))
        n += 1
    assert n > 19000


def test_multiply_by_reciprocal_is_not():
    # The round-2 form, e * RN(1/sum), misses the IEEE quotient on a few
    # percent of inputs; the check above would catch its return.
    off = sum(mul_only(e, s) != rn32(Fraction(float(e)) / Fraction(float(s)))
              for e, s in samples(4000, seed=11))
    assert off > 40
