"""The correctly rounded quotient the kernels use in place of a double division (div_rn in
stems.cpp_amd/csrc/common.hpp): q0 = RN(x r) with r = RN(1/h), then RN(q0 + r RN(x - q0 h)),
and q0 itself when q0 is not finite. Restated here with exact fused multiply-adds (rational
arithmetic, one rounding to double) and checked against IEEE division (Python's float /) on
random doubles over many binades and on the denominators the kernels divide by: band counts
per bin (1, 2), UVR window sums (sums of np.hanning values), HTDemucs 1e-5 + sd, and the
resampler's half-widths; plus infinite and NaN numerators (fma(-inf, h, inf) is NaN, so a
non-finite q0 must be returned as it is).
This pins Markstein's argument; the GPU parity tests pin the kernels themselves."""
import math
import random
from fractions import Fraction

import numpy as np


def rn(v):
    """Round an exact rational to the nearest double (ties to even), as float() does."""
    return float(v)


def fma(a, b, c):
    return rn(Fraction(a) * Fraction(b) + Fraction(c))


def div_rn(x, h, r):
    q0 = x * r
    if not math.isfinite(q0):
        return q0
    return fma(fma(-q0, h, x), r, q0)


def check(xs, hs):
    for h in hs:
        r = 1.0 / h
        for x in xs:
            got, want = div_rn(x, h, r), x / h
            assert got == want or (math.isnan(got) and math.isnan(want)), (x, h, got, want)


def test_random_binades():
    rng = random.Random(5)
    xs = [rng.uniform(-1, 1) * 2.0 ** rng.randint(-60, 60) for _ in range(400)]
    hs = [rng.uniform(0.5, 1) * 2.0 ** rng.randint(-30, 30) for _ in range(60)]
    check(xs, hs)


def test_kernel_denominators():
    rng = random.Random(6)
    xs = [rng.gauss(0, 1) * rng.choice([1e-3, 1, 7, 1e3]) for _ in range(300)]
    han = np.hanning(7680)
    sums = [float(han[i] + han[(i + 3840) % 7680]) for i in range(1, 7680, 97)]
    sums += [float(han[i]) for i in range(1, 7680, 211)]
    dens = [1e-5 + rng.uniform(0.01, 3.0) for _ in range(30)]
    halves = [44100 / 48000 * 64.0, 22050 / 44100 * 64.0, 64.0, 48000 / 44100 * 8.0]
    check(xs, [1.0, 2.0] + sums + dens + halves)


def test_non_finite_numerators():
    check([math.inf, -math.inf, math.nan, 1e308, -1e308], [1.0, 2.0, 0.75, 1e-5 + 0.3, 3e-300])
