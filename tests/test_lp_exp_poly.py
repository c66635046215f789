"""The bounded exp (artemis_amd/csrc/exp_poly.h, ExpPoly::exp_neg) that the log-probability kernel and
the finish kernel's histogram passes use takes 2^f for |f| <= 1/2 from a degree-8 polynomial whose
coefficients are written in that source. Its documented per-term bound kExpPolyRel (1.5e-12 relative,
which include/artemis_sampler.h's logprob bound e carries) rests on the polynomial's own relative
error, 1.064e-12 at most: this checks that error, evaluated exactly (mpmath) with the coefficients as
the source holds them, over a grid of the interval and at its ends. A wrong or mistyped coefficient
shows up as an error many times larger."""
import os
import re

import numpy as np
import pytest

mp = pytest.importorskip("mpmath")

SRC = os.path.join(os.path.dirname(__file__), "..", "artemis_amd", "csrc", "exp_poly.h")


def coefficients():
    text = open(SRC).read()
    body = re.search(r"__constant__ double kExp2Poly\[kPolyLen\] = \{([^}]*)\}", text).group(1)
    return [float(c) for c in body.replace("\n", " ").split(",") if c.strip()]


def test_the_polynomial_of_2_to_the_f_is_within_its_documented_error():
    c = coefficients()
    assert len(c) == 9 and c[-1] == 1.0
    mp.mp.dps = 30
    worst = mp.mpf(0)
    points = [mp.mpf(i) / 4000 - mp.mpf(1) / 2 for i in range(4001)]
    for t in points:
        p = mp.mpf(0)
        for a in c:
            p = p * t + mp.mpf(a)
        worst = max(worst, abs(p / mp.power(2, t) - 1))
    assert worst < 1.07e-12, float(worst)
    # The kernel's kExpRel adds the rounding of t = d log2(e) and of the Horner steps.
    kexprel = float(re.search(r"constexpr double kExpPolyRel = ([0-9.e-]+);", open(SRC).read()).group(1))
    assert worst + 1.6e-13 + 1e-15 <= kexprel


def test_the_fused_argument_stays_within_its_documented_error():
    # exp_fused takes t = fma(x, L, c) with L = f64(log2 e) and c = f64(-m L), one rounding, for parts
    # whose maximum has |m| <= kFusedMax. Its distance to (x - m) log2 e, moved through 2^t, is the
    # source's kFusedArgRel at most where the term is above 2^-1100 (|t| <= 1100, x >= m - 763). This
    # computes the fused rounding exactly (Fraction, then one correctly rounded conversion) at the
    # corners of that domain and at random points, and checks the polynomial error plus it against
    # kExpPolyRel.
    from fractions import Fraction
    import random

    text = open(SRC).read()
    fmax = float(re.search(r"constexpr double kFusedMax = ([0-9.e-]+);", text).group(1))
    arg_rel = float(re.search(r"constexpr double kFusedArgRel = ([0-9.e-]+);", text).group(1))
    kexprel = float(re.search(r"constexpr double kExpPolyRel = ([0-9.e-]+);", text).group(1))
    L = float(re.search(r"constexpr double kLog2e = ([0-9.e-]+);", text).group(1))
    mp.mp.dps = 50
    log2e = 1 / mp.log(2)
    rng = random.Random(7)
    cases = []
    for m in [fmax, -fmax, fmax / 3, 0.0, -1.0]:
        for d in [0.0, -1e-3, -1.0, -700.0, -762.0, -763.0]:
            cases.append((m, d))
    for _ in range(3000):
        cases.append((rng.uniform(-fmax, fmax), -rng.uniform(0, 763)))
    worst = 0.0
    for m, d in cases:
        m = float(np.float32(m))
        x = float(np.float32(m + d))
        if x > m:
            continue
        c = float(Fraction(-m) * Fraction(L))
        t = float(Fraction(x) * Fraction(L) + Fraction(c))
        exact = (mp.mpf(x) - mp.mpf(m)) * log2e
        if exact < -1100:
            continue
        rel = abs(mp.mpf(t) - exact) * mp.log(2)
        worst = max(worst, float(rel))
    assert worst <= arg_rel, worst
    assert 1.07e-12 + arg_rel + 1e-15 <= kexprel
