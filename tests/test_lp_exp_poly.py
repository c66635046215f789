"""The bounded exp (artemis_amd/csrc/exp_poly.h, ExpPoly::exp_neg) that the log-probability kernel and
the finish kernel's histogram passes use takes 2^f for |f| <= 1/2 from a degree-8 polynomial whose
coefficients are written in that source. Its documented per-term bound kExpPolyRel (1.5e-12 relative,
which include/artemis_sampler.h's logprob bound e carries) rests on the polynomial's own relative
error, 1.064e-12 at most: this checks that error, evaluated exactly (mpmath) with the coefficients as
the source holds them, over a grid of the interval and at its ends. A wrong or mistyped coefficient
shows up as an error many times larger."""
import os
import re

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
