"""Pins of the oracle's fixed-point arithmetic against libm and exact rationals.

DETEXP_FIX(d) must equal round(e^d * 2^40) up to the fp32 evaluation error of
the polynomial (a few 1e-7 relative); floor_mul must equal the exact rational
floor for every input it is given.
"""

import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle as O


def test_detexp_zero_is_one():
    assert O.detexp_fix(0.0) == 1 << 40
    assert O.detexp_fix(-0.0) == 1 << 40


def test_detexp_matches_exp_on_dense_grid():
    rng = np.random.default_rng(0)
    ds = np.concatenate([
        -np.linspace(0, 29.9, 4001, dtype=np.float32),
        -rng.random(4000, dtype=np.float32) * 3,
        -np.float32([1e-7, 1e-5, 0.5, math.log(2), 0.34657, 0.34658, 1.0, 10.0, 27.7]),
    ])
    worst = 0.0
    for d in ds:
        w = O.detexp_fix(float(d))
        ref = math.exp(float(d)) * 2.0**40
        # integer rounding (<= 0.5) plus the fp32 polynomial error (relative)
        assert abs(w - ref) <= 0.5 + ref * 2.5e-7, (d, w, ref)
        if ref > 2**32:  # where the integer rounding is negligible
            worst = max(worst, abs(w - ref) / ref)
    assert worst < 2e-7, worst


def test_detexp_monotone_and_cutoff():
    ds = -np.linspace(0, 31, 20001, dtype=np.float32)
    ws = [O.detexp_fix(float(d)) for d in ds]
    assert all(a >= b for a, b in zip(ws, ws[1:]))
    assert O.detexp_fix(-30.0001) == 0
    assert O.detexp_fix(float("-inf")) == 0
    # e^-28.5 * 2^40 = 0.46 -> rounds to 0; e^-27 * 2^40 = 2.07 -> 2
    assert O.detexp_fix(-28.5) == 0
    assert O.detexp_fix(-27.0) == 2


@pytest.mark.parametrize("f", [0.0, 2.0**-24, 0.5, 0.9, 0.95, 0.999999940395, 1e-30, 1e-42])
def test_floor_mul_exact(f):
    f32 = np.float32(f)
    for W in [1, 3, (1 << 40) + 12345, (1 << 58) - 1, 123456789012345678]:
        want = math.floor(Fraction(float(f32)) * W)
        assert O.floor_mul(float(f32), W) == want
