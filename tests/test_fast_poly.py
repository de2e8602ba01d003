"""The fast path's polynomial error claims, checked on the CPU.

luma_fast.h evaluates expm1 and log1p on (0, 1/8] with float32 Horner
polynomials and charges 3u (u = 2^-24) for each in its error bounds.  This
test reads the coefficients from the header, emulates the GPU evaluation
(fused multiply-add: exact product and sum, one rounding) and checks the
relative error against float64 on a dense grid plus random points.
"""

import os
import re

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
HEADER = os.path.join(HERE, "..", "luma_amd", "csrc", "luma_fast.h")
U = 2.0 ** -24
BOUND = 3.0 * U        # fast_expm1_relerr / fast_log1p_relerr for x_top <= kSmall


def _coeffs(name):
    text = open(HEADER).read()
    m = re.search(name + r"\[\d+\]\s*=\s*\{([^}]*)\}", text)
    assert m, name
    return [np.float32(float(v.strip().rstrip("f"))) for v in m.group(1).split(",")]


def _small_tier():
    text = open(HEADER).read()
    return float(re.search(r"kSmall\s*=\s*([0-9.e-]+)f", text).group(1))


def _horner_f32(coef, x):
    acc = np.full(x.shape, coef[-1], dtype=np.float32)
    for c in reversed(coef[:-1]):
        # fmaf: the float64 product/sum of float32 values is exact to 48 bits,
        # so one rounding to float32 models the fused operation
        acc = (acc.astype(np.float64) * x.astype(np.float64) + np.float64(c)).astype(np.float32)
    return (x.astype(np.float64) * acc.astype(np.float64)).astype(np.float32)


def _points():
    top = _small_tier()
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.uniform(0.0, top, 2_000_000),
                        np.linspace(0.0, top, 200_001),
                        np.geomspace(1e-30, top, 100_000)]).astype(np.float32)
    return x[x > 0]


@pytest.mark.parametrize("name,ref", [("kExpm1Poly", np.expm1), ("kLog1pPoly", np.log1p)])
def test_polynomial_error_within_bound(name, ref):
    x = _points()
    got = _horner_f32(_coeffs(name), x).astype(np.float64)
    want = ref(x.astype(np.float64))
    rel = np.abs(got - want) / want
    assert rel.max() < BOUND, (name, rel.max() / U)


def test_small_tier_is_one_eighth():
    assert _small_tier() == 0.125


def _medium_points(top):
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.uniform(0.0, top, 2_000_000),
                        np.linspace(0.0, top, 200_001),
                        np.geomspace(1e-30, top, 100_000)]).astype(np.float32)
    return x[x > 0]


def test_medium_expm1_polynomial_within_small_bound():
    """The medium regime's degree-5 expm1 on (0, 1/2]: within the 3u that
    make_bounds charges when x_top <= 1/8 (and so within the 10.5u or more
    it charges above)."""
    x = _medium_points(0.5)
    got = _horner_f32(_coeffs("kExpm1PolyMed"), x).astype(np.float64)
    want = np.expm1(x.astype(np.float64))
    rel = np.abs(got - want) / want
    assert rel.max() < BOUND, rel.max() / U


def test_medium_log1p_series_truncation():
    """The medium regime's log1p, 2 s (1 + s^2/3 + ... + s^8/9) with s = a/(2+a),
    on (0, 0.52]: with s rounded once, the series' truncation and roundings
    stay within 3u, leaving 7u of the 10u charged for the rounding of 2 + a,
    v_rcp_f32 (1.54u) and the product a * rcp."""
    a = _medium_points(0.52)
    a64 = a.astype(np.float64)
    s = (a64 / (2.0 + a64)).astype(np.float32)
    s2 = (s.astype(np.float64) ** 2).astype(np.float32)
    c = np.full(s2.shape, np.float32(2.0 / 9.0), dtype=np.float32)
    for k in (2.0 / 7.0, 2.0 / 5.0, 2.0 / 3.0, 2.0):
        c = (c.astype(np.float64) * s2.astype(np.float64) + np.float64(np.float32(k))).astype(np.float32)
    got = (s.astype(np.float64) * c.astype(np.float64)).astype(np.float32).astype(np.float64)
    want = np.log1p(a64)
    rel = np.abs(got - want) / want
    assert rel.max() < BOUND, rel.max() / U
