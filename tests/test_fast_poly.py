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
