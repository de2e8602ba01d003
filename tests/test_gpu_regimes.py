"""Tensors crossing the fast path's momentum regimes (small, medium,
general: luma_fast.h) from step to step, against the oracle.

The regime of a tensor's step depends on its old decode range
x_top = log1p(previous S_m) and its new S_m.  Here S_m rises through 1/8 and
1/2 and then halves per step (beta1 = 0.5, small gradients) back below 1/8,
so that some step has S_m <= 1/8 under an old range above 1/8 (the medium
log1p, charged as such).
Every step's codes and scales must be the oracle's (injected uniforms), the
parameters within 1e-6 of their scale.
"""

import math

import pytest
import torch

from config_util import SampledPair

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda")


def _regime(x_top, sm):
    if x_top <= 0.125 and sm <= 0.125:
        return "small"
    if x_top < 0.5 and sm <= 0.5:
        return "medium"
    return "general"


def test_regime_transitions_match_oracle():
    gen = torch.Generator(device=DEV).manual_seed(21)
    sizes = [20000, 4096, 300, 5000]
    params = [torch.randn(n, device=DEV, generator=gen) * 0.02 for n in sizes]
    hyper = dict(lr=1e-3, betas=(0.5, 0.999), eps=1e-8, weight_decay=0.01)
    pair = SampledPair(params, range(len(sizes)), hyper=hyper)
    scales = [5e-3, 0.05, 0.3] + [1e-4] * 7
    seen = set()
    prev_sm = None
    for sc in scales:
        g = [torch.randn(n, device=DEV, generator=gen) * sc for n in sizes]
        pair.step(g, {i: x.cpu() for i, x in enumerate(g)})
        pair.check()
        sm = float(pair.opt.state_dict()["state"][0]["S_m"])
        x_top = 0.0 if prev_sm is None else math.log1p(prev_sm)
        seen.add(_regime(x_top, sm))
        if sm <= 0.125 < x_top:
            seen.add("shrunk below 1/8")
        prev_sm = sm
    assert seen == {"small", "medium", "general", "shrunk below 1/8"}, seen
