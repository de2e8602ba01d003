"""A tensor of more than 2^31 elements (64-bit element offsets in every kernel).

The tensor repeats one 2^19-element pattern of parameters, gradients and
injected uniforms 4097 times (2,148,007,936 elements).  Its maxima are the
pattern's, so its grids are those of a tensor holding the pattern once, and
every element is computed on its own: after each step every period must
equal the single-pattern tensor bit for bit, the last one (past 2^31)
included.  About 40 GB of device memory.
"""

import pytest
import torch

from luma_amd import LUMA

pytestmark = pytest.mark.gpu

PERIOD = 1 << 19
REPS = 4097


def test_tensor_beyond_2_31_elements():
    n = PERIOD * REPS
    assert n > 2**31
    print(f"case large n={n}", flush=True)
    gen = torch.Generator().manual_seed(31)
    p0 = (torch.randn(PERIOD, generator=gen) * 0.02).cuda()
    small = p0.clone().requires_grad_(True)
    big = p0.repeat(REPS).requires_grad_(True)
    small.grad_dtype = None
    big.grad_dtype = None
    o_small = LUMA([small], lr=1e-3)
    o_big = LUMA([big], lr=1e-3)
    o_big._base_seed = o_small._base_seed
    for t in range(3):
        g = (torch.randn(PERIOD, generator=gen) * 1e-3).to(torch.bfloat16).cuda()
        um = torch.rand(PERIOD, generator=gen).cuda()
        uw = torch.rand(PERIOD, generator=gen).cuda()
        small.grad = g
        big.grad = g.repeat(REPS)
        o_small.inject_noise({small: (um, uw)})
        o_big.inject_noise({big: (um.repeat(REPS), uw.repeat(REPS))})
        o_small.step()
        o_big.step()
        torch.cuda.synchronize()
        ref = small.detach().view(torch.int32)
        assert torch.equal(big.detach().view(torch.int32).view(REPS, PERIOD), ref.expand(REPS, PERIOD)), t
        ss, sb = o_small.state[small], o_big.state[big]
        for k in ("Q_m", "Q_w"):
            assert torch.equal(sb[k].view(REPS, PERIOD), ss[k].expand(REPS, PERIOD)), (t, k)
        del g, um, uw
    a, b = o_small.state_dict()["state"][0], o_big.state_dict()["state"][0]
    assert a["S_m"] == b["S_m"] and a["S_v"] == b["S_v"]
    del o_big, big
    torch.cuda.empty_cache()
