"""Small tensors stepped one wavefront each (LumaStepArgs.small_chunks), and
medium tensors stepped one wavefront each by the fast kernels
(LumaStepArgs.medium_chunks).

Tensors of at most LUMA_SMALL_TENSOR elements take the last chunk records,
one wavefront each inside the main launches (pass 1 through the exact path,
pass 2 through the fast kernel's wavefront route).  Their results must be the
oracle's, as the workgroup kernels' are, whichever route a tensor takes from
step to step; a large tensor routed there is stepped correctly too, and the
code summaries of such a step are not used by the next one.
"""

import pytest
import torch

from luma_amd import _lib as L

from config_util import SampledPair, normal_grad

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda")
# around the limit, tiny, and a few tensors that take whole workgroups
SIZES = [1, 2, 7, 64, 100, 255, 256, 257, 511, 512, 513, 1000, 2047, 2048, 4096, 5000, 70000, 300,
         8]


def _params(seed=11):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    return [(torch.randn(n, device=DEV, generator=gen) * 0.02) for n in SIZES]


def _step(pair, t, dtype=torch.float32):
    gen = torch.Generator(device=DEV).manual_seed(500 + t)
    gd = [normal_grad(p.shape, 1e-3, gen, DEV, dtype, outliers=1e-2, zeros=0.02)
          for p in pair.params]
    pair.step(gd, {i: g.cpu() for i, g in enumerate(gd)})
    return pair.check()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_small_tensors_match_oracle(dtype):
    pair = SampledPair(_params(), range(len(SIZES)))
    for t in range(1, 5):
        _step(pair, t, dtype)
        eng = pair.opt._engine
        assert eng._small_chunks == sum(1 for n in SIZES if n <= L.SMALL_TENSOR)


def test_routes_change_between_steps(monkeypatch):
    """Step 2 routes every tensor (up to 70000 elements) to the wavefront
    kernels, step 3 none, step 4 the default: every step matches the oracle,
    so the summaries of step 2's large tensors (not written) are not used by
    step 3's pass 1."""
    pair = SampledPair(_params(12), range(len(SIZES)))
    _step(pair, 1)
    small = L.SMALL_TENSOR
    monkeypatch.setattr(L, "SMALL_TENSOR", 1 << 20)
    _step(pair, 2)
    assert pair.opt._engine._small_chunks == pair.opt._engine._n_chunks
    monkeypatch.setattr(L, "SMALL_TENSOR", small)
    pair.opt._engine.small_tensors = False
    _step(pair, 3)
    assert pair.opt._engine._small_chunks == 0
    pair.opt._engine.small_tensors = True
    _step(pair, 4)
    assert pair.opt._engine._small_chunks > 0


def test_small_route_matches_workgroup_route():
    """With Philox draws: the same codes, scales and parameters through
    either route, bit for bit (both routes' pass 2 is the fast path's, on the
    same draws)."""
    from luma_amd import LUMA
    gen = torch.Generator(device=DEV).manual_seed(3)
    sizes = [1, 5, 64, 200, L.SMALL_TENSOR, L.SMALL_TENSOR - 67] * 20
    a = [(torch.randn(n, device=DEV, generator=gen) * 0.02).requires_grad_(True) for n in sizes]
    b = [p.detach().clone().requires_grad_(True) for p in a]
    oa, ob = LUMA(a, lr=1e-3), LUMA(b, lr=1e-3)
    ob._base_seed = oa._base_seed
    eb = ob._get_engine(b[0].device)
    eb.small_tensors = eb.medium_tensors = False
    for t in range(4):
        for p, q in zip(a, b):
            g = torch.randn(p.shape, device=DEV, generator=gen) * 1e-3
            p.grad, q.grad = g, g.clone()
        oa.step()
        ob.step()
    torch.cuda.synchronize()
    assert oa._engine._small_chunks == len(sizes) and ob._engine._small_chunks == 0
    sa, sb = oa.state_dict()["state"], ob.state_dict()["state"]
    for i, (p, q) in enumerate(zip(a, b)):
        assert torch.equal(sa[i]["Q_m"], sb[i]["Q_m"]), i
        assert torch.equal(sa[i]["Q_w"], sb[i]["Q_w"]), i
        assert sa[i]["S_m"] == sb[i]["S_m"] and sa[i]["S_v"] == sb[i]["S_v"], i
        assert torch.equal(p.detach(), q.detach()), i


# medium tensors: above LUMA_SMALL_TENSOR and up to LUMA_MEDIUM_TENSOR
# elements, one wavefront each through the fast kernels
MEDIUM = [513, 600, 1000, 2047, 2048, 2049, 3000, 4095, 4096, 4097, 8191, 8192, 8193, 1, 300,
          70000, 9000]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_medium_tensors_match_oracle(dtype):
    gen = torch.Generator(device=DEV).manual_seed(21)
    params = [(torch.randn(n, device=DEV, generator=gen) * 0.02) for n in MEDIUM]
    pair = SampledPair(params, range(len(MEDIUM)))
    for t in range(1, 5):
        g = torch.Generator(device=DEV).manual_seed(700 + t)
        gd = [normal_grad(p.shape, 1e-3, g, DEV, dtype, outliers=1e-2, zeros=0.02)
              for p in pair.params]
        pair.step(gd, {i: x.cpu() for i, x in enumerate(gd)})
        pair.check()
        eng = pair.opt._engine
        assert eng._medium_chunks == sum(1 for n in MEDIUM if L.SMALL_TENSOR < n <= L.MEDIUM_TENSOR)
        assert eng._small_chunks == sum(1 for n in MEDIUM if n <= L.SMALL_TENSOR)


@pytest.mark.parametrize("scaled", [False, True])
def test_medium_route_matches_workgroup_route(scaled):
    """With Philox draws (and, scaled, GradScaler's scale handed to the
    kernels): the medium tensors' wavefront route and the workgroup route
    run the same per-element arithmetic on the same draws, so codes, scales
    and parameters agree bit for bit."""
    from luma_amd import LUMA
    gen = torch.Generator(device=DEV).manual_seed(5)
    sizes = [513, 700, 1024, 2047, 2048, 2500, 4095, 4096, 6000, 8192] * 5 + [9000, 100]
    a = [(torch.randn(n, device=DEV, generator=gen) * 0.02).requires_grad_(True) for n in sizes]
    b = [p.detach().clone().requires_grad_(True) for p in a]
    for p in a + b:
        p.grad_dtype = None        # allow bf16 gradients on fp32 parameters
    oa, ob = LUMA(a, lr=1e-3, weight_decay=0.01), LUMA(b, lr=1e-3, weight_decay=0.01)
    ob._base_seed = oa._base_seed
    ob._get_engine(b[0].device).medium_tensors = False
    scale = 2.0 ** 12
    if scaled:
        for o in (oa, ob):
            o.grad_scale = torch.tensor([scale], device=DEV)
            o.found_inf = torch.tensor([0.0], device=DEV)
    for t in range(5):
        for p, q in zip(a, b):
            g = torch.randn(p.shape, device=DEV, generator=gen) * 1e-3
            if t == 2:
                g[::97] *= 100.0          # outliers: codes near the top of the grid
            g = (g * scale if scaled else g).to(torch.bfloat16)
            p.grad, q.grad = g, g.clone()
        oa.step()
        ob.step()
    torch.cuda.synchronize()
    n_med = sum(1 for n in sizes if L.SMALL_TENSOR < n <= L.MEDIUM_TENSOR)
    assert oa._engine._medium_chunks == n_med and ob._engine._medium_chunks == 0
    sa, sb = oa.state_dict()["state"], ob.state_dict()["state"]
    for i, (p, q) in enumerate(zip(a, b)):
        assert torch.equal(sa[i]["Q_m"], sb[i]["Q_m"]), i
        assert torch.equal(sa[i]["Q_w"], sb[i]["Q_w"]), i
        assert sa[i]["S_m"] == sb[i]["S_m"] and sa[i]["S_v"] == sb[i]["S_v"], i
        assert torch.equal(p.detach(), q.detach()), i


def test_medium_route_for_every_tensor(monkeypatch):
    """Step 2 routes every tensor of one chunk (here up to 16384 elements)
    through the wavefront-per-tensor route of the fast kernels, step 3 none,
    step 4 the default: every
    step matches the oracle, and the code summaries that step 2 did not
    write are not used by step 3."""
    pair = SampledPair(_params(13), range(len(SIZES)))
    _step(pair, 1)
    medium = L.MEDIUM_TENSOR
    monkeypatch.setattr(L, "MEDIUM_TENSOR", 1 << 20)
    _step(pair, 2)
    eng = pair.opt._engine
    assert eng._medium_chunks == sum(1 for n in SIZES if L.SMALL_TENSOR < n <= eng._chunk)
    monkeypatch.setattr(L, "MEDIUM_TENSOR", medium)
    eng.medium_tensors = False
    _step(pair, 3)
    assert eng._medium_chunks == 0
    eng.medium_tensors = True
    _step(pair, 4)
    assert eng._medium_chunks > 0


def test_fast_launches_equal_exact_launches_on_every_route():
    """A set with small, medium and workgroup tensors: the fast launches (the
    small tensors' pass 1 inside the pass-1 launch, each medium tensor one
    wavefront) and the exact-only launches (the small tensors' pass 1 in a
    kernel of its own) give the same codes and scales, and parameters within
    1e-6 of their scale (the fast update's bound)."""
    from luma_amd import LUMA
    gen = torch.Generator(device=DEV).manual_seed(9)
    sizes = [1, 3, 64, 200, L.SMALL_TENSOR, L.SMALL_TENSOR + 1, 1000, 4096, L.MEDIUM_TENSOR,
             L.MEDIUM_TENSOR + 1, 70000] * 3
    a = [(torch.randn(n, device=DEV, generator=gen) * 0.02).requires_grad_(True) for n in sizes]
    b = [p.detach().clone().requires_grad_(True) for p in a]
    oa, ob = LUMA(a, lr=1e-3), LUMA(b, lr=1e-3)
    ob._base_seed = oa._base_seed
    ob._flags = L.FLAG_EXACT_ONLY
    for t in range(4):
        for p, q in zip(a, b):
            g = torch.randn(p.shape, device=DEV, generator=gen) * 1e-3
            p.grad, q.grad = g, g.clone()
        oa.step()
        ob.step()
    torch.cuda.synchronize()
    ea = oa._engine
    assert ea._small_chunks == 3 * sum(1 for n in set(sizes) if n <= L.SMALL_TENSOR)
    assert ea._medium_chunks == 3 * sum(1 for n in set(sizes)
                                        if L.SMALL_TENSOR < n <= L.MEDIUM_TENSOR)
    sa, sb = oa.state_dict()["state"], ob.state_dict()["state"]
    for i, (p, q) in enumerate(zip(a, b)):
        assert torch.equal(sa[i]["Q_m"], sb[i]["Q_m"]), i
        assert torch.equal(sa[i]["Q_w"], sb[i]["Q_w"]), i
        assert sa[i]["S_m"] == sb[i]["S_m"] and sa[i]["S_v"] == sb[i]["S_v"], i
        d = float((p.detach() - q.detach()).abs().max())
        assert d <= 1e-6 * float(q.detach().abs().max()) + 1e-8, (i, d)
