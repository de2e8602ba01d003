"""Mixed precision: torch.amp.GradScaler with the in-kernel unscale.

LUMA declares ``_step_supports_amp_scaling``: GradScaler then hands it the
scale and its found_inf flag (device tensors) instead of unscaling the
gradients and checking them on the host.  The kernels unscale each gradient
exactly as ``GradScaler.unscale_`` would store it and skip the step on the
device when found_inf is set.  The reference runs LUMA behind the classic
GradScaler path (unscale_, host check, step); a twin optimizer that declares
no support takes that path here, and the two must agree bit for bit,
including a step skipped for an overflow.
"""

import pytest
import torch
import torch.nn as nn

from luma_amd import LUMA
from luma_amd import functional as F

pytestmark = pytest.mark.gpu
DEV = "cuda"


class _Classic(LUMA):
    """LUMA behind GradScaler's classic path (unscale_, host check, step)."""
    _step_supports_amp_scaling = False


def _model():
    # weights of 8192 (a workgroup per chunk), 3072 (one wavefront each: the
    # medium route) and 24 elements (the small-tensor kernels), and biases
    torch.manual_seed(0)
    return nn.Sequential(nn.Linear(64, 128), nn.GELU(), nn.Linear(128, 24), nn.GELU(),
                         nn.Linear(24, 1)).to(DEV)


def _state(opt, model):
    sd = opt.state_dict()["state"]
    return ([p.detach().clone() for p in model.parameters()],
            [(s["Q_m"].clone(), s["Q_w"].clone(), s["S_m"], s["S_v"], s["step"])
             for _, s in sorted(sd.items())])


@pytest.mark.parametrize("autocast_dtype", [torch.float16, torch.bfloat16])
def test_gradscaler_in_kernel_unscale_equals_classic_path(autocast_dtype):
    ma, mb = _model(), _model()
    oa = LUMA(ma.parameters(), lr=1e-3, weight_decay=0.05)
    ob = _Classic(mb.parameters(), lr=1e-3, weight_decay=0.05)
    ob._base_seed = oa._base_seed
    sa = torch.amp.GradScaler("cuda", init_scale=2.0 ** 14, growth_interval=3)
    sb = torch.amp.GradScaler("cuda", init_scale=2.0 ** 14, growth_interval=3)
    gen = torch.Generator(device=DEV).manual_seed(1)
    for step in range(12):
        x = torch.randn(32, 64, device=DEV, generator=gen)
        y = torch.randn(32, 1, device=DEV, generator=gen)
        if step == 5:
            x[0, 0] = float("inf")   # this step's gradients overflow: both must skip it
        for model, opt, scaler in ((ma, oa, sa), (mb, ob, sb)):
            opt.zero_grad()
            with torch.amp.autocast("cuda", dtype=autocast_dtype):
                loss = (model(x).float() - y).square().mean()
            scaler.scale(loss).backward()
            scaler.step(opt)
            scaler.update()
        torch.cuda.synchronize()
        assert sa.get_scale() == sb.get_scale(), step
        pa, qa = _state(oa, ma)
        pb, qb = _state(ob, mb)
        for i, (x1, x2) in enumerate(zip(pa, pb)):
            assert torch.equal(x1, x2), f"step {step}: param {i}"
        for i, (s1, s2) in enumerate(zip(qa, qb)):
            assert torch.equal(s1[0], s2[0]) and torch.equal(s1[1], s2[1]), f"step {step}: codes {i}"
            assert s1[2:] == s2[2:], f"step {step}: scales/step {i}: {s1[2:]} vs {s2[2:]}"
    assert qa[0][4] < 12   # the overflow step (and any other) did not count


@pytest.mark.parametrize("gdt", [torch.float32, torch.bfloat16, torch.float16])
def test_grad_scale_equals_pre_unscaled_gradient(gdt):
    n = 50001
    gen = torch.Generator().manual_seed(2)
    x0 = (torch.randn(n, generator=gen) * 0.02).to(DEV)
    scale = torch.tensor([2.0 ** 13 * 1.37], device=DEV)   # not a power of two: rounding matters
    inv = (1.0 / scale.double()).float()
    a = [x0.clone(), torch.empty(n, dtype=torch.int16, device=DEV),
         torch.empty(n, dtype=torch.int16, device=DEV), F.new_slot(DEV)]
    b = [x0.clone(), a[1].clone(), a[2].clone(), F.new_slot(DEV)]
    zero = torch.zeros((), device=DEV)
    for t in range(3):
        g = torch.randn(n, generator=gen) * 1e-3
        scaled = (g.to(DEV) * scale).to(gdt)
        # what GradScaler.unscale_ stores: dtype(f32(g) * inv), torch's own cast
        unscaled = (scaled.float() * inv).to(gdt)
        F.luma_step(a[0], scaled, *a[1:], 0.9, 0.999, 1e-8, 1e-3, 0.01, 3, 77, grad_scale=scale,
                    found_inf=zero)
        F.luma_step(b[0], unscaled, *b[1:], 0.9, 0.999, 1e-8, 1e-3, 0.01, 3, 77)
        torch.cuda.synchronize()
        for u, v in zip(a[:3], b[:3]):
            assert torch.equal(u, v), f"t={t}"
        assert F.slot_state(a[3]) == F.slot_state(b[3])


def test_found_inf_skips_everything():
    n = 40000
    gen = torch.Generator().manual_seed(3)
    p = (torch.randn(n, generator=gen) * 0.02).to(DEV)
    qm = torch.empty(n, dtype=torch.int16, device=DEV)
    qw = torch.empty(n, dtype=torch.int16, device=DEV)
    slot = F.new_slot(DEV)
    g = (torch.randn(n, generator=gen) * 1e-3).to(DEV)
    F.luma_step(p, g, qm, qw, slot, 0.9, 0.999, 1e-8, 1e-3, 0.01, 0, 5)
    torch.cuda.synchronize()
    before = (p.clone(), qm.clone(), qw.clone(), F.slot_state(slot))
    one = torch.ones((), device=DEV)
    for exact in (False, True):
        F.luma_step(p, g * float("nan"), qm, qw, slot, 0.9, 0.999, 1e-8, 1e-3, 0.01, 0, 5,
                    exact=exact, found_inf=one)
    torch.cuda.synchronize()
    assert torch.equal(p, before[0]) and torch.equal(qm, before[1]) and torch.equal(qw, before[2])
    assert F.slot_state(slot) == before[3]
    F.luma_step(p, g, qm, qw, slot, 0.9, 0.999, 1e-8, 1e-3, 0.01, 0, 5,
                found_inf=torch.zeros((), device=DEV))
    torch.cuda.synchronize()
    assert F.slot_state(slot)[0] == 2 and not torch.equal(p, before[0])


def test_optimizer_scaling_attributes_exact_path():
    """The exact kernels (LUMA_FLAG_EXACT_ONLY) unscale the same way: codes and
    scales equal the fast path's, parameters within 1e-6 of their scale (the
    two paths' update roundings differ, as without scaling)."""
    from luma_amd import _lib as L
    n = 30011
    gen = torch.Generator().manual_seed(4)
    x0 = torch.randn(n, generator=gen) * 0.02
    xs = [x0.clone().to(DEV).requires_grad_(True) for _ in range(2)]
    opts = [LUMA([x], lr=1e-3) for x in xs]
    opts[1]._base_seed = opts[0]._base_seed
    opts[0]._flags = L.FLAG_EXACT_ONLY
    scale = torch.tensor([4096.0], device=DEV)
    for t in range(3):
        g = (torch.randn(n, generator=gen) * 1e-3).to(DEV)
        for x, o in zip(xs, opts):
            x.grad = g * scale
            o.grad_scale = scale
            o.found_inf = torch.zeros((), device=DEV)
            o.step()
            del o.grad_scale, o.found_inf
        torch.cuda.synchronize()
        err = float((xs[0].detach() - xs[1].detach()).abs().max() / xs[1].detach().abs().max())
        assert err <= 1e-6, (t, err)
        sa, sb = opts[0].state_dict()["state"][0], opts[1].state_dict()["state"][0]
        assert torch.equal(sa["Q_m"], sb["Q_m"]) and torch.equal(sa["Q_w"], sb["Q_w"])
        assert (sa["S_m"], sa["S_v"], sa["step"]) == (sb["S_m"], sb["S_v"], sb["step"])
