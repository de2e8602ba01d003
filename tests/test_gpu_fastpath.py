"""The fast path (certified decisions + exact fallback) vs the exact path.

Both paths run the same kernels' inputs; the fast path must reproduce the
exact path's int16 codes and scales bit for bit on every step, for gradient
distributions chosen to stress the error bounds: tiny and huge scales (both
decode regimes), heavy tails, exact zeros, constant and sign-flipping
gradients, every gradient dtype, ragged sizes, both noise sources.
Parameters agree within 1e-6 of their scale (the fast AdamW update is not
bit-matched by design).
"""

import math

import pytest
import torch

from luma_amd import LUMA
from luma_amd import _lib as L

pytestmark = pytest.mark.gpu


def _grads(kind, shape, t, dtype, gen):
    n = shape[0]
    if kind == "normal":
        g = torch.randn(n, generator=gen) * 1e-3
    elif kind == "tiny":
        g = torch.randn(n, generator=gen) * 1e-7
    elif kind == "large":
        g = torch.randn(n, generator=gen) * 3.0
    elif kind == "huge":
        g = torch.randn(n, generator=gen) * 300.0
    elif kind == "heavy":
        g = torch.randn(n, generator=gen) * 1e-3
        g[torch.rand(n, generator=gen) < 0.001] *= 1e4
    elif kind == "zeros":
        g = torch.randn(n, generator=gen) * 1e-2
        g[torch.rand(n, generator=gen) < 0.5] = 0.0
    elif kind == "constant":
        g = torch.full((n,), 2.5e-3)
    elif kind == "flip":
        base = torch.randn(n, generator=torch.Generator().manual_seed(5)) * 1e-2
        g = base * (1.0 if t % 2 else -1.0)
    elif kind == "loguniform":
        g = torch.randn(n, generator=gen) * torch.exp(torch.rand(n, generator=gen) * 30 - 25)
    else:
        raise ValueError(kind)
    return g.to(dtype)


def _run(kind, n, dtype, steps, inject, exact, seed=1234):
    gen = torch.Generator().manual_seed(seed)
    x = (torch.randn(n, generator=gen) * 0.02).cuda().requires_grad_(True)
    x.grad_dtype = None
    opt = LUMA([x], lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    opt._base_seed = 0x1D872B41
    opt._flags = L.FLAG_EXACT_ONLY if exact else 0
    ggen = torch.Generator().manual_seed(seed + 1)
    ugen = torch.Generator().manual_seed(seed + 2)
    out = []
    for t in range(1, steps + 1):
        x.grad = _grads(kind, (n,), t, dtype, ggen).cuda()
        if inject:
            opt.inject_noise({x: (torch.rand(n, generator=ugen).cuda(),
                                  torch.rand(n, generator=ugen).cuda())})
        opt.step()
        sd = opt.state_dict()["state"][0]
        out.append((sd["Q_m"].cpu(), sd["Q_w"].cpu(), sd["S_m"], sd["S_v"], x.detach().cpu().clone()))
    return out


KINDS = ["normal", "tiny", "large", "huge", "heavy", "zeros", "constant", "flip", "loguniform"]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("inject", [False, True])
def test_fast_equals_exact(kind, inject):
    n = 1_000_003
    dtype = {"normal": torch.bfloat16, "tiny": torch.float16, "heavy": torch.bfloat16}.get(
        kind, torch.float32)
    print(f"case kind={kind} inject={inject} n={n} dtype={dtype}", flush=True)
    fast = _run(kind, n, dtype, 6, inject, exact=False)
    slow = _run(kind, n, dtype, 6, inject, exact=True)
    for t, (a, b) in enumerate(zip(fast, slow), start=1):
        assert torch.equal(a[0], b[0]), f"Q_m differs at step {t}: {(a[0] != b[0]).sum()}"
        assert torch.equal(a[1], b[1]), f"Q_w differs at step {t}: {(a[1] != b[1]).sum()}"
        assert a[2] == b[2] and a[3] == b[3], f"scales differ at step {t}"
        scale = float(b[4].abs().max())
        assert float((a[4] - b[4]).abs().max()) <= 1e-6 * scale, f"params differ at step {t}"


@pytest.mark.parametrize("n", [1, 7, 8, 9, 4095, 32769, 65543])
def test_fast_equals_exact_ragged(n):
    fast = _run("heavy", n, torch.float32, 3, False, exact=False, seed=n)
    slow = _run("heavy", n, torch.float32, 3, False, exact=True, seed=n)
    for a, b in zip(fast, slow):
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
        assert a[2] == b[2] and a[3] == b[3]


def _hetero_set(seed=5, n_tensors=12, numel=70001):
    """Per-tensor grad std log-uniform in [1e-7, 1e-1]; fp16 grads produced the
    GradScaler way: scale by 2^16, cast to fp16, unscale in fp32, cast back."""
    g = torch.Generator().manual_seed(seed)
    stds = torch.exp(torch.empty(n_tensors).uniform_(math.log(1e-7), math.log(1e-1), generator=g))
    params = [(torch.randn(numel + 13 * i, generator=g) * 0.02) for i in range(n_tensors)]

    def grads(t):
        gt = torch.Generator().manual_seed(1000 * seed + t)
        out = []
        for p, s in zip(params, stds.tolist()):
            scaled = (torch.randn(p.shape, generator=gt) * s * 2.0 ** 16).half()
            out.append((scaled.float() * 2.0 ** -16).half())
        return out
    return params, grads


def _hetero_run(exact):
    params0, grads = _hetero_set()
    xs = [p.clone().cuda().requires_grad_(True) for p in params0]
    for x in xs:
        x.grad_dtype = None
    opt = LUMA(xs, lr=1e-3, weight_decay=0.01)
    opt._base_seed = 0x5EED
    opt._flags = L.FLAG_EXACT_ONLY if exact else 0
    for t in range(1, 4):
        for x, gr in zip(xs, grads(t)):
            x.grad = gr.cuda()
        opt.step()
    # restart from the checkpoint, as a resumed run does
    sd = opt.state_dict()
    opt = LUMA(xs, lr=1e-3, weight_decay=0.01)
    opt.load_state_dict(sd)
    opt._flags = L.FLAG_EXACT_ONLY if exact else 0
    out = []
    for t in range(4, 8):
        for x, gr in zip(xs, grads(t)):
            x.grad = gr.cuda()
        opt.step()
        st = opt.state_dict()["state"]
        out.append([(st[i]["Q_m"].cpu(), st[i]["Q_w"].cpu(), st[i]["S_m"], st[i]["S_v"],
                     xs[i].detach().cpu().clone()) for i in range(len(xs))])
    return out


def test_fast_equals_exact_heterogeneous_fp16_restored():
    """Heterogeneous-scale workload: fast path == exact path after a restore."""
    fast, slow = _hetero_run(False), _hetero_run(True)
    for t, (fs, ss) in enumerate(zip(fast, slow), start=4):
        for i, (a, b) in enumerate(zip(fs, ss)):
            assert torch.equal(a[0], b[0]), f"Q_m differs: step {t} tensor {i}"
            assert torch.equal(a[1], b[1]), f"Q_w differs: step {t} tensor {i}"
            assert a[2] == b[2] and a[3] == b[3], f"scales differ: step {t} tensor {i}"
            scale = float(b[4].abs().max())
            assert float((a[4] - b[4]).abs().max()) <= 1e-6 * scale
