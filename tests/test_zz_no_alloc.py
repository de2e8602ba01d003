"""luma_step_noalloc: the step with its workspace in a fixed device array of
the library, for callers that cannot allocate.  Its results must equal
luma_step's bit for bit, call after call, whatever the previous call left in
the array."""

import ctypes

import pytest
import torch

from luma_amd import LUMA
from luma_amd import _lib as L

HYPER = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
BASE = 0x0123456789ABCDEF


class _NoAllocLib:
    """The library as one optimizer's engine sees it, with luma_step routed
    through luma_step_noalloc (same LumaStepArgs, partials ignored)."""

    def __init__(self, lib):
        self._lib = lib
        self.calls = 0

    def __getattr__(self, name):
        return getattr(self._lib, name)

    def luma_step(self, args, stream):
        self.calls += 1
        return self._lib.luma_step_noalloc(args, stream)


def _run(shapes, noalloc, steps, seed):
    gen = torch.Generator().manual_seed(seed)
    params = [(torch.randn(s, generator=gen) * 0.02).cuda().requires_grad_(True) for s in shapes]
    for p in params:
        p.grad_dtype = None
    opt = LUMA(params, **HYPER)
    opt._base_seed = BASE
    proxy = None
    if noalloc:
        eng = opt._get_engine(params[0].device)
        proxy = eng.lib = _NoAllocLib(eng.lib)
    for t in range(steps):
        for i, p in enumerate(params):
            g = torch.randn(p.shape, generator=gen) * 1e-3
            if i == 0:
                g[..., -1] = 0.3 * (t + 1)   # a maximum in the tensor's last chunk
            p.grad = g.to(torch.bfloat16 if i % 2 else torch.float32).cuda()
        opt.step()
    torch.cuda.synchronize()
    if proxy is not None:
        assert proxy.calls == steps
    return [p.detach().clone() for p in params], opt.state_dict()["state"]


@pytest.mark.gpu
def test_noalloc_equals_luma_step():
    # the second input is smaller: fewer tensors and chunks than the first
    # left in the array
    for shapes, seed in (([(300007,), (1000, 517), (5,), (64, 64)], 1), ([(4097,)], 2)):
        print(f"case noalloc shapes={shapes}", flush=True)
        pa, sa = _run(shapes, False, 3, seed)
        pb, sb = _run(shapes, True, 3, seed)
        for i in range(len(shapes)):
            assert torch.equal(pa[i], pb[i]), i
            assert torch.equal(sa[i]["Q_m"], sb[i]["Q_m"]), i
            assert torch.equal(sa[i]["Q_w"], sb[i]["Q_w"]), i
            assert sa[i]["S_m"] == sb[i]["S_m"] and sa[i]["S_v"] == sb[i]["S_v"], i
            assert sa[i]["step"] == sb[i]["step"] == 3


def test_noalloc_rejects_too_many_chunks():
    """Rejected on the host before any device work (so this runs without a GPU)."""
    lib = L.load()
    args = L.StepArgs(tensors=256, n_tensors=1, n_chunks=L.NOALLOC_MAX_CHUNKS + 1, chunks=256,
                      groups=256, partials=None, base_seed=0, noise_mode=L.NOISE_PHILOX, flags=0,
                      chunk_elems=0, small_chunks=0, scaling=L.Scaling(None, None))
    rc = lib.luma_step_noalloc(ctypes.byref(args), None)
    assert rc != 0
    assert b"LUMA_NOALLOC_MAX_CHUNKS" in lib.luma_last_error()


@pytest.mark.gpu
def test_noalloc_graph_replays_equal_luma_step():
    """luma_step_noalloc under HIP graph capture (the callers it is for): a
    captured LUMA.step() routed through it is replayed on fresh gradients,
    and after every replay the parameters, codes, scales and step counts
    equal eager luma_step steps on the same gradients bit for bit."""
    print("case noalloc graph capture", flush=True)
    gen = torch.Generator().manual_seed(3)
    shapes = [(300007,), (64, 33), (5,)]
    p0 = [torch.randn(s, generator=gen) * 0.02 for s in shapes]
    pa = [p.clone().cuda().requires_grad_(True) for p in p0]
    pb = [p.clone().cuda().requires_grad_(True) for p in p0]
    grads = [[(torch.randn(s, generator=gen) * 1e-3).cuda() for s in shapes] for _ in range(8)]
    opt_a, opt_b = LUMA(pa, **HYPER), LUMA(pb, **HYPER)
    opt_a._base_seed = opt_b._base_seed = BASE
    proxy = opt_a._get_engine(pa[0].device).lib = _NoAllocLib(opt_a._get_engine(pa[0].device).lib)
    for p, g in zip(pa, grads[0]):
        p.grad = torch.empty_like(g)         # static gradient buffers of the captured step

    def load_a(k):
        for p, g in zip(pa, grads[k]):
            p.grad.copy_(g)

    def eager_b(k):
        for p, g in zip(pb, grads[k]):
            p.grad = g.clone()
        opt_b.step()

    def check(what):
        torch.cuda.synchronize()
        sa, sb = opt_a.state_dict()["state"], opt_b.state_dict()["state"]
        for i in range(len(shapes)):
            assert torch.equal(pa[i].detach(), pb[i].detach()), (what, i)
            assert torch.equal(sa[i]["Q_m"], sb[i]["Q_m"]) and torch.equal(sa[i]["Q_w"], sb[i]["Q_w"]), (what, i)
            assert (sa[i]["S_m"], sa[i]["S_v"], sa[i]["step"]) == (sb[i]["S_m"], sb[i]["S_v"], sb[i]["step"]), (what, i)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for k in range(2):                   # warm-up: init step + one update, eagerly
            load_a(k)
            opt_a.step()
    torch.cuda.current_stream().wait_stream(side)
    for k in range(2):
        eager_b(k)
    check("warm-up")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        opt_a.step()
    calls = proxy.calls
    for k in range(2, 7):
        load_a(k)
        graph.replay()
        eager_b(k)
        check(f"replay {k - 1}")
    assert proxy.calls == calls == 3         # replays launch without calling the library
