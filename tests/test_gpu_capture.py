"""Graph capture and torch.compile of the HIP step (the reference's
tests/test_compile.py, and its device step counter, optimizer.py:382-387).

* the step scalars derived on the device equal the reference's Python
  double arithmetic (luma_hyper_rows);
* LUMA.step() captured into a CUDA (HIP) graph after eager warm-up steps and
  replayed: after every replay the parameters, codes, scales and step counts
  equal those of an identical optimizer stepped eagerly (bitwise), and, with
  the oracle's uniforms refilled into the captured buffers, the oracle's;
* a capture whose tables would change is refused before anything launches;
* the per-tensor op (luma_amd.functional.luma_step) equals the multi-tensor
  step bit for bit, including its init step;
* torch.compile(fullgraph=True) of the per-tensor op, with zero graph breaks;
* a compiled training step (forward + backward + LUMA.step), also under
  autocast.
"""

import ctypes

import numpy as np
import pytest
import torch
import torch.nn as nn

from luma_amd import LUMA
from luma_amd import _lib as L
from luma_amd import functional as F

pytestmark = pytest.mark.gpu
DEV = "cuda"
SHAPES = [(4097,), (300, 257), (1,), (65543,), (2, 3, 5)]


@pytest.fixture(autouse=True)
def _dynamo_reset():
    torch._dynamo.reset()
    yield
    torch._dynamo.reset()


def _params(seed):
    gen = torch.Generator().manual_seed(seed)
    out = [(torch.randn(s, generator=gen) * 0.02).to(DEV).requires_grad_(True) for s in SHAPES]
    for p in out:
        p.grad_dtype = None   # gradients may be bf16 / fp16
    return out


def _grad_sets(k, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    out = []
    for _ in range(k):
        gs = []
        for s in SHAPES:
            g = torch.randn(s, generator=gen) * 1e-3
            g.view(-1)[::97] *= 100.0   # outliers, so the fast path's fallbacks run too
            gs.append(g.to(dtype).to(DEV))
        out.append(gs)
    return out


def _state(opt, params):
    sd = opt.state_dict()["state"]
    return [(p.detach().clone(), sd[i]["Q_m"].clone(), sd[i]["Q_w"].clone(), sd[i]["S_m"],
             sd[i]["S_v"], sd[i]["step"]) for i, p in enumerate(params)]


def _assert_same(a, b, where):
    for i, (x, y) in enumerate(zip(a, b)):
        assert torch.equal(x[0], y[0]), f"{where}: param {i}"
        assert torch.equal(x[1], y[1]), f"{where}: Q_m {i}"
        assert torch.equal(x[2], y[2]), f"{where}: Q_w {i}"
        assert x[3:] == y[3:], f"{where}: scales/step {i}: {x[3:]} vs {y[3:]}"


def _python_rows(lr, b1, b2, eps, wd, t0, n):
    rows = []
    for t in range(t0, t0 + n):
        bc1 = 1.0 - b1 ** t
        rows.append((b1, 1.0 - b1, b2, 1.0 - b2, 1.0 - wd * lr, -(lr / bc1), 1.0 - b2 ** t, eps))
    return np.array(rows, dtype=np.float64).astype(np.float32)


@pytest.mark.parametrize("hp", [(1e-3, 0.9, 0.999, 1e-8, 0.01), (3e-4, 0.95, 0.9999, 1e-6, 0.1),
                                (1e-2, 0.8, 0.99999, 1e-10, 0.05)])
def test_device_step_scalars_equal_python(hp):
    lib = L.load()
    n, t0 = 50000, 1
    g = np.array([hp + (0.0,)], dtype=L.GROUP_DTYPE)
    out = torch.empty(8 * n, dtype=torch.float32, device=DEV)
    L.check(lib.luma_hyper_rows(g.ctypes.data, t0, n, out.data_ptr(),
                                torch.cuda.current_stream().cuda_stream), "luma_hyper_rows")
    got = out.view(n, 8).cpu().numpy().view(np.uint32)
    want = _python_rows(*hp, t0, n).view(np.uint32)
    bad = np.nonzero((got != want).any(axis=1))[0]
    assert bad.size == 0, f"steps {bad[:5] + t0}"


@pytest.mark.parametrize("gdt", [torch.bfloat16, torch.float32])
def test_graph_replay_matches_eager(gdt):
    pa, pb = _params(1), _params(1)
    grads = _grad_sets(9, gdt, 2)
    hyper = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    opt_a, opt_b = LUMA(pa, **hyper), LUMA(pb, **hyper)
    opt_b._base_seed = opt_a._base_seed
    # static gradient buffers for the captured optimizer
    for p, g in zip(pa, grads[0]):
        p.grad = torch.empty_like(g)

    def load_a(k):
        for p, g in zip(pa, grads[k]):
            p.grad.copy_(g)

    def eager_b(k):
        for p, g in zip(pb, grads[k]):
            p.grad = g.clone()
        opt_b.step()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for k in range(2):          # warm-up: init step + one update, eagerly
            load_a(k)
            opt_a.step()
    torch.cuda.current_stream().wait_stream(side)
    for k in range(2):
        eager_b(k)
    torch.cuda.synchronize()
    _assert_same(_state(opt_a, pa), _state(opt_b, pb), "warm-up")

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        opt_a.step()
    torch.cuda.synchronize()
    for k in range(2, 8):
        load_a(k)
        graph.replay()
        eager_b(k)
        torch.cuda.synchronize()
        sa, sb = _state(opt_a, pa), _state(opt_b, pb)
        assert sa[0][5] == k + 1
        _assert_same(sa, sb, f"replay {k - 1}")
    # an eager step after the replays continues from the device step counts
    load_a(8)
    opt_a.step()
    eager_b(8)
    torch.cuda.synchronize()
    _assert_same(_state(opt_a, pa), _state(opt_b, pb), "eager after replay")
    assert opt_a.state[pa[0]]["step"] == 9


def test_graph_replay_matches_oracle():
    """A captured LUMA.step() against the correctly rounded CPU oracle: the
    injected-uniform buffers are persistent (the graph reads them), refilled
    with the oracle's draws of each step before the replay, and every replay's
    codes and scales must equal the oracle's, parameters within 1e-6 of their
    scale (the reference's compiled-step test, tests/test_compile.py:181-242,
    with its device step counter, optimizer.py:382-387)."""
    from oracle import luma_oracle as O

    hyper = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    pa = _params(5)
    cpu = [p.detach().cpu().clone() for p in pa]
    for c in cpu:
        c.grad_dtype = None
    grads = _grad_sets(8, torch.bfloat16, 6)
    base = 0x3C6EF372FE94F82B
    oracle = O.OracleLUMA([dict(params=cpu, **hyper)], base, "cr")
    opt = LUMA(pa, **hyper)
    opt._base_seed = base
    for p, g in zip(pa, grads[0]):
        p.grad = torch.empty_like(g)
    u_bufs = {p: (torch.empty_like(p), torch.empty_like(p)) for p in pa}

    def load(k):
        """Step k's gradients into both, the oracle's step, and its draws into
        the uniform buffers the captured step reads."""
        for p, c, g in zip(pa, cpu, grads[k]):
            p.grad.copy_(g)
            c.grad = g.cpu()
        oracle.step()
        for i, p in enumerate(pa):
            u_m, u_w = oracle.last_draws[i]
            u_bufs[p][0].copy_(u_m)
            u_bufs[p][1].copy_(u_w)

    def check(where):
        sd = opt.state_dict()["state"]
        for i, (p, c) in enumerate(zip(pa, cpu)):
            o = oracle.state[id(c)]
            assert torch.equal(sd[i]["Q_m"].cpu(), o["Q_m"]), f"{where}: Q_m {i}"
            assert torch.equal(sd[i]["Q_w"].cpu(), o["Q_w"]), f"{where}: Q_w {i}"
            assert (sd[i]["S_m"], sd[i]["S_v"]) == (o["S_m"], o["S_v"]), f"{where}: S {i}"
            assert sd[i]["step"] == o["step"], f"{where}: step {i}"
            err = float((p.detach().cpu() - c).abs().max())
            assert err <= 1e-6 * float(c.abs().max()) + 1e-8, f"{where}: param {i} {err}"

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for k in range(2):          # warm-up: init step + one update, eagerly
            load(k)
            opt.inject_noise(u_bufs)
            opt.step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    check("warm-up")
    graph = torch.cuda.CUDAGraph()
    opt.inject_noise(u_bufs)
    with torch.cuda.graph(graph):
        opt.step()
    for k in range(2, 8):
        load(k)
        graph.replay()
        torch.cuda.synchronize()
        check(f"replay {k - 1}")


def test_capture_refuses_changed_tables(monkeypatch):
    params = _params(3)
    opt = LUMA(params, lr=1e-3)
    for p, g in zip(params, _grad_sets(1, torch.float32, 4)[0]):
        p.grad = g
    opt.step()
    torch.cuda.synchronize()
    before = _state(opt, params)
    # pretend the stream is capturing: nothing may be uploaded or allocated
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    for p in params:
        p.grad = p.grad.clone()          # new gradient tensors: the table would change
    with pytest.raises(RuntimeError, match="graph capture"):
        opt.step()
    extra = torch.zeros(7, device=DEV, requires_grad=True)
    extra.grad = torch.ones(7, device=DEV)
    opt.add_param_group({"params": [extra]})
    with pytest.raises(RuntimeError, match="graph capture"):
        opt.step()
    monkeypatch.undo()
    torch.cuda.synchronize()
    after = _state(opt, params)
    assert [x[5] for x in after] == [x[5] for x in before]   # no step ran


@pytest.mark.parametrize("gdt", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("injected", [False, True])
def test_functional_op_equals_optimizer(gdt, injected):
    n = 70001
    gen = torch.Generator().manual_seed(5)
    x0 = torch.randn(n, generator=gen) * 0.02
    xa = x0.clone().to(DEV).requires_grad_(True)
    xa.grad_dtype = None
    xb = x0.clone().to(DEV)
    hyper = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    opt = LUMA([xa], **hyper)
    qm = torch.empty(n, dtype=torch.int16, device=DEV)
    qw = torch.empty(n, dtype=torch.int16, device=DEV)
    slot = F.new_slot(DEV)
    for t in range(1, 5):
        g = (torch.randn(n, generator=gen) * 1e-3).to(gdt).to(DEV)
        u = None
        if injected:
            u = (torch.rand(n, generator=gen).to(DEV), torch.rand(n, generator=gen).to(DEV))
            opt.inject_noise({xa: u})
        xa.grad = g
        opt.step()
        F.luma_step(xb, g, qm, qw, slot, 0.9, 0.999, 1e-8, 1e-3, 0.01, 0, opt._base_seed,
                    *(u if u else (None, None)))
        torch.cuda.synchronize()
        sd = opt.state_dict()["state"][0]
        assert torch.equal(xa.detach(), xb), f"param, t={t}"
        assert torch.equal(sd["Q_m"], qm) and torch.equal(sd["Q_w"], qw), f"codes, t={t}"
        assert F.slot_state(slot) == (t, sd["S_m"], sd["S_v"])


def _op_args(n, seed):
    gen = torch.Generator().manual_seed(seed)
    param = (torch.randn(n, generator=gen) * 0.02).to(DEV)
    grad = (torch.randn(n, generator=gen) * 1e-3).to(DEV)
    qm = torch.zeros(n, dtype=torch.int16, device=DEV)
    qw = torch.zeros(n, dtype=torch.int16, device=DEV)
    return param, grad, qm, qw, F.new_slot(DEV)


@pytest.mark.parametrize("n", [1, 127, 1024, 8192, 40000])
def test_functional_compiles_fullgraph(n):
    a = _op_args(n, 6)
    b = tuple(t.clone() for t in a)
    compiled = torch.compile(F.luma_step, fullgraph=True)
    for _ in range(5):
        compiled(*a, 0.9, 0.999, 1e-8, 1e-3, 0.01, 0, 42)
        F.luma_step(*b, 0.9, 0.999, 1e-8, 1e-3, 0.01, 0, 42)
    torch.cuda.synchronize()
    assert F.slot_state(a[4])[0] == 5
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    assert a[0].isfinite().all()


def test_functional_zero_graph_breaks():
    a = _op_args(4096, 7)
    explanation = torch._dynamo.explain(F.luma_step)(*a, 0.9, 0.999, 1e-8, 1e-3, 0.01, 0, 42)
    torch.cuda.synchronize()
    assert explanation.graph_break_count == 0, explanation.break_reasons
    assert F.slot_state(a[4])[0] == 1


def _mlp():
    torch.manual_seed(0)
    return nn.Sequential(nn.Linear(32, 64), nn.ReLU(), nn.Linear(64, 1)).to(DEV)


@pytest.mark.parametrize("autocast", [False, True])
def test_compiled_train_step(autocast):
    model = _mlp()
    opt = LUMA(model.parameters(), lr=1e-3)
    x = torch.randn(8, 32, device=DEV)
    y = torch.randn(8, 1, device=DEV)

    @torch.compile()
    def train_step(x, y):
        opt.zero_grad()
        with torch.amp.autocast("cuda", dtype=torch.float16, enabled=autocast):
            pred = model(x)
        loss = (pred.float() - y).square().mean()
        loss.backward()
        opt.step()
        return loss

    losses = [train_step(x, y).item() for _ in range(10)]
    assert all(np.isfinite(losses))
    assert losses[-1] < losses[0]
    for p in model.parameters():
        assert p.isfinite().all()
        assert opt.state[p]["step"] == 10
    assert all(s["step"] == 10 for s in opt.state_dict()["state"].values())


def test_library_entry_points_bound():
    lib = L.load()
    for name in ("luma_step_tensor", "luma_hyper_rows"):
        assert ctypes.cast(getattr(lib, name), ctypes.c_void_p).value
