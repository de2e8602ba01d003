"""Re-use of the previous step's tensor table (the plan) on the GPU.

An optimizer that re-uses its table must step exactly as one that rebuilds
it every step, through every change the plan has to notice: new gradient
tensors, a gradient of another dtype, a parameter without a gradient,
parameter storage replaced with ``p.data = ...``.  Both optimizers run the
same kernels on the same inputs, so the results are compared bit for bit.
"""

import pytest
import torch

from luma_amd import LUMA
from luma_amd import _lib as L

pytestmark = pytest.mark.gpu

HYPER = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
SHAPES = [(1000,), (64, 48), (3, 5, 7), (1,)]


def _pair():
    gen = torch.Generator(device="cuda").manual_seed(3)
    a = [(torch.randn(s, device="cuda", generator=gen) * 0.02).requires_grad_(True)
         for s in SHAPES]
    b = [p.detach().clone().requires_grad_(True) for p in a]
    for p in a + b:
        p.grad_dtype = None      # bf16 gradients on float32 parameters
    oa, ob = LUMA(a, **HYPER), LUMA(b, **HYPER)
    ob._base_seed = oa._base_seed
    return a, b, oa, ob, gen


def _step(oa, ob):
    ob._plan = None          # b rebuilds its table every step
    oa.step()
    ob.step()
    torch.cuda.synchronize()


def _same(a, b, oa, ob):
    for pa, pb in zip(a, b):
        assert torch.equal(pa.detach(), pb.detach())
        sa, sb = oa.state[pa], ob.state[pb]
        if "Q_m" in sa or "Q_m" in sb:
            assert torch.equal(sa["Q_m"], sb["Q_m"]) and torch.equal(sa["Q_w"], sb["Q_w"])
            assert sa["step"] == sb["step"]
    sda, sdb = oa.state_dict()["state"], ob.state_dict()["state"]
    for k in sda:
        assert sda[k]["S_m"] == sdb[k]["S_m"] and sda[k]["S_v"] == sdb[k]["S_v"]


def test_plan_steps_like_a_rebuilt_table():
    a, b, oa, ob, gen = _pair()
    matches = []

    def count(engine):
        # table checks: a full comparison (_match_table) or, for a planned
        # table whose pointers moved, the pointer-set lookup (_match_pointers)
        for name in ("_match_table", "_match_pointers"):
            orig = getattr(engine, name)

            def wrapped(tt, capturing, orig=orig, **kw):
                matches.append(len(tt))
                return orig(tt, capturing, **kw)
            setattr(engine, name, wrapped)

    def set_grads(gs):
        for p, q, g in zip(a, b, gs):
            p.grad = None if g is None else g.clone()
            q.grad = None if g is None else g.clone()

    def grads(dtype=torch.float32, skip=()):
        return [None if i in skip else (torch.randn(s, device="cuda", generator=gen)
                                        * 1e-3).to(dtype) for i, s in enumerate(SHAPES)]

    set_grads(grads())
    _step(oa, ob)
    count(oa._engine)
    assert oa._plan is not None
    _same(a, b, oa, ob)

    # same gradient tensors, new values in place: no table check, no upload
    for p, q in zip(a, b):
        g = torch.randn(p.shape, device="cuda", generator=gen) * 1e-3
        p.grad.copy_(g)
        q.grad.copy_(g)
    n0 = len(matches)
    _step(oa, ob)
    assert len(matches) == n0 and oa._plan is not None
    _same(a, b, oa, ob)

    # new gradient tensors: the pointers are refreshed and the table looked
    # up by its pointers (uploaded, as these pointers are new)
    set_grads(grads())
    _step(oa, ob)
    assert len(matches) == n0 + 1 and oa._plan is not None
    _same(a, b, oa, ob)

    # gradients alternating between two sets of buffers: each set's table is
    # uploaded once and then re-used, found by the host module's refresh
    # (which compares the cached pointer sets while it writes the pointers:
    # no comparison in Python from the third step on)
    sets = [grads(), grads()]
    uploads, compared = [], []
    eng = oa._engine
    up, same = eng._upload, eng._same_pointers
    # (tensor tables only: state_dict() below uploads slot pointers too)
    eng._upload = lambda arr: (arr.dtype == L.TENSOR_DTYPE and uploads.append(len(arr))) or up(arr)
    for k in range(4):
        eng._same_pointers = lambda tt, cols, k=k: compared.append(k) or same(tt, cols)
        for p, q, g in zip(a, b, sets[k % 2]):
            p.grad, q.grad = g, g.clone()
        _step(oa, ob)
        _same(a, b, oa, ob)
    eng._upload, eng._same_pointers = up, same
    assert uploads == [len(SHAPES)] * 2 and oa._plan is not None
    assert not [k for k in compared if k >= 2]

    # bf16 gradients: the plan no longer applies, the table is rebuilt
    plan = oa._plan
    set_grads(grads(torch.bfloat16))
    _step(oa, ob)
    assert oa._plan is not None and oa._plan is not plan
    _same(a, b, oa, ob)

    # a parameter without a gradient
    plan = oa._plan
    set_grads(grads(torch.bfloat16, skip=(2,)))
    _step(oa, ob)
    assert oa._plan is not plan and len(oa._plan.layout_at) == len(SHAPES) - 1
    _same(a, b, oa, ob)

    # parameter storage replaced (same layout): pointers refreshed
    plan = oa._plan
    for p, q in zip(a, b):
        p.data = p.data.clone()
        q.data = q.data.clone()
    set_grads(grads(torch.bfloat16, skip=(2,)))
    _step(oa, ob)
    assert oa._plan is plan
    _same(a, b, oa, ob)

    # a gradient with the parameter's shape but another layout: the step
    # copies it into the parameter's layout, and a converted gradient is
    # not re-used
    gs = grads(torch.bfloat16, skip=(2,))
    gs[1] = gs[1].t().contiguous().t()
    set_grads(gs)                # clone() keeps the strides
    assert a[1].grad.stride() != a[1].stride()
    _step(oa, ob)
    assert oa._plan is None
    _same(a, b, oa, ob)


def test_plan_step_counts_match_device_counts():
    a, b, oa, ob, gen = _pair()
    for _ in range(5):
        for p in a:
            p.grad = torch.randn(p.shape, device="cuda", generator=gen) * 1e-3
        oa.step()
    sd = oa.state_dict()["state"]
    assert [sd[i]["step"] for i in range(len(a))] == [5] * len(a)
    assert [oa.state[p]["step"] for p in a] == [5] * len(a)


def test_plan_dropped_when_the_chunk_length_changes():
    """A plan's code summaries were sized for its chunk length: a new fixed
    chunk length rebuilds the table (and the summaries) instead."""
    a, b, oa, ob, gen = _pair()
    for p in a:
        p.grad = torch.randn(p.shape, device="cuda", generator=gen) * 1e-3
    oa.step()
    plan = oa._plan
    assert plan is not None and plan.chunk_setting == 0
    oa._engine.chunk_elems = 2048
    oa.step()
    assert oa._plan is not plan and oa._plan.chunk_setting == 2048
    assert oa._engine._chunk == 2048
    torch.cuda.synchronize()
