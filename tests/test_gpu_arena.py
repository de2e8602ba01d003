"""Flat state arena: every parameter's Q_m / Q_w created by a step are views
of one int16 allocation (256-byte aligned, the parameter's shape and
strides), so a checkpoint of the optimizer state writes one storage."""

import io

import pytest
import torch
import torch.nn as nn

from luma_amd import LUMA

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _model():
    torch.manual_seed(0)
    m = nn.Sequential(nn.Conv2d(3, 8, 3), nn.ReLU(), nn.Conv2d(8, 4, 3), nn.Flatten(),
                      nn.Linear(4 * 4 * 4, 10)).to(DEV)
    return m.to(memory_format=torch.channels_last)


def test_codes_share_one_aligned_storage():
    m = _model()
    opt = LUMA(m.parameters(), lr=1e-3)
    m(torch.randn(2, 3, 8, 8, device=DEV).to(memory_format=torch.channels_last)).sum().backward()
    opt.step()
    torch.cuda.synchronize()
    qs = [(p, opt.state[p]["Q_m"], opt.state[p]["Q_w"]) for p in m.parameters()]
    base = qs[0][1].untyped_storage().data_ptr()
    for p, qm, qw in qs:
        for q in (qm, qw):
            assert q.untyped_storage().data_ptr() == base
            assert q.shape == p.shape and q.stride() == p.stride()
            assert q.data_ptr() % 256 == 0
            assert q.element_size() * q.numel() == 2 * p.numel()   # 4 B/param in all


def test_checkpoint_writes_one_storage_and_round_trips():
    m = _model()
    opt = LUMA(m.parameters(), lr=1e-3)
    x = torch.randn(2, 3, 8, 8, device=DEV).to(memory_format=torch.channels_last)
    for _ in range(3):
        opt.zero_grad()
        m(x).sum().backward()
        opt.step()
    sd = opt.state_dict()
    buf = io.BytesIO()
    torch.save(sd, buf)
    arena_bytes = sd["state"][0]["Q_m"].untyped_storage().nbytes()
    n_params = sum(p.numel() for p in m.parameters())
    assert arena_bytes < 4 * n_params + 256 * 2 * len(sd["state"])
    assert len(buf.getvalue()) < arena_bytes + 64 * 1024   # the storage once, plus metadata
    buf.seek(0)
    sd2 = torch.load(buf, weights_only=True)
    m2 = _model()
    m2.load_state_dict(m.state_dict())
    opt2 = LUMA(m2.parameters(), lr=1e-3)
    opt2.load_state_dict(sd2)
    # both optimizers step on the same gradients (the convolutions' weight
    # gradients need not repeat bit for bit between two backward passes)
    opt.zero_grad()
    m(x).sum().backward()
    for p1, p2 in zip(m.parameters(), m2.parameters()):
        assert torch.equal(p1, p2)
        p2.grad = p1.grad.clone()
    opt.step()
    opt2.step()
    for p1, p2 in zip(m.parameters(), m2.parameters()):
        assert torch.equal(p1, p2)
