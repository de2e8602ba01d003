"""The step's result does not depend on its chunk length.

Every element is computed on its own (its Philox uniforms are keyed by the
element's index in the tensor, not by its chunk) and the per-tensor maxima
are exact, so the same step at chunk lengths 2048, 16384, 65536 and 131072 must give
bit-identical parameters, codes and scales.
"""

import pytest
import torch

from luma_amd import LUMA

pytestmark = pytest.mark.gpu

SHAPES = [(1,), (2047,), (3 * 2048 + 5,), (65536 + 7,), (300, 700), (4096, 64), (2 * 131072 + 77,)]


def _run(chunk, grad_dtype, steps=3):
    """chunk: one length for every step, or a list of one length per step."""
    gen = torch.Generator().manual_seed(2024)
    ps = [(torch.randn(s, generator=gen) * 0.02).cuda().requires_grad_(True) for s in SHAPES]
    for p in ps:
        p.grad_dtype = None
    opt = LUMA(ps, lr=1e-3, weight_decay=0.01)
    opt._base_seed = 0x1234_5678_9ABC_DEF0 - (1 << 63)
    engine = opt._get_engine(ps[0].device)
    for t in range(steps):
        engine.chunk_elems = chunk[t] if isinstance(chunk, list) else chunk
        g = torch.Generator().manual_seed(77 + t)
        for p in ps:
            x = torch.randn(p.shape, generator=g) * 1e-3
            x.view(-1)[:: 997] *= 100.0   # a few outliers
            p.grad = x.to(grad_dtype).cuda()
        opt.step()
    torch.cuda.synchronize()
    sd = opt.state_dict()["state"]
    return [p.detach().cpu() for p in ps], sd


@pytest.mark.parametrize("grad_dtype", [torch.float32, torch.bfloat16])
def test_chunk_length_invariance(grad_dtype):
    ref_p, ref_s = _run(131072, grad_dtype)
    for chunk in (2048, 16384, 65536):
        print(f"case chunk={chunk} grad={grad_dtype}", flush=True)
        ps, st = _run(chunk, grad_dtype)
        for i, (a, b) in enumerate(zip(ps, ref_p)):
            assert torch.equal(a.view(torch.int32), b.view(torch.int32)), (chunk, i)
            for k in ("Q_m", "Q_w"):
                assert torch.equal(st[i][k].cpu(), ref_s[i][k].cpu()), (chunk, i, k)
            assert st[i]["S_m"] == ref_s[i]["S_m"] and st[i]["S_v"] == ref_s[i]["S_v"], (chunk, i)


def test_chunk_length_change_between_steps():
    """Steps that re-use the cached tensor table (same parameters and gradient
    tensors) at a different chunk length each step."""
    ref_p, ref_s = _run(131072, torch.bfloat16)
    ps, st = _run([131072, 2048, 16384], torch.bfloat16)
    for i, (a, b) in enumerate(zip(ps, ref_p)):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32)), i
        assert torch.equal(st[i]["Q_m"].cpu(), ref_s[i]["Q_m"].cpu()), i
        assert torch.equal(st[i]["Q_w"].cpu(), ref_s[i]["Q_w"].cpu()), i


def test_automatic_chunk_choice():
    """A small tensor set steps with shorter chunks."""
    p = torch.zeros(4096, 4096, device="cuda", requires_grad=True)
    opt = LUMA([p], lr=1e-3)
    p.grad = torch.full_like(p, 1e-3)
    opt.step()
    assert opt._engine._chunk == 16384
