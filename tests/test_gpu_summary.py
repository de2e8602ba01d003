"""Code summaries: pass 2 records, per thread of each chunk's workgroup, a
bound on the codes that thread stored (max |Q_m| widened upward, min Q_w
widened downward), and the next pass 1 reads a wave's codes only when some
thread's bound lets its groups hold the tensor's maximum.

* the bound holds for every block of every tensor after every step (the
  final codes, exact-path corrections included);
* steps with summaries equal steps without them bit for bit (codes, scales,
  parameters), over gradient distributions whose maxima move between blocks,
  ragged sizes and all three gradient dtypes;
* a checkpoint load and an AdamW import invalidate them (the slot's record),
  and the steps after that still equal steps without summaries;
* tensors small enough to be stepped a wavefront each have none, and their
  slots say so.
"""

import pytest
import torch

from luma_amd import LUMA
from luma_amd import _lib as L

pytestmark = pytest.mark.gpu
DEV = "cuda"
HYPER = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
SHAPES = [(300007,), (1000, 517), (2048,), (5,), (131072 * 3 + 4096,)]


def _grad(t, i, shape, dtype, kind):
    g = torch.Generator().manual_seed(97 * t + i)
    x = torch.randn(shape, generator=g) * 1e-3
    flat = x.view(-1)
    if kind == "moving_max":
        # one large gradient at a different block each step, decaying
        flat[(7919 * t * (i + 1)) % flat.numel()] = 0.5 / t
    elif kind == "outliers":
        flat[torch.rand(flat.shape, generator=g) < 1e-3] *= 100.0
    elif kind == "shrinking":
        x *= 10.0 ** (-t)      # every new maximum is far below the old scale
    return x.to(dtype)


def _pair(dtype, kind, steps, between=None):
    gen = torch.Generator().manual_seed(1)
    p0 = [torch.randn(s, generator=gen) * 0.02 for s in SHAPES]
    pa = [p.clone().to(DEV).requires_grad_(True) for p in p0]
    pb = [p.clone().to(DEV).requires_grad_(True) for p in p0]
    for p in pa + pb:
        p.grad_dtype = None
    oa, ob = LUMA(pa, **HYPER), LUMA(pb, **HYPER)
    ob._base_seed = oa._base_seed
    ob._summaries = False
    for t in range(1, steps + 1):
        if between is not None and t > 1:
            oa, ob = between(t, oa, ob, pa, pb)
        for i, (a, b) in enumerate(zip(pa, pb)):
            g = _grad(t, i, a.shape, dtype, kind).to(DEV)
            a.grad, b.grad = g, g.clone()
        oa.step()
        ob.step()
        torch.cuda.synchronize()
        sa, sb = oa.state_dict()["state"], ob.state_dict()["state"]
        for i in range(len(SHAPES)):
            assert torch.equal(pa[i], pb[i]), (t, i)
            assert torch.equal(sa[i]["Q_m"], sb[i]["Q_m"]), (t, i)
            assert torch.equal(sa[i]["Q_w"], sb[i]["Q_w"]), (t, i)
            assert (sa[i]["S_m"], sa[i]["S_v"]) == (sb[i]["S_m"], sb[i]["S_v"]), (t, i)
        _check_bounds(oa, pa, t)
    return oa, ob


def _check_bounds(opt, params, t):
    chunk = opt._engine._chunk
    for p in params:
        st = opt.state[p]
        slot = st["_slot"]
        summ_step = int(slot[8:16].view(torch.int64).item())
        summ_shift = int(slot[328:332].view(torch.int32).item())
        if p.numel() <= max(L.SMALL_TENSOR, L.MEDIUM_TENSOR) or p.numel() < 2048:
            # stepped by a single wavefront (either route), or below one
            # whole workgroup iteration: no summaries (none allocated), and
            # none claimed
            assert summ_step == 0, summ_step
            continue
        assert summ_step == st["step"], (summ_step, st["step"])
        assert 1 << summ_shift == chunk, (summ_shift, chunk)
        n = p.numel()
        # the word of element e: its chunk's words, then its thread in the chunk
        e = torch.arange(n, device=DEV)
        word = (e // chunk) * L.SUMMARY_WORDS + (e % chunk) % 2048 // 8
        nw = -(-n // chunk) * L.SUMMARY_WORDS
        assert st["_summary"].numel() >= nw
        s = st["_summary"][:nw].to(torch.int64) & 0xFFFFFFFF
        qm = st["Q_m"].reshape(-1).to(torch.int64).abs()
        qw = st["Q_w"].reshape(-1).to(torch.int64) & 0xFFFF
        mx = torch.zeros(nw, dtype=torch.int64, device=DEV).scatter_reduce(0, word, qm, "amax")
        mn = torch.full((nw,), 65535, dtype=torch.int64, device=DEV).scatter_reduce(0, word, qw,
                                                                                   "amin")
        used = torch.zeros(nw, dtype=torch.bool, device=DEV).index_fill(0, word, True)
        lo, hi = (s & 0xFFFF)[used], (s >> 16)[used]
        assert bool((lo >= mx[used]).all()), f"step {t}: max |Q_m| above its summary"
        assert bool((hi <= mn[used]).all()), f"step {t}: min Q_w below its summary"
        # the margin is small: the summary is within a few codes of the codes
        assert int((lo - mx[used]).max()) <= 4 and int((mn[used] - hi).max()) <= 4


@pytest.mark.parametrize("kind", ["moving_max", "outliers", "shrinking"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_summaries_change_nothing(kind, dtype):
    print(f"case summaries kind={kind} dtype={dtype}", flush=True)
    _pair(dtype, kind, 5)


def test_load_and_import_invalidate():
    def between(t, oa, ob, pa, pb):
        if t == 3:      # checkpoint round trip into fresh optimizers
            sa, sb = oa.state_dict(), ob.state_dict()
            oa, ob = LUMA(pa, **HYPER), LUMA(pb, **HYPER)
            ob._summaries = False
            oa.load_state_dict(sa)
            ob.load_state_dict(sb)
            for p in pa:   # restored slots record no summaries
                assert int(oa.state[p]["_slot"][8:16].view(torch.int64).item()) == 0
        if t == 5:      # an AdamW import, from the same exported state
            ex = oa.export_adamw_state()
            oa.import_adamw_state(ex)
            ob.import_adamw_state(ex)
        return oa, ob
    _pair(torch.bfloat16, "moving_max", 6, between)
