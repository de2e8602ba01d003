"""1,000-step training curves: HIP LUMA vs the CPU oracle (the reference's
PyTorch backend restated) on a nanoGPT-shaped model (tests/loss_curve_model.py:
the reference benchmark's 4-layer, 128-wide configuration, on synthetic text).

Two identical models see the same batches.  Model A steps with ``luma_amd.LUMA``
on the GPU; model B's gradients go to the CPU, the oracle steps its float32
copies, and the parameters come back.  Evaluation losses on fixed held-out
batches are compared every 100 steps, in three modes:

* exact -- injected noise (the oracle's generator draws fed to the HIP step)
  and the library's exact per-element path (LUMA_FLAG_EXACT_ONLY), whose
  parameter update is the reference's float32 operation sequence: the two
  runs must stay identical to within 1e-6 at every evaluation point;
* injected -- injected noise, production (fast) path: the codes are
  identical and the update within 1e-6 per step, but not the reference's
  bits;
* native -- HIP draws from Philox, the oracle from torch.Generator, so the
  curves are two independent samples of the same stochastic rounding.

The per-point tolerance of the last two is the criterion's own noise floor,
measured with the oracle against itself (tests/loss_curve_floor.py, CPU):
up to step 600 every perturbed run stays within 5e-4, but while the loss
falls fastest (steps 700-1000) training amplifies any difference, a one-ulp
one included.  The reference's ATen math against correctly rounded math,
same draws, differs by up to 1.09% (step 1000); four other base seeds by up
to 0.98%, 1.17%, 0.31% and 1.61%.  The reference's own backend-agreement
threshold, 0.5% (tests/test_correctness.py:333-339, a 100-step quadratic),
is below that floor.  So:

* injected: every point within 1.1% (the largest same-draws spread, ATen
  against correctly rounded math; measured on MI355X: 0.84% at step 1000),
  and the curve means within 2e-3 (floor 5.3e-4);
* native: every point within 1.7% (the largest other-seed spread, 1.61%;
  measured on MI355X: 0.77%), and the curve means within 5e-3 (floor 1.1e-3).
"""

import time

import pytest
import torch

import loss_curve_model as M
from luma_amd import LUMA
from luma_amd import _lib as L
from oracle import luma_oracle as O

pytestmark = pytest.mark.gpu

POINT_TOL = {"injected": 1.1e-2, "native": 1.7e-2, "exact": 1e-6}
MEAN_TOL = {"injected": 2e-3, "native": 5e-3, "exact": 1e-6}


def _run(inject, exact=False):
    model_a, train, val_batches = M.setup("cuda")
    # a second model initialised as the first was (drawing from the global
    # generator, which LUMA's _base_seed draw follows), then made equal to it
    model_b = M.TinyGPT(model_a.wte.num_embeddings).cuda()
    model_b.load_state_dict(model_a.state_dict())
    params_a = list(model_a.parameters())
    params_b = list(model_b.parameters())
    cpu_b = [p.detach().cpu().clone() for p in params_b]

    opt = LUMA(M.groups(params_a))
    if exact:
        opt._flags = L.FLAG_EXACT_ONLY
    oracle = O.OracleLUMA(M.groups(cpu_b), opt._base_seed, math_mode="cr")
    order_a = [p for g in opt.param_groups for p in g["params"]]

    curve = []
    batches = M.batches(train, 7, "cuda")
    t0 = time.time()
    for step in range(1, M.STEPS + 1):
        x, y = next(batches)
        for model in (model_a, model_b):
            model.zero_grad(set_to_none=True)
            model(x, y).backward()
            torch.nn.utils.clip_grad_norm_(model.parameters(), M.CLIP)
        for pb, cb in zip(params_b, cpu_b):
            cb.grad = pb.grad.detach().cpu()
        oracle.step()
        if inject:
            noise = {}
            for pid, pa in enumerate(order_a):
                u_m, u_w = oracle.last_draws[pid]
                noise[pa] = (u_m.reshape(pa.shape).cuda(), u_w.reshape(pa.shape).cuda())
            opt.inject_noise(noise)
        opt.step()
        with torch.no_grad():
            for pb, cb in zip(params_b, cpu_b):
                pb.copy_(cb)
        if step % M.EVAL_EVERY == 0:
            la, lb = M.evaluate(model_a, val_batches), M.evaluate(model_b, val_batches)
            curve.append((step, la, lb))
            print(f"step {step}: HIP {la:.4f} oracle {lb:.4f} rel {abs(la - lb) / lb:.2e} "
                  f"({time.time() - t0:.0f}s)", flush=True)
    return curve


@pytest.mark.timeout(600)
@pytest.mark.parametrize("mode", ["injected", "native", "exact"])
def test_loss_curves_match_oracle(mode):
    print(f"case loss curve {mode}", flush=True)
    curve = _run(mode != "native", exact=mode == "exact")
    first, last = curve[0], curve[-1]
    assert last[2] < first[2] - 0.5, "the model did not train"
    for step, la, lb in curve:
        assert abs(la - lb) / lb <= POINT_TOL[mode], (step, la, lb)
    mean_a = sum(c[1] for c in curve) / len(curve)
    mean_b = sum(c[2] for c in curve) / len(curve)
    print(f"mean eval loss HIP {mean_a:.4f} oracle {mean_b:.4f}", flush=True)
    assert abs(mean_a - mean_b) / mean_b <= MEAN_TOL[mode]
