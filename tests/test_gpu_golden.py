"""HIP step vs the reference's own outputs (golden vectors from tests/golden/).

The vectors were written by the reference's PyTorch backend
(functional.py:183-298, optimizer.py:413-524) with its seeded generators; the
same uniforms are regenerated here (torch.Generator is portable) and injected
into the HIP step.  Criterion: int16 states equal except +-1 on at most 1e-5
of the codes (the reference's float32 transcendentals are not correctly
rounded, so a code whose bin edge falls between the two results may differ),
S_m / S_v and parameters within 1e-6 relative.
"""

import json
import os

import numpy as np
import pytest
import torch

from luma_amd import LUMA
from oracle import luma_oracle as O

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
RATE = 1e-5
REL = 1e-6


@pytest.fixture(scope="module")
def golden():
    arrays = np.load(os.path.join(HERE, "golden", "luma_golden.npz"), allow_pickle=False)
    with open(os.path.join(HERE, "golden", "luma_golden.json")) as f:
        return arrays, json.load(f)


def _t(a, dtype_name=None):
    t = torch.from_numpy(np.array(a))
    return t.view(torch.bfloat16) if dtype_name == "bfloat16" else t


def _draws(seed, n):
    d = O.generator_draw(seed)
    return d((n,)), d((n,))


def _u16(q):
    return q.to(torch.int32) & 0xFFFF


class Tally:
    def __init__(self):
        self.codes = 0
        self.mismatch = 0
        self.max_dq = 0
        self.s_rel = 0.0
        self.p_rel = 0.0

    def add(self, qm, qw, ref_qm, ref_qw, s, ref_s, p, ref_p):
        qm, qw = qm.cpu().reshape(-1), qw.cpu().reshape(-1)
        ref_qm, ref_qw = ref_qm.reshape(-1), ref_qw.reshape(-1)
        self.codes += 2 * qm.numel()
        self.mismatch += int((qm != ref_qm).sum() + (qw != ref_qw).sum())
        self.max_dq = max(self.max_dq, int((qm.int() - ref_qm.int()).abs().max()),
                          int((_u16(qw) - _u16(ref_qw)).abs().max()))
        for a, b in zip(s, ref_s):
            self.s_rel = max(self.s_rel, abs(a - b) / max(abs(b), 1e-300))
        p = p.detach().cpu().reshape(-1)
        ref_p = ref_p.reshape(-1)
        self.p_rel = max(self.p_rel, float((p - ref_p).abs().max()) /
                         max(float(ref_p.abs().max()), 1e-30))

    def check(self):
        print(f"codes {self.codes} mismatches {self.mismatch} "
              f"({self.mismatch / max(self.codes, 1):.2e}) max|dQ| {self.max_dq} "
              f"S rel {self.s_rel:.2e} p rel {self.p_rel:.2e}", flush=True)
        assert self.max_dq <= 1
        assert self.mismatch <= RATE * self.codes
        assert self.s_rel <= REL and self.p_rel <= REL


def _load(opt, x, t, pid, qm, qw, sm, sv):
    sd = opt.state_dict()
    sd["state"] = {0: {"step": t, "param_id": pid, "Q_m": qm.clone(), "Q_w": qw.clone(),
                       "S_m": sm, "S_v": sv}}
    opt.load_state_dict(sd)


@pytest.mark.parametrize("free_running", [False, True])
def test_functional_vectors(golden, free_running):
    """Each golden case, stepped from the golden state (or free-running)."""
    arrays, meta = golden
    tally = Tally()
    for case, m in meta["functional"].items():
        print(f"case {case}", flush=True)
        hyper = dict(lr=m["lr"], betas=(m["beta1"], m["beta2"]), eps=m["eps"],
                     weight_decay=m["weight_decay"])
        x = _t(arrays[f"f/{case}/param0"]).clone().cuda().requires_grad_(True)
        x.grad_dtype = None
        opt = LUMA([x], **hyper)
        opt._base_seed = m["base_seed"]
        n = x.numel()
        for rec in m["records"]:
            t = rec["t"]
            if t > 1 and not free_running:
                prev = m["records"][t - 2]
                x.data.copy_(_t(arrays[f"f/{case}/param{t - 1}"]))
                _load(opt, x, t - 1, m["param_id"], _t(arrays[f"f/{case}/Q_m{t - 1}"]),
                      _t(arrays[f"f/{case}/Q_w{t - 1}"]), prev["S_m"], prev["S_v"])
            x.grad = _t(arrays[f"f/{case}/grad{t}"], m["grad_dtype"]).cuda()
            u_m, u_w = _draws(rec["seed"], n)
            opt.inject_noise({x: (u_m.cuda(), u_w.cuda())})
            opt.step()
            sd = opt.state_dict()["state"][0]
            tally.add(sd["Q_m"], sd["Q_w"], _t(arrays[f"f/{case}/Q_m{t}"]),
                      _t(arrays[f"f/{case}/Q_w{t}"]), (sd["S_m"], sd["S_v"]),
                      (rec["S_m"], rec["S_v"]), x, _t(arrays[f"f/{case}/param{t}"]))
    tally.check()


def test_optimizer_trajectory(golden):
    """Two groups, skipped grads, five steps (optimizer.py:413-524), plus export."""
    arrays, meta = golden
    om = meta["optimizer"]
    xs = [_t(arrays[f"o/param0_{i}"]).clone().cuda().requires_grad_(True)
          for i in range(len(om["shapes"]))]
    opt = LUMA([{"params": xs[:2], "lr": 2e-3}, {"params": xs[2:], "lr": 5e-4,
                                                  "betas": (0.85, 0.99)}], weight_decay=0.05)
    opt._base_seed = om["base_seed"]
    tally = Tally()
    for t, sm in enumerate(om["steps"], start=1):
        noise = {}
        for i, x in enumerate(xs):
            if i in sm["skipped"]:
                x.grad = None
                continue
            x.grad = _t(arrays[f"o/grad{t}_{i}"]).cuda()
            st = opt.state[x]
            step = (st["step"] if st else 0) + 1
            seed = O.make_step_seed(om["base_seed"], step, i)
            noise[x] = tuple(u.reshape(x.shape).cuda() for u in _draws(seed, x.numel()))
        opt.inject_noise(noise)
        opt.step()
        sd = opt.state_dict()["state"]
        for i, x in enumerate(xs):
            if str(i) in sm["state"]:
                ref = sm["state"][str(i)]
                s = sd[i]
                assert s["step"] == ref["step"] and s["param_id"] == ref["param_id"]
                tally.add(s["Q_m"], s["Q_w"], _t(arrays[f"o/Q_m{t}_{i}"]),
                          _t(arrays[f"o/Q_w{t}_{i}"]), (s["S_m"], s["S_v"]),
                          (ref["S_m"], ref["S_v"]), x, _t(arrays[f"o/param{t}_{i}"]))
            else:
                assert i not in sd
    tally.check()
    ex = opt.export_adamw_state()
    for idx, s in ex["state"].items():
        assert float(s["step"].item()) == om["export"]["steps"][str(idx)]
        for k in ("exp_avg", "exp_avg_sq"):
            ref = _t(arrays[f"o/export_{k}_{idx}"])
            got = s[k].cpu()
            assert torch.allclose(got, ref, rtol=1e-6, atol=0.0), (idx, k)


def test_import_vectors(golden):
    arrays, meta = golden
    om = meta["optimizer"]
    imp = om["import"]
    xs = [torch.zeros(s, device="cuda", requires_grad=True) for s in om["shapes"]]
    luma = LUMA(xs, lr=1e-3, weight_decay=0.01)
    luma._base_seed = imp["base_seed"]
    sd = {"state": {i: {"step": torch.tensor(3.0),
                        "exp_avg": _t(arrays[f"o/adamw_exp_avg_{i}"]).cuda(),
                        "exp_avg_sq": _t(arrays[f"o/adamw_exp_avg_sq_{i}"]).cuda()}
                    for i in range(len(xs))}}
    luma.inject_noise({x: tuple(u.reshape(x.shape).cuda() for u in
                                _draws(O.make_step_seed(imp["base_seed"], 0, i), x.numel()))
                       for i, x in enumerate(xs)})
    luma.import_adamw_state(sd)
    out = luma.state_dict()["state"]
    tally = Tally()
    for i, x in enumerate(xs):
        ref = imp["state"][str(i)]
        assert out[i]["step"] == ref["step"] and out[i]["param_id"] == ref["param_id"]
        tally.add(out[i]["Q_m"], out[i]["Q_w"], _t(arrays[f"o/import_Q_m_{i}"]),
                  _t(arrays[f"o/import_Q_w_{i}"]), (out[i]["S_m"], out[i]["S_v"]),
                  (ref["S_m"], ref["S_v"]), x, x.detach().cpu())
    tally.check()
