"""Drive the HIP LUMA and the CPU oracle side by side on the same inputs.

The oracle draws its uniforms exactly as the reference does (seeded generator
per (param, step)); the same uniforms are injected into the HIP step, so the
int16 states can be compared element for element.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Callable, List

import torch

from luma_amd import LUMA
from oracle import luma_oracle as O


@dataclass
class StepStats:
    t: int
    n: int = 0
    qm_mismatch: int = 0
    qw_mismatch: int = 0
    q_max_abs_diff: int = 0
    s_rel: float = 0.0
    p_rel: float = 0.0
    s_exact: bool = True


@dataclass
class PairResult:
    steps: List[StepStats] = field(default_factory=list)
    # per step: {"S_m": [per tensor], "S_v": [per tensor]} of the HIP optimizer
    scales: List[dict] = field(default_factory=list)

    def total_mismatch(self):
        return sum(s.qm_mismatch + s.qw_mismatch for s in self.steps)

    def worst_rate(self):
        return max((s.qm_mismatch + s.qw_mismatch) / (2 * s.n) for s in self.steps)


def normal_grads(std=1e-3, dtype=torch.float32, seed=1000):
    def fn(t, i, shape):
        g = torch.Generator().manual_seed(seed + 7919 * t + i)
        return (torch.randn(shape, generator=g) * std).to(dtype)
    return fn


def _u16(q):
    return q.to(torch.int32) & 0xFFFF


def run_pair(shapes, grad_fn: Callable, n_steps: int, math_mode: str = "cr",
             hyper=None, resync: bool = False, base_seed: int = 0x5DEECE66D,
             init_std: float = 0.02, groups_split=None, chunk_elems: int = 0) -> PairResult:
    """Step the HIP optimizer and the oracle ``n_steps`` times; compare each step.

    ``resync`` loads the oracle's state into the HIP optimizer before every
    step, so each comparison is one step from an identical state.
    ``chunk_elems`` fixes the step's chunk length (0: the optimizer's choice).
    """
    hyper = dict(hyper or dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01))
    gen = torch.Generator().manual_seed(12345)
    cpu = [(torch.randn(s, generator=gen) * init_std).float() for s in shapes]
    dev = [p.clone().cuda().requires_grad_(True) for p in cpu]
    for p in cpu + dev:
        p.grad_dtype = None   # allow bf16 / fp16 grads on fp32 params
    if groups_split is None:
        groups_cpu = [dict(params=cpu, **hyper)]
        groups_dev = [dict(params=dev)]
    else:
        groups_cpu = [dict(params=cpu[:groups_split], **hyper), dict(params=cpu[groups_split:], **hyper)]
        groups_dev = [dict(params=dev[:groups_split]), dict(params=dev[groups_split:])]
    oracle = O.OracleLUMA(groups_cpu, base_seed, math_mode)
    opt = LUMA(groups_dev, **hyper)
    opt._base_seed = base_seed
    if chunk_elems:
        opt._get_engine(dev[0].device).chunk_elems = chunk_elems
    res = PairResult()
    for t in range(1, n_steps + 1):
        if resync and t > 1:
            sd = opt.state_dict()
            for i, p in enumerate(cpu):
                st = oracle.state[id(p)]
                sd["state"][i] = {"step": st["step"], "param_id": st["param_id"],
                                  "Q_m": st["Q_m"].clone(), "Q_w": st["Q_w"].clone(),
                                  "S_m": st["S_m"], "S_v": st["S_v"]}
                dev[i].data.copy_(p)
            opt.load_state_dict(sd)
        grads = [grad_fn(t, i, tuple(p.shape)) for i, p in enumerate(cpu)]
        for p, g in zip(cpu, grads):
            p.grad = g
        oracle.step()
        noise = {}
        for i, (dp, g) in enumerate(zip(dev, grads)):
            dp.grad = g.cuda()
            u_m, u_w = oracle.last_draws[i]
            noise[dp] = (u_m.cuda(), u_w.cuda())
        opt.inject_noise(noise)
        opt.step()
        torch.cuda.synchronize()
        sd = opt.state_dict()
        st = StepStats(t=t)
        for i, p in enumerate(cpu):
            o = oracle.state[id(p)]
            s = sd["state"][i]
            qm, qw = s["Q_m"].cpu(), s["Q_w"].cpu()
            st.n += p.numel()
            st.qm_mismatch += int((qm != o["Q_m"]).sum())
            st.qw_mismatch += int((qw != o["Q_w"]).sum())
            dq = max(int((qm.int() - o["Q_m"].int()).abs().max()),
                     int((_u16(qw) - _u16(o["Q_w"])).abs().max()))
            st.q_max_abs_diff = max(st.q_max_abs_diff, dq)
            for a, b in ((s["S_m"], o["S_m"]), (s["S_v"], o["S_v"])):
                if a != b:
                    st.s_exact = False
                rel = abs(a - b) / max(abs(b), 1e-300)
                if not math.isnan(rel):
                    st.s_rel = max(st.s_rel, rel)
            pd = dev[i].detach().cpu()
            scale = float(p.abs().max())
            st.p_rel = max(st.p_rel, float((pd - p).abs().max()) / max(scale, 1e-30))
        res.steps.append(st)
        res.scales.append({k: [sd["state"][i][k] for i in range(len(cpu))] for k in ("S_m", "S_v")})
    return res
