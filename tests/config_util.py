"""Parity of the HIP step with the CPU oracle on whole benchmark workloads.

The HIP optimizer steps every tensor of a parameter set on the GPU; the
oracle steps a chosen sample of them on the CPU (all of them for the smaller
sets).  The oracle's own uniforms are injected into the HIP step for the
sampled tensors only; the others draw from Philox.  Each sampled tensor is
compared after every step: codes and scales exactly, parameters within
1e-6 * max|p| + 1e-8 (the parameter criterion of the reference's parity
tests, tests/test_correctness.py:265-285; the codes, which those tests
leave free, are exact against the correctly rounded oracle).

The oracle sees every parameter in order (unsampled ones as empty
placeholders without a gradient), so the sampled tensors keep their
param_id, and with it their seeds.
"""

from __future__ import annotations

import math
import time
from typing import Callable, Dict, List, Optional, Sequence

import torch

from luma_amd import LUMA
from oracle import luma_oracle as O

HYPER = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
P_TOL = 1e-6


def _u16(q):
    return q.to(torch.int32) & 0xFFFF


class SampledPair:
    """HIP LUMA over ``params`` (GPU, float32) and the oracle over
    ``params[i]`` for i in ``sample``."""

    def __init__(self, params: Sequence[torch.Tensor], sample: Sequence[int],
                 base_seed: int = 0x5DEECE66D, hyper=None, math_mode: str = "cr"):
        self.hyper = dict(hyper or HYPER)
        self.params = list(params)
        for p in self.params:
            p.requires_grad_(True)
            p.grad_dtype = None          # bf16 / fp16 grads on fp32 params
        self.sample = sorted(set(sample))
        self.cpu: Dict[int, torch.Tensor] = {}
        flat = []
        chosen = set(self.sample)
        for i, p in enumerate(self.params):
            if i not in chosen:
                flat.append(torch.empty(0))   # counted in param_id, never stepped
                continue
            c = p.detach().cpu().clone()
            c.grad_dtype = None
            self.cpu[i] = c
            flat.append(c)
        self.base_seed = base_seed
        self.oracle = O.OracleLUMA([dict(params=flat, **self.hyper)], base_seed, math_mode)
        self.opt = self._new_opt()
        self.t = 0
        self.log: List[str] = []

    def _new_opt(self) -> LUMA:
        opt = LUMA(self.params, **self.hyper)
        opt._base_seed = self.base_seed
        return opt

    def restore(self):
        """Checkpoint round trip: state_dict of the current optimizer, loaded
        into a fresh one, which takes the following steps."""
        sd = self.opt.state_dict()
        self.opt = self._new_opt()
        self.opt.load_state_dict(sd)
        del sd

    def step(self, grads_dev: Sequence[torch.Tensor], grads_cpu: Dict[int, torch.Tensor],
             driver: Optional[Callable[[LUMA], None]] = None):
        """One step of both.  ``grads_dev`` are the GPU gradients the HIP
        optimizer sees; ``grads_cpu[i]`` the gradient the oracle sees for
        sampled tensor i (the same values, unscaled).  ``driver(opt)`` makes
        the HIP step (default ``opt.step()``), e.g. through a GradScaler."""
        self.t += 1
        t0 = time.perf_counter()
        for i, c in self.cpu.items():
            c.grad = grads_cpu[i]
        self.oracle.step()
        t1 = time.perf_counter()
        for p, g in zip(self.params, grads_dev):
            p.grad = g
        noise = {}
        for i in self.sample:
            u_m, u_w = self.oracle.last_draws[i]
            noise[self.params[i]] = (u_m.to(self.params[i].device), u_w.to(self.params[i].device))
        self.opt.inject_noise(noise, strict=False)
        if driver is None:
            self.opt.step()
        else:
            driver(self.opt)
        torch.cuda.synchronize()
        self.log.append(f"t={self.t}: oracle {t1 - t0:.1f} s, HIP {time.perf_counter() - t1:.1f} s")
        print(self.log[-1], flush=True)

    def compare(self) -> List[dict]:
        """Per sampled tensor: code mismatches, max |dQ|, scale equality and
        the parameters' largest difference relative to their largest value."""
        sd = self.opt.state_dict()["state"]
        out = []
        for i in self.sample:
            o = self.oracle.state[id(self.cpu[i])]
            s = sd[i]
            qm, qw = s["Q_m"].cpu(), s["Q_w"].cpu()
            pd = self.params[i].detach().cpu()
            pc = self.cpu[i]
            out.append(dict(
                i=i, n=pc.numel(), t=self.t,
                qm_mismatch=int((qm != o["Q_m"]).sum()),
                qw_mismatch=int((qw != o["Q_w"]).sum()),
                dq=max(int((qm.int() - o["Q_m"].int()).abs().max()),
                       int((_u16(qw) - _u16(o["Q_w"])).abs().max())),
                s_exact=(s["S_m"] == o["S_m"] and s["S_v"] == o["S_v"]),
                p_diff=float((pd - pc).abs().max()), p_scale=float(pc.abs().max()),
                p_rel=float((pd - pc).abs().max()) / max(float(pc.abs().max()), 1e-30),
                step=s["step"]))
        return out

    def check(self):
        """Compare and assert the exact criterion for every sampled tensor."""
        rows = self.compare()
        for r in rows:
            assert r["qm_mismatch"] == 0 and r["qw_mismatch"] == 0, r
            assert r["s_exact"], r
            assert r["p_diff"] <= P_TOL * r["p_scale"] + 1e-8, r
            assert r["step"] == self.t, r
        return rows


def normal_grad(shape, std, gen, device, dtype, outliers=0.0, zeros=0.0):
    """N(0, std) on the device, with a fraction ``outliers`` of elements x100
    and a fraction ``zeros`` set to exactly 0, cast to ``dtype``."""
    g = torch.randn(shape, device=device, generator=gen) * std
    if outliers:
        g = torch.where(torch.rand(shape, device=device, generator=gen) < outliers, g * 100.0, g)
    if zeros:
        g = torch.where(torch.rand(shape, device=device, generator=gen) < zeros,
                        torch.zeros_like(g), g)
    return g.to(dtype)


def numel(shape) -> int:
    return math.prod(shape)
