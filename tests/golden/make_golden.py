"""Write golden vectors for the LUMA step by running the reference on CPU.

Run in the build container only (the reference sources are not present on
the GPU machines):

    python tests/golden/make_golden.py

It imports the reference's PyTorch backend from
``/root/reference/src/luma_optimizer`` and records inputs and outputs of

* ``functional.luma_init_step`` / ``luma_update_step`` (functional.py:183-298)
  over five steps for a set of tensors (sizes 1..65543, fp32/bf16/fp16
  grads, all-zero and single-outlier grads), each with its seeded generator;
* ``LUMA.step`` (optimizer.py:413-524) on a two-group parameter set where
  some grads are ``None`` on some steps, plus ``state_dict()``,
  ``export_adamw_state()`` and ``import_adamw_state()``.

Outputs: ``tests/golden/luma_golden.npz`` (arrays only, load with
``allow_pickle=False``) and ``tests/golden/luma_golden.json`` (scalars and
provenance).  bf16 tensors are stored as their int16 bit patterns.
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REF_SRC = "/root/reference/src"


def _np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().copy()
    return t.numpy().copy()


def _make_grad(gen, n, dtype, kind):
    g = torch.randn(n, generator=gen) * 1e-3
    if kind == "zeros":
        g = torch.zeros(n)
    elif kind == "outlier":
        g[n // 3] = 0.5
    elif kind == "heavy":
        mask = torch.rand(n, generator=gen) < 0.01
        g[mask] = 0.0
        out = torch.rand(n, generator=gen) < 0.002
        g[out] *= 100.0
    return g.to(dtype)


FUNCTIONAL_CASES = [
    # name, n, grad dtype, kind, hyper (lr, b1, b2, eps, wd), steps
    ("n1_f32", 1, torch.float32, "normal", (1e-3, 0.9, 0.999, 1e-8, 0.01), 5),
    ("n127_bf16", 127, torch.bfloat16, "normal", (1e-3, 0.9, 0.999, 1e-8, 0.01), 5),
    ("n4096_f16", 4096, torch.float16, "normal", (1e-3, 0.9, 0.999, 1e-8, 0.01), 5),
    ("n65543_f32", 65543, torch.float32, "heavy", (1e-3, 0.9, 0.999, 1e-8, 0.01), 3),
    ("zeros_f32", 300, torch.float32, "zeros", (1e-3, 0.9, 0.999, 1e-8, 0.01), 4),
    ("outlier_bf16", 1000, torch.bfloat16, "outlier", (1e-3, 0.9, 0.999, 1e-8, 0.01), 5),
    ("hyper2_f32", 2048, torch.float32, "normal", (5e-4, 0.95, 0.98, 1e-6, 0.1), 5),
]


def functional_vectors(RF, arrays, meta):
    for ci, (name, n, gdt, kind, (lr, b1, b2, eps, wd), steps) in enumerate(FUNCTIONAL_CASES):
        gen = torch.Generator().manual_seed(1000 + ci)
        param = (torch.randn(n, generator=gen) * 0.02).float()
        arrays[f"f/{name}/param0"] = _np(param)
        seed_base = int(torch.randint(-(2**63), 2**63 - 1, (1,), generator=gen).item())
        pid = ci
        recs = []
        Q_m = Q_w = None
        S_m = S_v = None
        for t in range(1, steps + 1):
            grad = _make_grad(gen, n, gdt, kind)
            arrays[f"f/{name}/grad{t}"] = _np(grad)
            seed = RF._make_step_seed(seed_base, t, pid)
            g = torch.Generator()
            g.manual_seed(seed)
            if t == 1:
                Q_m, Q_w, S_m, S_v = RF.luma_init_step(param, grad, b1, b2, eps, lr, wd,
                                                       generator=g)
            else:
                S_m, S_v = RF.luma_update_step(param, grad, Q_m, Q_w, S_m, S_v, t,
                                               b1, b2, eps, lr, wd, generator=g)
            arrays[f"f/{name}/param{t}"] = _np(param)
            arrays[f"f/{name}/Q_m{t}"] = _np(Q_m)
            arrays[f"f/{name}/Q_w{t}"] = _np(Q_w)
            recs.append({"t": t, "seed": seed, "S_m": S_m, "S_v": S_v})
        meta["functional"][name] = {
            "n": n, "grad_dtype": str(gdt).replace("torch.", ""), "kind": kind,
            "lr": lr, "beta1": b1, "beta2": b2, "eps": eps, "weight_decay": wd,
            "steps": steps, "param_id": pid, "base_seed": seed_base, "records": recs,
        }


def optimizer_vectors(LUMA, arrays, meta):
    """Two groups; param 1 gets no grad on step 2, param 3 none until step 3."""
    torch.manual_seed(7)
    shapes = [(8, 16), (16,), (4, 8), (8,)]
    params = [torch.nn.Parameter(torch.randn(*s) * 0.05) for s in shapes]
    for i, p in enumerate(params):
        arrays[f"o/param0_{i}"] = _np(p.data)
    torch.manual_seed(42)
    opt = LUMA([{"params": params[:2], "lr": 2e-3},
                {"params": params[2:], "lr": 5e-4, "betas": (0.85, 0.99)}],
               weight_decay=0.05, backend="pytorch")
    meta["optimizer"] = {"base_seed": opt._base_seed, "shapes": shapes, "steps": []}
    gen = torch.Generator().manual_seed(99)
    n_steps = 5
    for t in range(1, n_steps + 1):
        for i, p in enumerate(params):
            g = torch.randn(p.shape, generator=gen) * 1e-2
            skip = (i == 1 and t == 2) or (i == 3 and t < 3)
            p.grad = None if skip else g
            arrays[f"o/grad{t}_{i}"] = _np(g)
        opt.step()
        step_meta = {"skipped": [i for i, p in enumerate(params) if p.grad is None],
                     "state": {}}
        for i, p in enumerate(params):
            arrays[f"o/param{t}_{i}"] = _np(p.data)
            st = opt.state[p]
            if st:
                arrays[f"o/Q_m{t}_{i}"] = _np(st["Q_m"])
                arrays[f"o/Q_w{t}_{i}"] = _np(st["Q_w"])
                step_meta["state"][i] = {"step": st["step"], "param_id": st["param_id"],
                                         "S_m": st["S_m"], "S_v": st["S_v"]}
        meta["optimizer"]["steps"].append(step_meta)

    sd = opt.state_dict()
    meta["optimizer"]["state_dict"] = {
        "keys": sorted(sd.keys()),
        "state_keys": {int(k): sorted(v.keys()) for k, v in sd["state"].items()},
        "param_groups": [{k: (list(v) if isinstance(v, tuple) else v)
                          for k, v in g.items()} for g in sd["param_groups"]],
        "_base_seed": sd["_base_seed"],
    }
    ex = opt.export_adamw_state()
    for idx, s in ex["state"].items():
        arrays[f"o/export_exp_avg_{idx}"] = _np(s["exp_avg"])
        arrays[f"o/export_exp_avg_sq_{idx}"] = _np(s["exp_avg_sq"])
    meta["optimizer"]["export"] = {
        "steps": {int(i): float(s["step"].item()) for i, s in ex["state"].items()},
        "param_groups": [{k: (list(v) if isinstance(v, tuple) else v)
                          for k, v in g.items()} for g in ex["param_groups"]],
    }

    # import_adamw_state from a short AdamW run on fresh params
    torch.manual_seed(11)
    pa = [torch.nn.Parameter(torch.randn(*s) * 0.05) for s in shapes]
    adamw = torch.optim.AdamW(pa, lr=1e-3, weight_decay=0.01)
    for _ in range(3):
        for p in pa:
            p.grad = torch.randn(p.shape, generator=gen) * 1e-2
        adamw.step()
    asd = adamw.state_dict()
    for idx, s in asd["state"].items():
        arrays[f"o/adamw_exp_avg_{idx}"] = _np(s["exp_avg"])
        arrays[f"o/adamw_exp_avg_sq_{idx}"] = _np(s["exp_avg_sq"])
    torch.manual_seed(5)
    luma = LUMA(pa, lr=1e-3, weight_decay=0.01, backend="pytorch")
    luma.import_adamw_state(asd)
    imp = {"base_seed": luma._base_seed, "state": {}}
    for i, p in enumerate(pa):
        st = luma.state[p]
        arrays[f"o/import_Q_m_{i}"] = _np(st["Q_m"])
        arrays[f"o/import_Q_w_{i}"] = _np(st["Q_w"])
        imp["state"][i] = {"step": st["step"], "param_id": st["param_id"],
                           "S_m": st["S_m"], "S_v": st["S_v"]}
    meta["optimizer"]["import"] = imp


def main():
    sys.path.insert(0, REF_SRC)
    import luma_optimizer.functional as RF  # noqa: E402
    from luma_optimizer import LUMA  # noqa: E402

    torch.set_num_threads(1)
    arrays: dict = {}
    meta = {"torch": torch.__version__,
            "cpu_capability": torch.backends.cpu.get_cpu_capability(),
            "num_threads": 1,
            "functional": {}}
    functional_vectors(RF, arrays, meta)
    optimizer_vectors(LUMA, arrays, meta)
    np.savez_compressed(os.path.join(HERE, "luma_golden.npz"), **arrays)
    with open(os.path.join(HERE, "luma_golden.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)
    print("wrote", len(arrays), "arrays")


if __name__ == "__main__":
    main()
