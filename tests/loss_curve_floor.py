"""Noise floor of the 1,000-step loss-curve criterion: the oracle against
itself, on the CPU only.

    python tests/loss_curve_floor.py [--jobs 4] [--threads 2]

The model, text, batches and evaluation are those of
tests/test_gpu_loss_curve.py (tests/loss_curve_model.py), run on the CPU.
Every run trains the model with the oracle (the reference's PyTorch backend
restated, oracle/luma_oracle.py) on the same batches from the same start;
the runs differ only as named:

  base    correctly rounded math ("cr"), base seed S0
  seedK   "cr", another base seed (K = 1..4): independent stochastic rounding,
          the spread that HIP Philox against the CPU generator can reach
  torch   the reference's own ATen CPU math, S0 (same draws): the spread
          between the reference's arithmetic and correctly rounded arithmetic
  ulp     "cr", S0, one weight moved by one ulp after step 1
  ulpall  "cr", S0, after every step 0.1% of every tensor's elements moved
          by one ulp up or down: a last-bit difference in the update

Each evaluation point's relative difference from `base` is printed, with
the largest over the curve and the relative difference of the curve means.

Measured (torch 2.10 CPU, 8-core Xeon with AVX-512; eval losses of the base
run 2.830 at step 100 to 0.721 at step 1000):

  run      largest point difference (step)   difference of the means
  seed1    0.98% (1000)                      6.7e-4
  seed2    1.17% (700)                       1.1e-3
  seed3    0.31% (800)                       3.4e-4
  seed4    1.61% (700)                       1.1e-3
  torch    1.09% (1000)                      5.3e-4
  ulp      0.27% (900)                       1.7e-4
  ulpall   0.32% (1000)                      1.7e-5

Up to step 600 every run stays within 5e-4 of the base; from step 700, while
the loss falls fastest, training amplifies any difference, a last-bit one
included, to about 1%.  So the reference against itself -- with another
seed, or on a host whose math library rounds differently -- misses a 0.5%
per-point bound.  The test's per-point tolerances come from this table.
"""

import argparse
import json
import os
import subprocess
import sys
import tempfile
import time

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
for p in (ROOT, HERE):
    if p not in sys.path:
        sys.path.insert(0, p)

VARIANTS = ("base", "seed1", "seed2", "seed3", "seed4", "torch", "ulp", "ulpall")
S0 = 0x1234_5678_9ABC_DEF0 - (1 << 63)
SEEDS = {1: 0x0FED_CBA9_8765_4321}
_GOLD = 0x9E37_79B9_7F4A_7C15


def base_seed(variant: str) -> int:
    if variant.startswith("seed"):
        k = int(variant[4:])
        return SEEDS.get(k, S0 ^ (k * _GOLD & ((1 << 63) - 1)))
    return S0


def run(variant: str) -> list:
    """One training run; returns [(step, eval loss)] every EVAL_EVERY steps."""
    import loss_curve_model as M
    from oracle import luma_oracle as O

    model, train, val_batches = M.setup("cpu")
    params = list(model.parameters())
    oracle = O.OracleLUMA(M.groups(params), base_seed(variant),
                          math_mode="torch" if variant == "torch" else "cr")
    batches = M.batches(train, 7)
    nudge = torch.Generator().manual_seed(5)
    curve = []
    for step in range(1, M.STEPS + 1):
        x, y = next(batches)
        model.zero_grad(set_to_none=True)
        model(x, y).backward()
        torch.nn.utils.clip_grad_norm_(model.parameters(), M.CLIP)
        oracle.step()
        with torch.no_grad():
            if variant == "ulp" and step == 1:
                f = params[4].view(-1)          # block 0's qkv weight
                f[3] = torch.nextafter(f[3], torch.tensor(float("inf")))
            if variant == "ulpall":
                for p in params:
                    f = p.view(-1)
                    sel = torch.rand(f.numel(), generator=nudge) < 1e-3
                    up = torch.rand(f.numel(), generator=nudge) < 0.5
                    to = torch.where(up, torch.full_like(f, float("inf")),
                                     torch.full_like(f, float("-inf")))
                    f[sel] = torch.nextafter(f[sel], to[sel])
        if step % M.EVAL_EVERY == 0:
            curve.append((step, M.evaluate(model, val_batches)))
            print(f"{variant} step {step}: {curve[-1][1]:.4f}", file=sys.stderr, flush=True)
    return curve


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    ap.add_argument("--threads", type=int, default=2)
    ap.add_argument("--variant", choices=VARIANTS, help=argparse.SUPPRESS)
    ap.add_argument("--out", help=argparse.SUPPRESS)
    a = ap.parse_args()
    torch.set_num_threads(a.threads)
    if a.variant:
        with open(a.out, "w") as f:
            json.dump(run(a.variant), f)
        return
    tmp = tempfile.mkdtemp(prefix="luma_floor_")
    out = {v: os.path.join(tmp, v + ".json") for v in VARIANTS}
    pending, procs = list(VARIANTS), []
    t0 = time.time()
    while pending or procs:
        while pending and len(procs) < a.jobs:
            v = pending.pop(0)
            procs.append(subprocess.Popen([sys.executable, __file__, "--variant", v, "--out",
                                           out[v], "--threads", str(a.threads)]))
        time.sleep(1)
        for p in [p for p in procs if p.poll() is not None]:
            if p.returncode:
                raise SystemExit(f"a run failed: {p.args}")
            procs.remove(p)
    curves = {v: json.load(open(out[v])) for v in VARIANTS}
    base = curves["base"]
    mean_b = sum(c[1] for c in base) / len(base)
    print(f"base: {' '.join(f'{c[1]:.4f}' for c in base)}  ({time.time() - t0:.0f} s)")
    for v in VARIANTS[1:]:
        rel = [abs(c[1] - b[1]) / b[1] for c, b in zip(curves[v], base)]
        k = max(range(len(rel)), key=rel.__getitem__)
        mean = sum(c[1] for c in curves[v]) / len(curves[v])
        print(f"{v:7s} largest {100 * rel[k]:.2f}% (step {base[k][0]})  means {abs(mean - mean_b) / mean_b:.1e}"
              f"  | {' '.join(f'{r:.1e}' for r in rel)}")


if __name__ == "__main__":
    main()
