"""Benchmark of the LUMA optimizer step on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config llama3_8b]
                    [--no-cpu] [--no-others] [--no-pretouch]

A step is one ``LUMA.step()`` over the whole synthetic parameter set with
gradients already resident in HBM.  Two gradient sets, drawn independently
from the workload's distribution, alternate through the warm-up and timed
steps, so that every step sees fresh gradients.  Before any of that, a
short-lived child process writes 90% of the free HBM once and releases it
(--no-pretouch skips it): on a freshly started machine, the first process to
allocate most of the HBM runs the streaming kernels about 6% slower for its
whole life (pass 2 on the 8B set 29.9 ms against 28.1 ms), and a process
started after HBM was written once does not.  Prints one JSON line with:
  value        Gparams/s of the whole step (params / ms_per_step) on the
               headline workload (the 8B-parameter Llama-3-shaped set)
  roofline     the dominant kernel's algorithmic HBM bytes per launch over its
               average launch time (HIP events on the launch stream) vs 8 TB/s
  cpu_baseline the CPU oracle (the reference's PyTorch backend restated) timed
               on this host on a bounded sample of the same workload
  other_configs  (default run) the single 4096x4096 tensor, the GPT-2-small list
               and the 20,000-tensor set at their stated step counts: step time
               from HIP events around each step() (the gradient switch between
               steps is host work outside them), Gparams/s, the reference
               bytes model's fraction of 8 TB/s, and each one's CPU baseline
               on its whole parameter set
Bytes per parameter (G = gradient element size):
  reference algorithm  pass 1 reads grad + Q_m + Q_w (G + 4), pass 2 reads grad +
                       Q_m + Q_w + param and writes Q_m + Q_w + param (G + 16):
                       2G + 20 per step (the reference's own traffic model)
  this implementation  pass 1 reads the gradients and one summary word per 256
                       threads x chunk, and reads codes only for the groups that
                       can hold a tensor's maximum (a few per tensor once the
                       step has run twice): G + 1024 / chunk; pass 2 as above
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
import types

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "LUMA step Gparams/s + achieved HBM GB/s (% of peak), 8B-param fp32 set"
HBM_PEAK = 8.0e12


# ── synthetic parameter sets ─────────────────────────────────────────────────

def llama3_8b_shapes():
    """Llama-3-8B: 32 layers of q/k/v/o, gate/up/down, two RMSNorms; embed, lm_head, norm."""
    shapes = [(128256, 4096)]
    for _ in range(32):
        shapes += [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096),
                   (14336, 4096), (14336, 4096), (4096, 14336), (4096,), (4096,)]
    shapes += [(4096,), (128256, 4096)]
    return shapes


def gpt2_small_shapes():
    shapes = [(50257, 768), (1024, 768)]
    for _ in range(12):
        shapes += [(768,), (768,), (768, 2304), (2304,), (768, 768), (768,),
                   (768,), (768,), (768, 3072), (3072,), (3072, 768), (768,)]
    shapes += [(768,), (768,)]
    return shapes


def many_small_shapes(n=20000, seed=3):
    g = torch.Generator().manual_seed(seed)
    u = torch.rand(n, generator=g, dtype=torch.float64)
    sizes = torch.exp(u * math.log(65536.0)).round().clamp(1, 65536).long().tolist()
    return [(s,) for s in sizes]


CONFIGS = {
    "llama3_8b": dict(shapes=llama3_8b_shapes, grad=torch.bfloat16, std=1e-3, outliers=1e-3,
                      desc="Llama-3-8B-shaped fp32 param set (291 tensors), bf16 grads "
                           "N(0,1e-3) with 0.1% x100 outliers"),
    "llama3_8b_hetero": dict(shapes=llama3_8b_shapes, grad=torch.float16, hetero=(1e-7, 1e-1, 5),
                             restore=True,
                             desc="Llama-3-8B-shaped fp32 param set (291 tensors), per-tensor grad std "
                                  "log-uniform in [1e-7, 1e-1], fp16 grads scaled by 2^16 and "
                                  "unscaled (GradScaler path), stepping from a restored state_dict"),
    "gpt2_small": dict(shapes=gpt2_small_shapes, grad=torch.bfloat16, std=1e-3, outliers=0.0,
                       desc="GPT-2-small-shaped fp32 param list (148 tensors), bf16 grads N(0,1e-3)"),
    "many_small": dict(shapes=many_small_shapes, grad=torch.float32, std=1e-4, outliers=0.0,
                       zeros=0.01, desc="20,000 fp32 tensors, sizes log-uniform in [1, 65536], "
                                        "fp32 grads N(0,1e-4) with 1% exact zeros"),
    "single_4096": dict(shapes=lambda: [(4096, 4096)], grad=torch.float32, std=1e-3,
                        outliers=0.0, desc="single fp32 4096x4096 param, fp32 grads N(0,1e-3)"),
}


def make_set(cfg, device, grad_sets=2):
    """Parameters and `grad_sets` gradient sets of a configuration (each set
    drawn afresh from the configuration's distribution); the steps of a run
    cycle through the sets, so that no two consecutive steps see the same
    gradients."""
    shapes = cfg["shapes"]()
    torch.manual_seed(0)
    stds = None
    if cfg.get("hetero"):
        lo, hi, seed = cfg["hetero"]
        gen = torch.Generator().manual_seed(seed)
        stds = torch.exp(torch.empty(len(shapes), dtype=torch.float64)
                         .uniform_(math.log(lo), math.log(hi), generator=gen)).tolist()
    params = []
    for s in shapes:
        p = torch.randn(s, device=device) * 0.02
        if len(s) == 1 and cfg["shapes"] is not many_small_shapes:
            p.fill_(1.0)                             # norm weights
        p.requires_grad_(True)
        p.grad_dtype = None        # allow bf16 / fp16 grads on fp32 params
        params.append(p)
    sets = []
    for k in range(grad_sets):
        torch.manual_seed(1000 + k)
        grads = []
        for i, s in enumerate(shapes):
            if stds is not None:
                # GradScaler: the backward pass produces grads scaled by 2^16 in
                # fp16, unscale_ multiplies by 2^-16 in fp32 and stores fp16 again
                g16 = (torch.randn(s, device=device) * (stds[i] * 2.0 ** 16)).half()
                grads.append((g16.float() * 2.0 ** -16).half())
                continue
            g = torch.randn(s, device=device) * cfg["std"]
            if cfg.get("outliers"):
                g = torch.where(torch.rand(s, device=device) < cfg["outliers"], g * 100.0, g)
            if cfg.get("zeros"):
                g = torch.where(torch.rand(s, device=device) < cfg["zeros"], torch.zeros_like(g), g)
            grads.append(g.to(cfg["grad"]))
        sets.append(grads)
    return params, sets


# ── CPU baseline: the oracle on a bounded sample ─────────────────────────────

def host_cores():
    """CPU cores this process may use: its affinity set, capped by the cgroup's
    CPU quota (cpu.max) when one is set."""
    n = len(os.sched_getaffinity(0))
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota, period = f.read().split()
        if quota != "max":
            n = min(n, max(1, int(quota) // int(period)))
    except (OSError, ValueError):
        pass
    return n


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def _cpu_grads(shapes, cfg, gen, n_sets=2):
    """Gradient sets for the CPU baseline, drawn as make_set draws them."""
    sets = []
    for _ in range(n_sets):
        grads = []
        for s in shapes:
            g = torch.randn(s, generator=gen) * cfg.get("std", 1e-3)
            if cfg.get("outliers"):
                g = torch.where(torch.rand(s, generator=gen) < cfg["outliers"], g * 100.0, g)
            if cfg.get("zeros"):
                g = torch.where(torch.rand(s, generator=gen) < cfg["zeros"], torch.zeros_like(g), g)
            grads.append(g.to(cfg["grad"]))
        sets.append(grads)
    return sets


def cpu_baseline(cfg_name, warmup=2, timed=5, whole=False):
    """The oracle in the reference's own math ("torch": ATen's CPU kernels)
    with every core this process may use, on the configuration's largest
    tensor (or, with ``whole``, its whole parameter set), two gradient sets
    alternating: the init step and warmup - 1 update steps untimed, then the
    median of ``timed`` update steps (time.perf_counter around each step)."""
    from oracle import luma_oracle as O

    cores = host_cores()
    torch.set_num_threads(cores)
    cfg = CONFIGS[cfg_name]
    shapes = cfg["shapes"]() if whole else [max(cfg["shapes"](), key=math.prod)]
    n = sum(math.prod(s) for s in shapes)
    gen = torch.Generator().manual_seed(1)
    params = []
    for s in shapes:
        p = torch.randn(s, generator=gen) * 0.02
        p.grad_dtype = None
        params.append(p)
    sets = _cpu_grads(shapes, cfg, gen)
    opt = O.OracleLUMA([dict(params=params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8,
                             weight_decay=0.01)], 12345, "torch")
    times = []
    t_all = time.perf_counter()
    for i in range(warmup + timed):
        for p, g in zip(params, sets[i % 2]):
            p.grad = g
        t0 = time.perf_counter()
        opt.step()
        dt = time.perf_counter() - t0
        if i >= warmup:
            times.append(dt)
        if i < 3 or (i + 1) % 10 == 0 or i + 1 == warmup + timed:
            print(f"bench: cpu baseline {cfg_name} step {i + 1}/{warmup + timed} {dt:.3f} s",
                  file=sys.stderr, flush=True)
    total = time.perf_counter() - t_all
    med = sorted(times)[len(times) // 2]
    what = (f"its whole parameter set ({len(shapes)} tensors, {n} fp32 params)" if whole else
            f"the configuration's largest tensor {tuple(shapes[0])} ({n} fp32 params)")
    return {"value": round(n / med / 1e9, 6), "unit": "Gparams/s", "cores": cores,
            "kind": "port", "ms_per_step": round(med * 1e3, 2),
            "steps": warmup + timed, "total_s": round(total, 1),
            "sample": f"oracle (the reference's PyTorch backend restated, torch CPU ops) on "
                      f"{what}, {str(cfg['grad']).replace('torch.', '')} grads, two gradient "
                      f"sets alternating; median of {timed} update steps after the init step "
                      f"and {warmup - 1} untimed update step(s); {cores} threads (all cores "
                      f"this process may use; os.cpu_count() {os.cpu_count()}); {cpu_model()}"}


# ── bytes model ───────────────────────────────────────────────────────────────

def chunk_elems(shapes):
    """The chunk length the optimizer picks for this set (luma_amd.optimizer
    _Engine.chunk_for)."""
    import numpy as np
    from luma_amd.optimizer import _Engine
    numels = np.array([math.prod(s) for s in shapes], dtype=np.int64)
    eng = types.SimpleNamespace(chunk_elems=0, small_tensors=True, medium_tensors=True)
    eng._small_limit = lambda: _Engine._small_limit(eng)
    eng._medium_limit = lambda: _Engine._medium_limit(eng)
    eng._wave_limit = lambda: _Engine._wave_limit(eng)
    return _Engine.chunk_for(eng, numels)


def pass1_bytes(cfg, n_params, gbytes):
    """Pass 1's algorithmic bytes per launch in steady state: the gradients
    and one 4-byte summary word per thread (256) of every chunk of the
    tensors that keep summaries (above the single-wavefront routes and at
    least one whole 2048-element iteration)."""
    from luma_amd import _lib as L
    shapes = cfg["shapes"]()
    c = chunk_elems(shapes)
    least = max(2048, max(L.SMALL_TENSOR, L.MEDIUM_TENSOR) + 1)
    words = sum(-(-math.prod(s) // c) * 256 for s in shapes if math.prod(s) >= least)
    return n_params * gbytes + 4 * words


# ── HBM traffic: rocprofv3 FETCH_SIZE / WRITE_SIZE, calibrated on a copy ─────

TRAFFIC_DIR = os.path.join(ROOT, "profiles")
COPY_ELEMS = 1 << 28          # float32 elements of the calibration copy (1 GiB each way)


def copy_calibration(reps):
    """A plain copy kernel of known size: y = x * 1 over 2^28 float32 (reads and
    writes 1 GiB per launch); its FETCH_SIZE / WRITE_SIZE give the counters' scale."""
    x = torch.randn(COPY_ELEMS, device="cuda")
    y = torch.empty_like(x)
    for _ in range(reps):
        torch.mul(x, 1.0, out=y)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_each_way": COPY_ELEMS * 4, "launches": reps}))


def ceilings(reps=5):
    """Achievable HBM rates of plain torch kernels on this GPU, next to which
    the step's passes are read: a copy (y = x * 1: reads and writes), and a
    read-only reduction (max), each over 2^32 float32 (16 GiB read)."""
    n = 1 << 32
    x = torch.ones(n, device="cuda")
    out = {}
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    half = x[: n // 2]
    y = torch.empty_like(half)
    for name, fn, nbytes in (("copy", lambda: torch.mul(half, 1.0, out=y), n * 4),
                             ("read_max", lambda: torch.amax(x), n * 4)):
        fn()
        torch.cuda.synchronize()
        ev[0].record()
        for _ in range(reps):
            fn()
        ev[1].record()
        torch.cuda.synchronize()
        ms = ev[0].elapsed_time(ev[1]) / reps
        out[name] = {"ms": round(ms, 3), "bytes": nbytes, "GB_s": round(nbytes / ms / 1e6, 1)}
    print(json.dumps({"hbm_ceilings": out, "peak_GB_s": HBM_PEAK / 1e9}))


def kernel_key(name):
    """A profiler's kernel name without its return type, template arguments
    and parameter list: "void luma::pass2_fast_kernel<false>(...)" ->
    "luma::pass2_fast_kernel"."""
    name = name.split("(")[0]
    if name.startswith("void "):
        name = name[5:]
    return name.split("<")[0]


def _pmc_per_dispatch(path, kernel_prefix, counter):
    import csv
    vals = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] == counter and kernel_key(r["Kernel_Name"]).startswith(kernel_prefix):
                key = int(r["Dispatch_Id"])
                vals[key] = vals.get(key, 0.0) + float(r["Counter_Value"])
    if not vals:
        raise SystemExit(f"no {counter} rows for {kernel_prefix} in {path}")
    return [vals[k] for k in sorted(vals)]          # in dispatch order


def traffic_report(config, kernel, fetch_csv, write_csv, copy_fetch_csv, copy_write_csv, out):
    """Write the HBM-traffic summary that the bench line's roofline.traffic reads."""
    cfg = CONFIGS[config]
    n_params = sum(math.prod(s) for s in cfg["shapes"]())
    gbytes = torch.tensor([], dtype=cfg["grad"]).element_size()
    algo = {"luma::pass1": pass1_bytes(cfg, n_params, gbytes),
            "luma::pass2": n_params * (gbytes + 16)}[kernel]
    copy_bytes = COPY_ELEMS * 4
    cf = _pmc_per_dispatch(copy_fetch_csv, "at::native::vectorized_elementwise_kernel", "FETCH_SIZE")
    cw = _pmc_per_dispatch(copy_write_csv, "at::native::vectorized_elementwise_kernel", "WRITE_SIZE")
    # the calibration copy is the largest elementwise launch of its run
    f_scale = copy_bytes / (max(cf) * 1024.0)
    w_scale = copy_bytes / (max(cw) * 1024.0)
    kf = _pmc_per_dispatch(fetch_csv, kernel, "FETCH_SIZE")
    kw = _pmc_per_dispatch(write_csv, kernel, "WRITE_SIZE")
    # steady-state launches: from the third on (t = 1 is the init step, and
    # t = 2 has no code summaries or seeds yet)
    kf_ss, kw_ss = (kf[2:] or kf[1:] or kf), (kw[2:] or kw[1:] or kw)
    fetch = sum(kf_ss) / len(kf_ss) * 1024.0 * f_scale
    write = sum(kw_ss) / len(kw_ss) * 1024.0 * w_scale
    lines = [
        f"# HBM traffic of {kernel} on {config} ({n_params} params, {gbytes}-byte grads)",
        "",
        "Commands (each a separate rocprofv3 run, after `python bench.py --pretouch-only`):",
        f"    rocprofv3 --pmc FETCH_SIZE --output-format csv -d <dir> -- python bench.py --config {config} --steps 3 --warmup 1 --no-cpu --no-others --no-pretouch",
        f"    rocprofv3 --pmc WRITE_SIZE --output-format csv -d <dir> -- python bench.py --config {config} --steps 3 --warmup 1 --no-cpu --no-others --no-pretouch",
        "    rocprofv3 --pmc FETCH_SIZE --output-format csv -d <dir> -- python bench.py --copy-calibration 3",
        "    rocprofv3 --pmc WRITE_SIZE --output-format csv -d <dir> -- python bench.py --copy-calibration 3",
        f"    python bench.py --traffic-report {config} {kernel} <fetch.csv> <write.csv> <copy_fetch.csv> <copy_write.csv>",
        "",
        f"copy kernel: {copy_bytes} B each way; FETCH_SIZE {max(cf):.0f} KiB -> scale {f_scale:.4f}; "
        f"WRITE_SIZE {max(cw):.0f} KiB -> scale {w_scale:.4f}",
        f"{kernel}: FETCH_SIZE per launch (KiB) {', '.join(f'{v:.0f}' for v in kf)}",
        f"{kernel}: WRITE_SIZE per launch (KiB) {', '.join(f'{v:.0f}' for v in kw)}",
        f"algorithmic bytes per launch: {algo}",
        f"calibrated fetch bytes per launch: {fetch:.0f} ({fetch / (n_params * (gbytes + 8) if kernel.endswith('2') else algo):.3f} x algorithmic reads)",
        f"calibrated write bytes per launch: {write:.0f}",
        f"traffic_bytes_per_launch: {fetch + write:.0f}",
        f"traffic_over_algorithmic: {(fetch + write) / algo:.4f}",
    ]
    if kernel == "luma::pass1":
        # what pass 1 fetched beyond its gradients and summaries, as a share
        # of the 4 code bytes per parameter it would read without them
        extra = fetch - algo
        lines.append(f"fetched beyond gradients and summaries: {extra:.0f} B = "
                     f"{100 * extra / (4 * n_params):.2f}% of the code bytes (4 B/param)")
    with open(out, "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))


def stats_report(config, trace_csv, bench_json, out):
    """Write the kernel-time summary of a `rocprofv3 --kernel-trace --stats` run of
    bench.py: per LUMA kernel, the average over every launch and over the
    steady-state launches (from the third on: t = 1 is the init step, t = 2
    has no code summaries or seeds yet), next to the bench's own HIP-event
    averages from the same run."""
    import csv
    durs = {}
    with open(trace_csv) as f:
        rows = list(csv.DictReader(f))
    for r in sorted(rows, key=lambda r: int(r["Start_Timestamp"])):
        key = kernel_key(r["Kernel_Name"])
        if key.startswith("luma::"):
            durs.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e6)
    total = sum((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e6 for r in rows)
    bench = None
    with open(bench_json) as f:
        for line in f:
            if line.startswith("{"):
                bench = json.loads(line)
    cfg = CONFIGS[config]
    n_params = sum(math.prod(s) for s in cfg["shapes"]())
    lines = [
        f"# Kernel time of the LUMA step on {config} ({n_params} params, {len(cfg['shapes']())} tensors, "
        f"{str(cfg['grad']).replace('torch.', '')} grads)",
        "",
        "Commands (MI355X, one GPU):",
        "    python bench.py --pretouch-only",
        f"    rocprofv3 --kernel-trace --stats --output-format csv -d <dir> -o kt -- python bench.py --config {config} "
        f"--steps {bench['steps']} --warmup {bench['warmup']} --no-cpu --no-others --no-pretouch > <bench.json>",
        f"    python bench.py --stats-report {config} <dir>/.../kt_kernel_trace.csv <bench.json> <out.md>",
        "",
        f"{bench['warmup'] + bench['steps']} launches of each kernel: {bench['warmup']} warm-up + "
        f"{bench['steps']} timed steps; the first is the init step (t = 1).",
        "",
        "| kernel | launches | avg ms (all) | avg ms (t >= 3) | min ms | max ms | % of GPU time | bench HIP events ms |",
        "|---|---|---|---|---|---|---|---|",
    ]
    ev = {"luma::pass1_fast_kernel": "luma_pass1", "luma::finalize_kernel": "luma_finalize",
          "luma::pass2_fast_kernel": "luma_pass2"}
    for key in sorted(durs, key=lambda k: -sum(durs[k])):
        d = durs[key]
        ss = d[2:] or d[1:] or d
        bev = bench["kernel_ms"].get(ev.get(key, ""), None)
        lines.append(f"| `{key}` | {len(d)} | {sum(d) / len(d):.3f} | {sum(ss) / len(ss):.3f} | "
                     f"{min(d):.3f} | {max(d):.3f} | {100 * sum(d) / total:.2f} | "
                     f"{'' if bev is None else f'{bev:.3f}'} |")
    lines += ["",
              "The bench's HIP-event intervals bracket each pass; the tensors of at most 256 "
              "elements (one wavefront each) are stepped inside `luma::pass1_fast_kernel` and "
              "`luma::pass2_fast_kernel`.",
              "",
              f"Step time in the same run (bench wall clock): {bench['ms_per_step']:.3f} ms; "
              f"{bench['value']} Gparams/s.",
              "Kernels not listed are torch's synthetic-data set-up outside the timed region."]
    with open(out, "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))


ISSUE_COUNTERS = ("SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_WAIT_ANY SQ_WAIT_INST_ANY SQ_ACTIVE_INST_ANY "
                  "SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_VALU2 SQ_INSTS_VALU")


def issue_report(config, kernel, pmc_csv, out):
    """Write the instruction-issue summary of a kernel from one rocprofv3 run
    of bench.py with ISSUE_COUNTERS (steady-state launches: from the third
    on).  The SQ counters are summed over the shader engines; cycle counts
    other than SQ_BUSY_CYCLES are in quad-cycles."""
    cfg = CONFIGS[config]
    n_params = sum(math.prod(s) for s in cfg["shapes"]())
    c = {}
    for name in ISSUE_COUNTERS.split():
        v = _pmc_per_dispatch(pmc_csv, kernel, name)
        v = v[2:] or v[1:] or v
        c[name] = sum(v) / len(v)
    n_se = 32                      # MI355X: 8 XCDs x 4 shader engines, 8 CUs each
    se_cycles = c["SQ_BUSY_CYCLES"] / n_se
    wave_cycles = 4.0 * c["SQ_WAVE_CYCLES"]
    lines = [
        f"# Instruction issue of {kernel} on {config} ({n_params} params)",
        "",
        "Commands (MI355X, one GPU):",
        "    python bench.py --pretouch-only",
        f"    rocprofv3 --pmc {ISSUE_COUNTERS} --output-format csv -d <dir> -- "
        f"python bench.py --config {config} --steps 3 --warmup 1 --no-cpu --no-others --no-pretouch",
        f"    python bench.py --issue-report {config} {kernel} <counter_collection.csv> <out.md>",
        "",
        f"kernel time from SQ_BUSY_CYCLES at 2.4 GHz: {se_cycles / 2.4e6:.2f} ms",
        f"VALU instructions per element: {c['SQ_INSTS_VALU'] * 64 / n_params:.1f}",
        f"VALU issue rate: {c['SQ_INSTS_VALU'] / (se_cycles * 256):.2f} wave instructions per clock per CU",
        f"quad-cycles with two VALU instructions issued, per VALU instruction: "
        f"{c['SQ_ACTIVE_INST_VALU2'] / c['SQ_INSTS_VALU']:.3f} "
        f"(so {200 * c['SQ_ACTIVE_INST_VALU2'] / c['SQ_INSTS_VALU']:.0f}% of the instructions issued in pairs)",
        f"resident waves per SIMD: {wave_cycles / (se_cycles * n_se * 32):.2f}",
        f"wave cycles waiting for an issue slot with an instruction ready (SQ_WAIT_INST_ANY): "
        f"{100 * 4 * c['SQ_WAIT_INST_ANY'] / wave_cycles:.0f}%",
        f"wave cycles waiting on a dependency or counter (SQ_WAIT_ANY): {100 * 4 * c['SQ_WAIT_ANY'] / wave_cycles:.0f}%",
        f"wave cycles issuing (SQ_ACTIVE_INST_ANY): {100 * 4 * c['SQ_ACTIVE_INST_ANY'] / wave_cycles:.0f}%",
    ]
    with open(out, "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))


def read_traffic(config, kernel):
    path = os.path.join(TRAFFIC_DIR, f"{kernel.replace('::', '_')}_{config}_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1]), os.path.relpath(path, ROOT)
    except OSError:
        pass
    return None, None


# ── main ─────────────────────────────────────────────────────────────────────

GRAD_SETS = 2            # gradient sets that alternate through every run's steps

# Run in a child process before this one touches the GPU: allocate and zero
# 90% of the free HBM in 1 GiB blocks, then exit (releasing it).
PRETOUCH_SRC = (
    "import torch\n"
    "free, _ = torch.cuda.mem_get_info()\n"
    "bufs = [torch.zeros(1 << 28, dtype=torch.float32, device='cuda')\n"
    "        for _ in range(int(free * 0.9) >> 30)]\n"
    "torch.cuda.synchronize()\n"
    "print(len(bufs))\n")


def pretouch_hbm() -> int:
    """Write most of the HBM once from a child process (see the module
    docstring); returns the GiB written.  Must run before this process
    initialises the GPU."""
    import subprocess
    r = subprocess.run([sys.executable, "-c", PRETOUCH_SRC], capture_output=True, text=True,
                       timeout=600)
    if r.returncode != 0:
        raise RuntimeError(f"bench.py: HBM pre-touch failed ({r.returncode}): {r.stderr[-2000:]}")
    return int(r.stdout.split()[-1])


# the other benchmark workloads timed by the default run (name, timed steps:
# the step counts the workloads are stated with), and their CPU baselines on
# the whole parameter set (untimed warm-up steps incl. the init step, timed)
OTHER_CONFIGS = (("single_4096", 100), ("gpt2_small", 200), ("many_small", 100))
OTHER_CPU = {"single_4096": (1, 99), "gpt2_small": (1, 10), "many_small": (1, 10)}


def run_gpu(name, steps, warmup, dev, grad_sets=GRAD_SETS):
    """Time `steps` LUMA steps of workload `name` after `warmup` untimed ones.
    The steps run back to back, as in a training loop; before each, the
    gradients switch to the next of GRAD_SETS sets (host work outside the
    timed events).  Per step: an event before step() and the four the step
    records around its kernels.  Returns the wall time per step (every
    step between two synchronisations), the mean event time per step, and
    the mean time of pass 1, finalize and pass 2."""
    from luma_amd import LUMA

    cfg = CONFIGS[name]
    params, sets = make_set(cfg, dev, grad_sets)
    n_params = sum(p.numel() for p in params)
    gbytes = torch.tensor([], dtype=cfg["grad"]).element_size()
    print(f"bench: {name} {len(params)} tensors {n_params} params", file=sys.stderr, flush=True)

    def use(i):
        for p, g in zip(params, sets[i % grad_sets]):
            p.grad = g

    opt = LUMA(params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    i = 0
    for _ in range(warmup):
        use(i)
        opt.step()
        i += 1
    torch.cuda.synchronize()
    if cfg.get("restore"):
        # resume from a checkpoint: the timed steps run on a fresh optimizer
        sd = opt.state_dict()
        opt = LUMA(params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
        opt.load_state_dict(sd)
        del sd
        use(i)
        opt.step()
        i += 1
        torch.cuda.synchronize()
    print(f"bench: {name} warmup done", file=sys.stderr, flush=True)

    # five events per timed step: before step(), then before pass 1, after
    # pass 1, after finalize, after pass 2 (recorded by the step itself)
    ev_sets = [[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in range(steps)]
    for es in ev_sets:
        for e in es:
            e.record()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for es in ev_sets:
        use(i)
        i += 1
        es[0].record()
        opt._engine.profile_events = es[1:]
        opt.step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    opt._engine.profile_events = None
    k_times = [[es[k + 1].elapsed_time(es[k + 2]) for es in ev_sets] for k in range(3)]
    ev_ms = sum(es[0].elapsed_time(es[4]) for es in ev_sets) / steps
    avg = [sum(v) / len(v) for v in k_times]
    print(f"bench: {name} kernel ms pass1 {avg[0]:.3f} finalize {avg[1]:.3f} pass2 {avg[2]:.3f}; "
          f"step {wall * 1e3 / steps:.3f} ms wall, {ev_ms:.3f} ms events",
          file=sys.stderr, flush=True)
    out = {"params": n_params, "tensors": len(params), "gbytes": gbytes,
           "wall_ms": wall * 1e3 / steps, "event_ms": ev_ms, "kernel_avg": avg}
    del opt, params, sets
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="llama3_8b", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--grad-sets", type=int, default=GRAD_SETS,
                    help="gradient sets that alternate through the steps (1: the same "
                         "gradients every step)")
    ap.add_argument("--no-others", dest="others", action="store_false",
                    help="time the headline workload only (default: also the single 4096^2 "
                         "tensor, the GPT-2-small list and the 20,000-tensor set)")
    ap.add_argument("--no-pretouch", dest="pretouch", action="store_false",
                    help="skip writing the HBM once from a child process before the run")
    ap.add_argument("--pretouch-only", action="store_true",
                    help="only write the HBM once (from a child process) and exit: run it before "
                         "a profiled bench.py --no-pretouch")
    ap.add_argument("--ceilings", action="store_true",
                    help="time torch's copy and max over 16 GiB (achievable HBM rates)")
    ap.add_argument("--copy-calibration", type=int, metavar="REPS",
                    help="only run the copy kernel used to scale the HBM counters")
    ap.add_argument("--traffic-report", nargs=7,
                    metavar=("CONFIG", "KERNEL", "FETCH_CSV", "WRITE_CSV", "COPY_FETCH_CSV",
                             "COPY_WRITE_CSV", "OUT"),
                    help="summarise rocprofv3 FETCH_SIZE/WRITE_SIZE runs into OUT")
    ap.add_argument("--issue-report", nargs=4, metavar=("CONFIG", "KERNEL", "PMC_CSV", "OUT"),
                    help="summarise a rocprofv3 --pmc run with the SQ issue counters")
    ap.add_argument("--stats-report", nargs=4, metavar=("CONFIG", "TRACE_CSV", "BENCH_JSON", "OUT"),
                    help="summarise a rocprofv3 --kernel-trace --stats run of bench.py into OUT")
    args = ap.parse_args()
    if args.pretouch_only:
        print(f"bench.py: wrote {pretouch_hbm()} GiB of HBM once", file=sys.stderr)
        return
    if args.traffic_report:
        traffic_report(*args.traffic_report)
        return
    if args.stats_report:
        stats_report(*args.stats_report)
        return
    if args.issue_report:
        issue_report(*args.issue_report)
        return
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.ceilings:
        ceilings()
        return
    if args.gpus != 1:
        print(f"bench.py: measures one GPU only (--gpus {args.gpus} requested); "
              "the LUMA step is rank-local and shards with no exchange", file=sys.stderr)
        sys.exit(2)

    t_start = time.perf_counter()
    touched = pretouch_hbm() if args.pretouch else 0
    dev = torch.device("cuda:0")
    head = run_gpu(args.config, args.steps, args.warmup, dev, args.grad_sets)
    cfg = CONFIGS[args.config]
    n_params, gbytes, avg, ms = head["params"], head["gbytes"], head["kernel_avg"], head["wall_ms"]
    pass_bytes = [pass1_bytes(cfg, n_params, gbytes), 0, n_params * (gbytes + 16)]
    dom = 0 if avg[0] > avg[2] else 2
    achieved = pass_bytes[dom] / (avg[dom] * 1e-3)
    step_bytes = pass_bytes[0] + pass_bytes[2]
    step_gbps = step_bytes / (ms * 1e-3)
    ref_gbps = n_params * (2 * gbytes + 20) / (ms * 1e-3)
    names = ["luma_pass1", "luma_finalize", "luma_pass2"]
    traffic, traffic_src = read_traffic(args.config, "luma::" + names[dom][5:])

    others = {}
    if args.others and args.config == "llama3_8b":
        # the other benchmark workloads at their stated step counts, after the
        # headline's memory is released
        for name, steps in OTHER_CONFIGS:
            r = run_gpu(name, steps, 3, dev)
            o = CONFIGS[name]
            ref_bytes = r["params"] * (2 * r["gbytes"] + 20)
            others[name] = {
                "workload": o["desc"], "params": r["params"], "tensors": r["tensors"],
                "steps": steps, "warmup": 3,
                "ms_per_step": round(r["event_ms"], 4),
                "wall_ms_per_step": round(r["wall_ms"], 4),
                "gparams_s": round(r["params"] / (r["event_ms"] * 1e-3) / 1e9, 2),
                "reference_model_gbps": round(ref_bytes / (r["event_ms"] * 1e-3) / 1e9, 1),
                "reference_model_frac": round(ref_bytes / (r["event_ms"] * 1e-3) / HBM_PEAK, 4),
                "kernel_ms": {names[i]: round(r["kernel_avg"][i], 4) for i in range(3)},
            }
    cpu = None if args.no_cpu else cpu_baseline(args.config)
    if not args.no_cpu:
        for name, (warm, timed) in OTHER_CPU.items():
            if name in others:
                others[name]["cpu_baseline"] = cpu_baseline(name, warm, timed, whole=True)
    out = {
        "metric": METRIC,
        "value": round(n_params / (ms * 1e-3) / 1e9, 3),
        "unit": "Gparams/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": cfg["desc"], "params": n_params, "tensors": head["tensors"],
                   "grad_dtype": str(cfg["grad"]).replace("torch.", ""),
                   "grad_sets": args.grad_sets, "hbm_pretouch_gib": touched,
                   "bytes_per_param": round(step_bytes / n_params, 3),
                   "reference_bytes_per_param": 2 * gbytes + 20},
        "step_hbm_gbps": round(step_gbps / 1e9, 1),
        "step_hbm_frac": round(step_gbps / HBM_PEAK, 4),
        "step_reference_model_gbps": round(ref_gbps / 1e9, 1),
        "step_reference_model_frac": round(ref_gbps / HBM_PEAK, 4),
        "kernel_ms": {names[i]: round(avg[i], 4) for i in range(3)},
        "roofline": {"bound": "hbm", "kernel": names[dom],
                     "achieved": round(achieved / 1e9, 1), "peak": HBM_PEAK / 1e9,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK, 4),
                     "traffic": None if traffic is None else round(traffic),
                     "traffic_source": traffic_src,
                     "algorithmic_bytes": pass_bytes[dom]},
        "cpu_baseline": cpu,
    }
    if others:
        out["other_configs"] = others
    out["bench_wall_s"] = round(time.perf_counter() - t_start, 1)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
