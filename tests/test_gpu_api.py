"""HIP LUMA behaviour on the GPU, mirroring the reference's own test suites
(tests/test_basic.py, test_determinism.py, test_state_dict.py,
test_correctness.py, test_convergence.py, test_mixed_precision.py)."""

import math
import random

import pytest
import torch
import torch.nn as nn

from luma_amd import LUMA
from oracle import luma_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def seed_all(seed=42):
    random.seed(seed)
    torch.manual_seed(seed)
    torch.cuda.manual_seed_all(seed)


def _fixed_grad_steps(opt, x, g, n):
    for _ in range(n):
        opt.zero_grad()
        x.grad = g.clone()
        opt.step()


def _quadratic(d):
    a = torch.rand(d, device=DEV) + 0.5
    b = torch.randn(d, device=DEV)
    return lambda x: 0.5 * (a * (x - b).square()).sum()


def _train(opt, x, loss_fn, n):
    for _ in range(n):
        opt.zero_grad()
        loss = loss_fn(x)
        loss.backward()
        opt.step()
    return loss.item()


# ── stepping / edge cases (test_basic.py) ────────────────────────────────────

def test_single_and_multiple_steps():
    model = nn.Linear(8, 4).to(DEV)
    opt = LUMA(model.parameters(), lr=1e-3)
    for _ in range(10):
        model(torch.randn(2, 8, device=DEV)).sum().backward()
        opt.step()
        opt.zero_grad()
    for p in model.parameters():
        assert p.isfinite().all()
        s = opt.state[p]
        assert s["Q_m"].dtype == torch.int16 and s["Q_w"].dtype == torch.int16
        assert s["Q_m"].shape == p.shape and s["Q_w"].shape == p.shape
        assert s["Q_m"].device.type == "cuda"
        assert s["step"] == 10


def test_lr_zero_no_update():
    model = nn.Linear(8, 4).to(DEV)
    opt = LUMA(model.parameters(), lr=0.0, weight_decay=0.0)
    before = [p.data.clone() for p in model.parameters()]
    model(torch.randn(2, 8, device=DEV)).sum().backward()
    opt.step()
    for p, b in zip(model.parameters(), before):
        assert torch.equal(p.data, b)


def test_scalar_parameter():
    x = torch.tensor(5.0, device=DEV, requires_grad=True)
    opt = LUMA([x], lr=1e-2)
    for _ in range(5):
        opt.zero_grad()
        (x ** 2).backward()
        opt.step()
    assert x.item() < 5.0


def test_closure_returns_loss():
    model = nn.Linear(4, 2).to(DEV)
    opt = LUMA(model.parameters())
    x = torch.randn(2, 4, device=DEV)

    def closure():
        opt.zero_grad()
        loss = model(x).sum()
        loss.backward()
        return loss
    assert torch.is_tensor(opt.step(closure))


def test_none_grad_keeps_param_id_counting():
    """A param without grad is skipped but still counted (optimizer.py:428-431)."""
    a = torch.zeros(4, device=DEV, requires_grad=True)
    b = torch.zeros(4, device=DEV, requires_grad=True)
    opt = LUMA([a, b])
    b.grad = torch.ones(4, device=DEV)
    opt.step()
    assert len(opt.state[a]) == 0
    assert opt.state[b]["param_id"] == 1 and opt.state[b]["step"] == 1


def test_zero_grad_modes():
    for set_to_none in (False, True):
        model = nn.Linear(8, 4).to(DEV)
        opt = LUMA(model.parameters(), lr=1e-3)
        model(torch.randn(2, 8, device=DEV)).sum().backward()
        opt.step()
        opt.zero_grad(set_to_none=set_to_none)
        model(torch.randn(2, 8, device=DEV)).sum().backward()
        opt.step()
        assert all(p.isfinite().all() for p in model.parameters())


def test_4_bytes_per_param():
    model = nn.Linear(256, 256, bias=False).to(DEV)
    opt = LUMA(model.parameters())
    model(torch.randn(1, 256, device=DEV)).sum().backward()
    opt.step()
    for p in model.parameters():
        s = opt.state[p]
        assert s["Q_m"].element_size() * s["Q_m"].numel() + \
            s["Q_w"].element_size() * s["Q_w"].numel() == 4 * p.numel()


def test_noncontiguous_grad_accepted():
    p = torch.randn(8, 8, device=DEV, requires_grad=True)
    opt = LUMA([p])
    p.grad = torch.randn(8, 8, device=DEV).t()
    opt.step()
    assert p.isfinite().all()


# ── determinism (test_determinism.py) ────────────────────────────────────────

def _run_fixed(d=4099, steps=20, seed=42, pollute=None):
    seed_all(0)
    x0 = torch.randn(d, device=DEV)
    g = torch.randn(d, device=DEV) * 1e-2
    seed_all(seed)
    x = x0.clone().requires_grad_(True)
    opt = LUMA([x], lr=1e-2, weight_decay=0.01)
    for i in range(steps):
        opt.zero_grad()
        x.grad = g.clone()
        if pollute:
            pollute(i)
        opt.step()
    s = opt.state[x]
    return x.detach().clone(), s["Q_m"].clone(), s["Q_w"].clone()


def test_same_seed_bitwise_identical():
    a, b = _run_fixed(), _run_fixed()
    for u, v in zip(a, b):
        assert torch.equal(u, v)


def test_global_rng_isolation_and_ddp_ranks():
    clean = _run_fixed()

    def pollute(i):
        torch.rand(500 + 37 * i, device=DEV)
        torch.rand(11)
        random.random()
    dirty = _run_fixed(pollute=pollute)
    for u, v in zip(clean, dirty):
        assert torch.equal(u, v)


def test_different_seed_different_quant():
    a = _run_fixed(steps=2, seed=100)
    b = _run_fixed(steps=2, seed=200)
    assert not torch.equal(a[1], b[1])


def test_determinism_survives_checkpoint():
    seed_all(0)
    x0 = torch.randn(3000, device=DEV)
    g = torch.randn(3000, device=DEV)
    seed_all(42)
    x_ref = x0.clone().requires_grad_(True)
    opt_ref = LUMA([x_ref], lr=1e-2)
    _fixed_grad_steps(opt_ref, x_ref, g, 30)
    seed_all(42)
    x_a = x0.clone().requires_grad_(True)
    opt_a = LUMA([x_a], lr=1e-2)
    _fixed_grad_steps(opt_a, x_a, g, 10)
    sd = opt_a.state_dict()
    x_b = x_a.detach().clone().requires_grad_(True)
    opt_b = LUMA([x_b], lr=1e-2)
    opt_b.load_state_dict(sd)
    _fixed_grad_steps(opt_b, x_b, g, 20)
    assert torch.equal(x_ref.data, x_b.data)


def test_multi_param_determinism():
    def run():
        seed_all(42)
        model = nn.Sequential(nn.Linear(32, 64), nn.ReLU(), nn.Linear(64, 16)).to(DEV)
        opt = LUMA(model.parameters(), lr=1e-3, weight_decay=0.01)
        x = torch.randn(4, 32, device=DEV)
        for _ in range(30):
            opt.zero_grad()
            model(x).sum().backward()
            opt.step()
        return [p.data.clone() for p in model.parameters()]
    for a, b in zip(run(), run()):
        assert torch.equal(a, b)


# ── state dict (test_state_dict.py) ──────────────────────────────────────────

def test_state_dict_keys_and_round_trip():
    model = nn.Linear(8, 4).to(DEV)
    opt = LUMA(model.parameters())
    model(torch.randn(2, 8, device=DEV)).sum().backward()
    opt.step()
    sd = opt.state_dict()
    assert "_base_seed" in sd
    for s in sd["state"].values():
        assert set(s) == {"step", "param_id", "Q_m", "Q_w", "S_m", "S_v"}
        assert isinstance(s["S_m"], float) and s["S_m"] >= 1e-9


def test_state_dict_before_step():
    model = nn.Linear(8, 4).to(DEV)
    opt = LUMA(model.parameters())
    sd = opt.state_dict()
    assert sd["state"] == {} and len(sd["param_groups"]) == 1
    model2 = nn.Linear(8, 4).to(DEV)
    opt2 = LUMA(model2.parameters())
    opt2.load_state_dict(sd)
    model2(torch.randn(1, 8, device=DEV)).sum().backward()
    opt2.step()


def test_round_trip_single_param_bitwise():
    d = 32
    loss_fn = _quadratic(d)
    kw = dict(lr=1e-2, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    seed_all(0)
    x_ref = torch.randn(d, device=DEV, requires_grad=True)
    opt_ref = LUMA([x_ref], **kw)
    _train(opt_ref, x_ref, loss_fn, 10)
    seed_all(0)
    x = torch.randn(d, device=DEV, requires_grad=True)
    opt = LUMA([x], **kw)
    _train(opt, x, loss_fn, 5)
    for _ in range(2):
        sd = opt.state_dict()
        x = x.data.clone().requires_grad_(True)
        opt = LUMA([x], **kw)
        opt.load_state_dict(sd)
    _train(opt, x, loss_fn, 5)
    assert torch.equal(x.data, x_ref.data)


def test_export_matches_cr_oracle_and_loads_into_adamw():
    torch.manual_seed(3)
    shapes = [(16, 8), (8,)]
    cpu = [torch.randn(s) * 0.05 for s in shapes]
    dev = [p.clone().cuda().requires_grad_(True) for p in cpu]
    base = 987654321
    oracle = O.OracleLUMA([dict(params=cpu, lr=1e-3, betas=(0.9, 0.999), eps=1e-8,
                                weight_decay=0.01)], base, "cr")
    opt = LUMA(dev, lr=1e-3)
    opt._base_seed = base
    for t in range(1, 6):
        grads = [torch.randn(s) * 1e-2 for s in shapes]
        for p, g in zip(cpu, grads):
            p.grad = g
        oracle.step()
        for i, (p, g) in enumerate(zip(dev, grads)):
            p.grad = g.cuda()
        opt.inject_noise({p: tuple(u.cuda() for u in oracle.last_draws[i])
                          for i, p in enumerate(dev)})
        opt.step()
    ex = opt.export_adamw_state()
    ref = oracle.export_adamw_state()
    for idx in ref["state"]:
        assert ex["state"][idx]["step"].item() == 5.0
        assert torch.equal(ex["state"][idx]["exp_avg"].cpu(), ref["state"][idx]["exp_avg"])
        assert torch.equal(ex["state"][idx]["exp_avg_sq"].cpu(), ref["state"][idx]["exp_avg_sq"])
    adamw = torch.optim.AdamW(dev, lr=1e-3)
    adamw.load_state_dict(ex)
    for p in dev:
        p.grad = torch.randn_like(p)
    adamw.step()
    assert all(p.isfinite().all() for p in dev)


def test_import_matches_cr_oracle():
    torch.manual_seed(5)
    shapes = [(32, 16), (16,)]
    pa = [torch.nn.Parameter(torch.randn(s, device=DEV) * 0.05) for s in shapes]
    adamw = torch.optim.AdamW(pa, lr=1e-3, weight_decay=0.01)
    for _ in range(10):
        for p in pa:
            p.grad = torch.randn_like(p) * 1e-2
        adamw.step()
    asd = adamw.state_dict()
    luma = LUMA(pa, lr=1e-3, weight_decay=0.01)
    cpu_params = [torch.zeros(s) for s in shapes]
    oracle = O.OracleLUMA([dict(params=cpu_params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8,
                                weight_decay=0.01)], luma._base_seed, "cr")
    cpu_sd = {"state": {i: {k: (v.cpu() if torch.is_tensor(v) else v) for k, v in s.items()}
                        for i, s in asd["state"].items()}}
    oracle.import_adamw_state(cpu_sd)
    luma.inject_noise({p: tuple(u.cuda() for u in oracle.last_draws[i]) for i, p in enumerate(pa)})
    luma.import_adamw_state(asd)
    sd = luma.state_dict()
    for i, p in enumerate(cpu_params):
        o = oracle.state[id(p)]
        s = sd["state"][i]
        assert s["step"] == 10 and s["param_id"] == i
        assert s["S_m"] == o["S_m"] and s["S_v"] == o["S_v"]
        assert torch.equal(s["Q_m"].cpu(), o["Q_m"]) and torch.equal(s["Q_w"].cpu(), o["Q_w"])
    # round trip error bound (test_state_dict.py:522-561)
    ex = luma.export_adamw_state()
    for idx, s in asd["state"].items():
        for k in ("exp_avg", "exp_avg_sq"):
            orig, back = s[k].float(), ex["state"][idx][k]
            scale = float(orig.abs().max())
            assert float((back - orig).abs().max()) / scale < 0.002


# ── LogSR unbiasedness with native Philox (10^7 draws) ───────────────────────

@pytest.mark.parametrize("frac_pos", [0.1, 0.37, 0.5, 0.83])
def test_philox_logsr_unbiased_1e7(frac_pos):
    """Quantise 10^7 copies of one value with native Philox noise; the round-up
    frequency must match the kernel's own p* (z < 5) and the mean decode must
    equal the linear value within the float32 representation bound."""
    n = 10_000_000
    S = 1.0
    dm = math.log1p(S) / O.K_M
    zm = math.expm1(dm)
    y = 20000.0 + frac_pos
    x = float(torch.tensor(math.expm1(y * dm), dtype=torch.float32))
    m = torch.full((n,), x, device=DEV)
    m[0] = S                      # fixes S_m = 1.0
    v = torch.full((n,), 1e-6, device=DEV)
    v[0] = 1e-2
    p = torch.nn.Parameter(torch.zeros(n, device=DEV))
    luma = LUMA([p])
    luma.import_adamw_state({"state": {0: {"step": 1, "exp_avg": m, "exp_avg_sq": v}}})
    q = luma.state[p]["Q_m"][1:].to(torch.int64)
    # the kernel's y and p* for this element, in float32 as the oracle forms them
    dm32 = torch.tensor([dm], dtype=torch.float32)
    yk = float((torch.log1p(torch.tensor([x]).double()).float() / dm32).item())
    k = math.floor(yk)
    assert int(q.min()) >= k and int(q.max()) <= k + 1
    f_hat = float((q == k + 1).double().mean())
    fr = torch.tensor([yk - k], dtype=torch.float32)
    p_star = float((torch.expm1((fr * dm32).double()).float()
                    / torch.tensor([zm], dtype=torch.float32)).item())
    sigma = math.sqrt(p_star * (1 - p_star) / (n - 1))
    assert abs(f_hat - p_star) < 5 * sigma, (f_hat, p_star, sigma)
    ex = luma.export_adamw_state()["state"][0]["exp_avg"][1:].double()
    mean = float(ex.mean())
    bin_w = math.expm1((k + 1) * dm) - math.expm1(k * dm)
    assert abs(mean - x) < 5 * sigma * bin_w + 4e-7 * x, (mean, x)


# ── convergence / tracking (test_correctness.py, test_convergence.py) ────────

def test_tracks_adamw_on_quadratic():
    d = 32
    a = torch.rand(d, device=DEV) + 0.5
    b = torch.randn(d, device=DEV)
    x_a = torch.randn(d, device=DEV, requires_grad=True)
    x_l = x_a.data.clone().requires_grad_(True)
    opt_a = torch.optim.AdamW([x_a], lr=1e-2, weight_decay=0.0)
    opt_l = LUMA([x_l], lr=1e-2, weight_decay=0.0)
    loss_fn = lambda x: 0.5 * (a * (x - b).square()).sum()  # noqa: E731
    init = loss_fn(x_a).item()
    la, ll = [], []
    for _ in range(300):
        for opt, x, losses in ((opt_a, x_a, la), (opt_l, x_l, ll)):
            opt.zero_grad()
            loss = loss_fn(x)
            losses.append(loss.item())
            loss.backward()
            opt.step()
    assert ll[-1] < init * 0.035
    assert ll[-1] < la[-1] * 1.015 + 1e-7
    for s in (49, 149, 299):
        assert abs(ll[s] - la[s]) / max(la[s], 1e-8) < 0.015
    assert (x_l - x_a).norm() < 0.01 * x_a.norm() + 1e-6


def test_rosenbrock_and_mlp_converge():
    xy = torch.tensor([-1.0, 1.0], device=DEV, requires_grad=True)
    opt = LUMA([xy], lr=1e-3, weight_decay=0.0)
    for _ in range(3000):
        opt.zero_grad()
        x, y = xy[0], xy[1]
        ((1 - x) ** 2 + 100 * (y - x ** 2) ** 2).backward()
        opt.step()
    assert abs(xy[0].item() - 1) < 0.5 and abs(xy[1].item() - 1) < 0.5
    X = torch.randn(200, 10, device=DEV)
    Y = X @ torch.randn(10, 1, device=DEV) + 0.1 * torch.randn(200, 1, device=DEV)
    model = nn.Sequential(nn.Linear(10, 32), nn.ReLU(), nn.Linear(32, 1)).to(DEV)
    opt = LUMA([{"params": model[0].parameters(), "lr": 2e-3},
                {"params": model[2].parameters(), "lr": 1e-3}], weight_decay=0.01)
    init = None
    for _ in range(300):
        opt.zero_grad()
        loss = nn.functional.mse_loss(model(X), Y)
        init = init or loss.item()
        loss.backward()
        opt.step()
    assert loss.item() < init * 0.1


# ── mixed precision (test_mixed_precision.py) ────────────────────────────────

@pytest.mark.parametrize("amp_dtype", [torch.float16, torch.bfloat16])
def test_autocast_converges(amp_dtype):
    model = nn.Sequential(nn.Linear(16, 32), nn.ReLU(), nn.Linear(32, 1)).to(DEV)
    opt = LUMA(model.parameters(), lr=1e-3, weight_decay=0.01)
    X = torch.randn(100, 16, device=DEV)
    Y = torch.randn(100, 1, device=DEV)
    init = None
    for _ in range(200):
        opt.zero_grad()
        with torch.autocast("cuda", dtype=amp_dtype):
            pred = model(X)
        loss = nn.functional.mse_loss(pred.float(), Y)
        init = init or loss.item()
        loss.backward()
        opt.step()
    assert loss.item() < init * 0.5
    assert all(p.dtype == torch.float32 and p.isfinite().all() for p in model.parameters())


def test_grad_scaler_fp16():
    model = nn.Sequential(nn.Linear(16, 32), nn.ReLU(), nn.Linear(32, 1)).to(DEV)
    opt = LUMA(model.parameters(), lr=1e-3, weight_decay=0.01)
    scaler = torch.amp.GradScaler()
    X = torch.randn(100, 16, device=DEV)
    Y = torch.randn(100, 1, device=DEV)
    init = None
    for _ in range(200):
        opt.zero_grad()
        with torch.autocast("cuda", dtype=torch.float16):
            pred = model(X)
        loss = nn.functional.mse_loss(pred.float(), Y)
        init = init or loss.item()
        scaler.scale(loss).backward()
        scaler.step(opt)
        scaler.update()
    assert loss.item() < init * 0.5


# ── parameters replaced between steps (the re-used step plan re-checks them) ─

def test_replaced_parameter_storage():
    torch.manual_seed(0)
    model = nn.Linear(64, 32).to(DEV)
    opt = LUMA(model.parameters(), lr=1e-3)
    x = torch.randn(4, 64, device=DEV)
    for _ in range(2):
        opt.zero_grad()
        model(x).sum().backward()
        opt.step()
    torch.cuda.synchronize()
    # same layout, new storage: the step updates the new storage
    new_w = model.weight.detach().clone()
    model.weight.data = new_w
    before = new_w.clone()
    opt.zero_grad()
    model(x).sum().backward()
    opt.step()
    torch.cuda.synchronize()
    assert model.weight.data_ptr() == new_w.data_ptr() and not torch.equal(new_w, before)
    # reduced precision: rejected, nothing launched
    model.weight.data = model.weight.detach().half()
    opt.zero_grad()
    model.weight.grad = torch.zeros_like(model.weight)
    with pytest.raises(ValueError, match="float32"):
        opt.step()
    # a resized parameter no longer matches its codes: rejected
    model.weight.data = torch.zeros(32, 65, device=DEV)
    model.weight.grad = torch.zeros_like(model.weight)
    with pytest.raises(ValueError, match="does not match"):
        opt.step()
