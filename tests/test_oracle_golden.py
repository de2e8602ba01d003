"""Pin the CPU oracle to the reference: golden vectors and closed forms.

The golden vectors were written by ``tests/golden/make_golden.py`` running
the reference's PyTorch backend; the oracle in ``"torch"`` math mode must
reproduce them bit for bit (functional.py:183-298, optimizer.py:413-524).
"""

import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import luma_oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")


@pytest.fixture(scope="module")
def golden():
    arrays = np.load(os.path.join(GOLD, "luma_golden.npz"), allow_pickle=False)
    with open(os.path.join(GOLD, "luma_golden.json")) as f:
        meta = json.load(f)
    return arrays, meta


def _t(arr, dtype_name=None):
    t = torch.from_numpy(np.array(arr))
    if dtype_name == "bfloat16":
        return t.view(torch.bfloat16)
    return t


@pytest.fixture(autouse=True)
def _one_thread():
    n = torch.get_num_threads()
    torch.set_num_threads(1)
    yield
    torch.set_num_threads(n)


# ── functional-level vectors ─────────────────────────────────────────────────

CASES = ["n1_f32", "n127_bf16", "n4096_f16", "n65543_f32", "zeros_f32",
         "outlier_bf16", "hyper2_f32"]


@pytest.mark.parametrize("case", CASES)
def test_oracle_matches_reference_steps(golden, case):
    arrays, meta = golden
    m = meta["functional"][case]
    param = _t(arrays[f"f/{case}/param0"]).clone()
    Q_m = Q_w = None
    S_m = S_v = None
    for rec in m["records"]:
        t = rec["t"]
        grad = _t(arrays[f"f/{case}/grad{t}"], m["grad_dtype"])
        seed = O.make_step_seed(m["base_seed"], t, m["param_id"])
        assert seed == rec["seed"]
        draw = O.generator_draw(seed)
        if t == 1:
            Q_m, Q_w, S_m, S_v = O.init_step(param, grad, m["beta1"], m["beta2"], m["eps"],
                                             m["lr"], m["weight_decay"], draw, "torch")
        else:
            S_m, S_v = O.update_step(param, grad, Q_m, Q_w, S_m, S_v, t, m["beta1"],
                                     m["beta2"], m["eps"], m["lr"], m["weight_decay"],
                                     draw, "torch")
        assert S_m == rec["S_m"] and S_v == rec["S_v"], (t, S_m, rec["S_m"], S_v, rec["S_v"])
        assert np.array_equal(Q_m.numpy(), arrays[f"f/{case}/Q_m{t}"]), f"Q_m step {t}"
        assert np.array_equal(Q_w.numpy(), arrays[f"f/{case}/Q_w{t}"]), f"Q_w step {t}"
        assert np.array_equal(param.numpy(), arrays[f"f/{case}/param{t}"]), f"param step {t}"


# ── optimizer-level vectors ──────────────────────────────────────────────────

def _oracle_from_golden(arrays, meta):
    om = meta["optimizer"]
    params = [_t(arrays[f"o/param0_{i}"]).clone() for i in range(len(om["shapes"]))]
    groups = [
        {"params": params[:2], "lr": 2e-3, "betas": (0.9, 0.999), "eps": 1e-8,
         "weight_decay": 0.05},
        {"params": params[2:], "lr": 5e-4, "betas": (0.85, 0.99), "eps": 1e-8,
         "weight_decay": 0.05},
    ]
    return params, O.OracleLUMA(groups, om["base_seed"], "torch")


def test_oracle_optimizer_trajectory(golden):
    arrays, meta = golden
    om = meta["optimizer"]
    params, opt = _oracle_from_golden(arrays, meta)
    for t, sm in enumerate(om["steps"], start=1):
        for i, p in enumerate(params):
            p.grad = None if i in sm["skipped"] else _t(arrays[f"o/grad{t}_{i}"])
        opt.step()
        for i, p in enumerate(params):
            assert np.array_equal(p.numpy(), arrays[f"o/param{t}_{i}"]), (t, i)
            st = opt.state.get(id(p))
            if str(i) in sm["state"]:
                ref = sm["state"][str(i)]
                assert st["step"] == ref["step"] and st["param_id"] == ref["param_id"]
                assert st["S_m"] == ref["S_m"] and st["S_v"] == ref["S_v"]
                assert np.array_equal(st["Q_m"].numpy(), arrays[f"o/Q_m{t}_{i}"])
                assert np.array_equal(st["Q_w"].numpy(), arrays[f"o/Q_w{t}_{i}"])
            else:
                assert not st


def test_oracle_export_matches_reference(golden):
    arrays, meta = golden
    om = meta["optimizer"]
    params, opt = _oracle_from_golden(arrays, meta)
    for t, sm in enumerate(om["steps"], start=1):
        for i, p in enumerate(params):
            p.grad = None if i in sm["skipped"] else _t(arrays[f"o/grad{t}_{i}"])
        opt.step()
    ex = opt.export_adamw_state()
    for idx, s in ex["state"].items():
        assert float(s["step"].item()) == om["export"]["steps"][str(idx)]
        assert np.array_equal(s["exp_avg"].numpy(), arrays[f"o/export_exp_avg_{idx}"])
        assert np.array_equal(s["exp_avg_sq"].numpy(), arrays[f"o/export_exp_avg_sq_{idx}"])
    assert [g["params"] for g in ex["param_groups"]] == \
        [g["params"] for g in om["export"]["param_groups"]]


def test_oracle_import_matches_reference(golden):
    arrays, meta = golden
    om = meta["optimizer"]
    imp = om["import"]
    params = [torch.zeros(*s) for s in om["shapes"]]
    groups = [{"params": params, "lr": 1e-3, "betas": (0.9, 0.999), "eps": 1e-8,
               "weight_decay": 0.01}]
    opt = O.OracleLUMA(groups, imp["base_seed"], "torch")
    sd = {"state": {i: {"step": torch.tensor(3.0),
                        "exp_avg": _t(arrays[f"o/adamw_exp_avg_{i}"]),
                        "exp_avg_sq": _t(arrays[f"o/adamw_exp_avg_sq_{i}"])}
                    for i in range(len(params))}}
    opt.import_adamw_state(sd)
    for i, p in enumerate(params):
        st = opt.state[id(p)]
        ref = imp["state"][str(i)]
        assert st["step"] == ref["step"] and st["param_id"] == ref["param_id"]
        assert st["S_m"] == ref["S_m"] and st["S_v"] == ref["S_v"]
        assert np.array_equal(st["Q_m"].numpy(), arrays[f"o/import_Q_m_{i}"])
        assert np.array_equal(st["Q_w"].numpy(), arrays[f"o/import_Q_w_{i}"])


def test_base_seed_draw_matches_reference(golden):
    """optimizer.py:94-96: the seed is one int64 draw from the global generator."""
    _, meta = golden
    torch.manual_seed(42)
    s = int(torch.randint(-(2**63), 2**63 - 1, (1,), dtype=torch.int64).item())
    assert s == meta["optimizer"]["base_seed"]


# ── closed forms and special cases ───────────────────────────────────────────

@pytest.mark.parametrize("val", [0, 1, 32767, 32768, 65535])
def test_uint16_roundtrip(val):
    t = torch.tensor([val], dtype=torch.int32)
    assert O.decode_uint16(O.encode_uint16(t)).item() == float(val)


def test_precompute_closed_form():
    S_m, S_v, eps = 2.5, 4.0, 1e-8
    w_min, dm, zm, dw, zw = O.precompute(S_m, S_v, eps)
    assert w_min == 1.0 / (2.0 + eps)
    assert dm == math.log1p(2.5) / 32767
    assert zm == math.expm1(dm)
    assert dw == math.log((2.0 + eps) / eps) / 65535
    assert zw == math.expm1(dw)
    # S_v = 0: ratio == 1 -> delta_w = 0, z_w = 1 (functional.py:86-90)
    w_min, _, _, dw, zw = O.precompute(1.0, 0.0, eps)
    assert w_min == 1.0 / eps and dw == 0.0 and zw == 1.0


def test_step_seed_closed_form():
    assert O.make_step_seed(0, 1, 0) == 1 << 32
    assert O.make_step_seed(0, 3, 5) == (3 << 32) | 10
    b = -1234567890123
    assert O.make_step_seed(b, 2, 7) == ((2 << 32) | 14) ^ b


@pytest.mark.parametrize("mode", ["torch", "cr"])
def test_decode_known_answers(mode):
    # Q = 0 -> 0 ; Q = K_M -> S_m ; sign symmetry (test_correctness.py:109-140)
    S_m = 2.5
    dm = math.log1p(S_m) / O.K_M
    q = torch.tensor([0, O.K_M, -O.K_M, 42, -42], dtype=torch.int16)
    m = O.decode_momentum(q, dm, mode)
    assert m[0].item() == 0.0
    assert m[1].item() == pytest.approx(S_m, rel=1e-5)
    assert m[2].item() == -m[1].item() and m[3].item() == -m[4].item()
    # Q_w = 0 -> w_min ; Q_w = K_W -> 1/eps (test_correctness.py:143-159)
    w_min, _, _, dw, _ = O.precompute(1.0, 1.0, 1e-8)
    qw = O.encode_uint16(torch.tensor([0, O.K_W], dtype=torch.int32))
    w = O.decode_preconditioner(qw, w_min, dw, mode)
    assert w[0].item() == pytest.approx(w_min, rel=1e-6)
    assert w[1].item() == pytest.approx(1e8, rel=1e-3)


def test_zero_variance_quantises_to_zero():
    """S_v = 0 -> delta_w = 0 -> Q_w == 0 and decode gives 1/eps exactly."""
    eps = 1e-8
    w_min, _, _, dw, zw = O.precompute(1.0, 0.0, eps)
    q = O.quantize_preconditioner(torch.zeros(16), eps, w_min, dw, zw, torch.rand(16))
    assert torch.equal(q, torch.zeros(16, dtype=torch.int16))
    assert torch.all(O.decode_preconditioner(q, w_min, dw) == np.float32(1.0 / eps))


@pytest.mark.parametrize("mode", ["torch", "cr"])
def test_log_sr_extreme_uniforms(mode):
    """u = 0 rounds every fractional y up; u -> 1- rounds down (functional.py:62-67)."""
    dm = math.log1p(1.0) / O.K_M
    zm = math.expm1(dm)
    y = torch.tensor([0.25, 10.5, 100.999, 7.0])
    up = O.log_sr(y, dm, zm, torch.zeros(4), O.K_M, mode)
    dn = O.log_sr(y, dm, zm, torch.full((4,), 1.0 - 2**-24), O.K_M, mode)
    assert up.tolist() == [1.0, 11.0, 101.0, 7.0]
    assert dn.tolist() == [0.0, 10.0, 100.0, 7.0]


def test_log_sr_unbiased_brute_force():
    """E[decode(q)] equals the linear value, checked exactly in float64 from (k, p*).

    For y = k + f the two outcomes decode to expm1(k*d) and expm1((k+1)*d); with
    p* = expm1(f*d)/expm1(d) the mean is expm1(y*d) (functional.py:38-67).
    """
    d = math.log1p(0.5) / O.K_M
    z = math.expm1(d)
    for y in [0.3, 17.25, 1234.875, 32766.5]:
        k = math.floor(y)
        p = math.expm1((y - k) * d) / z
        mean = (1 - p) * math.expm1(k * d) + p * math.expm1((k + 1) * d)
        assert mean == pytest.approx(math.expm1(y * d), rel=1e-12)


def test_cr_math_is_correctly_rounded_on_samples():
    """The "cr" mode agrees with float64 numpy rounded once (a different library)."""
    x = torch.rand(100000) * 5
    for fn, ref in [("expm1", np.expm1), ("log1p", np.log1p), ("exp", np.exp),
                    ("log", np.log), ("sqrt", np.sqrt)]:
        a = getattr(O._CRMath, fn)(x + (1.0 if fn == "log" else 0.0)).numpy()
        b = ref((x + (1.0 if fn == "log" else 0.0)).numpy().astype(np.float64)).astype(np.float32)
        assert (a != b).sum() <= 1, fn
