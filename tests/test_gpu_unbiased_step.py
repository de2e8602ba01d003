"""LogSR unbiasedness of the optimizer step itself, with native Philox noise.

Every element but the first of a 10^7 + 1 element tensor has the same codes
and gradient, so all of them share one m', v' and one continuous bin index y
on the new grid; the first element sets the scales.  One ``LUMA.step()`` then
rounds those 10^7 copies of y with pass 2's production decision (the top 16
uniform bits decide, the low 8 bits are drawn only for elements whose
threshold falls inside their 2^-16 bucket).  The round-up frequency must
match the oracle's p* (z < 5) and the mean decoded value must equal the
linear value (the reference's TestLogSR, tests/test_correctness.py:40-103,
scaled to 10^7 draws; the draws are those of the step,
src/luma_optimizer/triton_kernel.py:93-128).

The gradient of the shared elements is chosen, among consecutive float32
values, to put p* of the momentum code at a target: inside a bucket, and just
above the bucket edge 100/256 (where the draws in the edge's 2^-16 bucket
need their low 8 bits).  The preconditioner code's p* falls where that gradient puts it.
"""

import math

import pytest
import torch

from luma_amd import LUMA
from oracle import luma_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
N = 10_000_000
HY = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
B1, B2 = HY["betas"]
EPS = HY["eps"]
# restored state (step 5): element 0 at the top of both grids, the others at
# codes QM / QW
OLD_S_M, OLD_S_V, QM, QW = 0.01, 1e-5, 20000, 40000
QW_BITS = QW - 65536   # Q_w holds the uint16 code's bits in int16
G0 = 0.05
EDGE = 100 / 256


def _moments(g, restored):
    """m', v' of elements with gradients g (element 0: G0) -- the oracle, cr."""
    if not restored:
        return O.init_moments(g, B1, B2)
    qm = torch.full(g.shape, QM, dtype=torch.int16)
    qw = torch.full(g.shape, QW_BITS, dtype=torch.int16)
    qm[0], qw[0] = O.K_M, 0
    return O.ema(qm, qw, g, OLD_S_M, OLD_S_V, B1, B2, EPS, "cr")


def _grid(restored):
    m, v = _moments(torch.tensor([G0]), restored)
    s_m = max(float(m.abs().max()), O.SCALE_FLOOR_M)
    s_v = max(float(v.max()), 0.0)
    return s_m, s_v, O.precompute(s_m, s_v, EPS)


def _thresholds(g, restored):
    """Per gradient: m', the momentum code's floor k_m and p*_m, v', the
    preconditioner code's floor k_w and p*_w, on the grid element 0 sets."""
    s_m, s_v, (w_min, dm, zm, dw, zw) = _grid(restored)
    x = torch.cat([torch.tensor([G0]), g])
    m, v = _moments(x, restored)
    assert float(m[1:].abs().max()) < s_m and float(v[1:].max()) < s_v   # element 0 sets S
    _, ym = O.momentum_bin(m, s_m, dm, "cr")
    km, pm = O.log_sr_threshold(ym, dm, zm, "cr")
    yw = O.preconditioner_bin(v, EPS, w_min, dw, "cr")
    kw, pw = O.log_sr_threshold(yw, dw, zw, "cr")
    return m[1:], km[1:], pm[1:], v[1:], kw[1:], pw[1:]


def _pick_grad(target, restored, lo=None):
    """Among 20,000 consecutive float32 gradients from 4e-3, the one whose p*_m
    is closest to target (or, with lo, the smallest p*_m >= lo)."""
    start = torch.tensor([4e-3], dtype=torch.float32).view(torch.int32)
    g = (start + torch.arange(20000, dtype=torch.int32)).view(torch.float32)
    _, _, pm, _, _, _ = _thresholds(g, restored)
    if lo is None:
        i = int((pm - target).abs().argmin())
    else:
        d = torch.where(pm >= lo, pm - lo, torch.full_like(pm, 2.0))
        i = int(d.argmin())
    return float(g[i])


def _check_code(codes, k, p, dec_k, dec_k1, x, what):
    """Codes in {k, k+1}; frequency of k+1 against p (z < 5); the mean decode
    (1-f) dec(k) + f dec(k+1) against the linear value x."""
    lo_n = int((codes == k).sum())
    hi_n = int((codes == k + 1).sum())
    assert lo_n + hi_n == N, (what, lo_n, hi_n)
    f = hi_n / N
    sigma = math.sqrt(max(p * (1 - p), 1e-12) / N)
    z = abs(f - p) / sigma
    mean = (1 - f) * dec_k + f * dec_k1
    bin_w = dec_k1 - dec_k
    print(f"{what}: k={k} p*={p:.6f} f={f:.6f} z={z:.2f} mean={mean:.9g} x={x:.9g}", flush=True)
    assert z < 5, (what, f, p, z)
    assert abs(mean - x) < 5 * sigma * abs(bin_w) + 4e-7 * abs(x), (what, mean, x)


CASES = [("restored", 0.1), ("restored", 0.37), ("restored", 0.5), ("restored", 0.83),
         ("restored", "edge"), ("init", 0.37), ("init", "edge")]


@pytest.mark.parametrize("mode,target", CASES)
def test_step_logsr_unbiased_1e7(mode, target):
    restored = mode == "restored"
    g = (_pick_grad(None, restored, lo=EDGE) if target == "edge"
         else _pick_grad(target, restored))
    m, km, pm, v, kw, pw = (float(a[0]) for a in _thresholds(torch.tensor([g]), restored))
    km, kw = int(km), int(kw)
    if target == "edge":
        assert EDGE <= pm < EDGE + 2e-3, pm      # just above the bucket edge
    print(f"case {mode} target={target}: g={g!r} p*_m={pm:.6f} p*_w={pw:.6f}", flush=True)

    p = torch.nn.Parameter(torch.zeros(N + 1, device=DEV))
    opt = LUMA([p], **HY)
    opt._base_seed = 0x6A09E667F3BCC908
    if restored:
        q_m = torch.full((N + 1,), QM, dtype=torch.int16, device=DEV)
        q_w = torch.full((N + 1,), QW_BITS, dtype=torch.int16, device=DEV)
        q_m[0], q_w[0] = O.K_M, 0
        sd = opt.state_dict()
        sd["state"] = {0: {"step": 5, "param_id": 0, "Q_m": q_m, "Q_w": q_w,
                           "S_m": OLD_S_M, "S_v": OLD_S_V}}
        opt.load_state_dict(sd)
    grad = torch.full((N + 1,), g, device=DEV)
    grad[0] = G0
    p.grad = grad
    opt.step()
    torch.cuda.synchronize()
    st = opt.state_dict()["state"][0]
    assert st["step"] == (6 if restored else 1)
    s_m, s_v, (w_min, dm, zm, dw, zw) = _grid(restored)
    assert st["S_m"] == s_m and st["S_v"] == s_v
    # momentum: decode of codes k, k+1 and the linear value m'
    dec = O.decode_momentum(torch.tensor([km, km + 1], dtype=torch.int16), dm, "cr").double()
    _check_code(st["Q_m"][1:].to(torch.int32), km, pm, float(dec[0]), float(dec[1]), m, "Q_m")
    # preconditioner: LogSR is unbiased in w = 1 / (sqrt(v') + eps) (clamped)
    w = min(max(1.0 / (float(torch.tensor(v).double().sqrt()) + EPS), w_min), 1.0 / EPS)
    decw = O.decode_preconditioner(torch.tensor([kw, kw + 1], dtype=torch.int32).to(torch.int16),
                                   w_min, dw, "cr").double()
    _check_code(st["Q_w"][1:].to(torch.int32) & 0xFFFF, kw, pw, float(decw[0]), float(decw[1]),
                w, "Q_w")
