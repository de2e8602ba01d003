"""CPU oracle for the LUMA optimizer step -- TEST INFRASTRUCTURE ONLY.

This module restates, on CPU with torch float32 arithmetic, the reference's
PyTorch backend (``src/luma_optimizer/functional.py``) and the bookkeeping of
``LUMA.step`` / ``state_dict`` / ``export_adamw_state`` /
``import_adamw_state`` (``src/luma_optimizer/optimizer.py``).  The tests
compare the HIP implementation in ``luma_amd`` against it: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import it,
and never as the code path being measured or shipped.

Two knobs make it useful for those comparisons:

* ``math`` -- the elementwise transcendental functions.  ``"torch"`` uses the
  same ATen CPU kernels the reference calls (MKL VML for exp/log/sqrt, SLEEF
  for expm1/log1p), so it reproduces the reference bit for bit.  ``"cr"``
  evaluates expm1/log1p/exp/log/sqrt in float64 and rounds once to float32,
  i.e. correctly rounded results; every other operation is unchanged.  The
  GPU implementation is correctly rounded, so it must match ``"cr"``
  bit for bit, and the reference (``"torch"``) up to the elements where the
  CPU libraries are not correctly rounded.
* ``draw`` -- where the stochastic-rounding uniforms come from.  By default a
  ``torch.Generator`` seeded exactly as the reference seeds it (one
  generator per (param, step), momentum draws first, then preconditioner
  draws).  Tests capture those draws and inject the same uniforms into the
  GPU kernels.

Every function cites the reference lines it follows.  Pinning (see the
tests): golden vectors written by running the reference in the build
container (``tests/golden/``), closed forms for the codec / seed / grid
scalars, and brute-force float64 checks on tiny inputs.
"""

from __future__ import annotations

import math
from typing import Callable, Dict, Optional, Tuple

import torch
from torch import Tensor

# config.py:23-25
K_M: int = (1 << 15) - 1
K_W: int = (1 << 16) - 1
SCALE_FLOOR_M: float = 1e-9


# ---------------------------------------------------------------------------
#  Elementwise math modes
# ---------------------------------------------------------------------------

class _TorchMath:
    """The ATen CPU kernels the reference uses (functional.py:65,116,126,143,163,167)."""

    name = "torch"
    expm1 = staticmethod(torch.expm1)
    log1p = staticmethod(torch.log1p)
    exp = staticmethod(torch.exp)
    log = staticmethod(torch.log)
    sqrt = staticmethod(torch.sqrt)


class _CRMath:
    """Correctly rounded float32 results: evaluate in float64, round once."""

    name = "cr"

    @staticmethod
    def expm1(x: Tensor) -> Tensor:
        return torch.expm1(x.double()).float()

    @staticmethod
    def log1p(x: Tensor) -> Tensor:
        return torch.log1p(x.double()).float()

    @staticmethod
    def exp(x: Tensor) -> Tensor:
        return torch.exp(x.double()).float()

    @staticmethod
    def log(x: Tensor) -> Tensor:
        return torch.log(x.double()).float()

    @staticmethod
    def sqrt(x: Tensor) -> Tensor:
        return torch.sqrt(x.double()).float()


MATH = {"torch": _TorchMath, "cr": _CRMath}


def _m(math_mode):
    return MATH[math_mode] if isinstance(math_mode, str) else math_mode


# ---------------------------------------------------------------------------
#  Codec, LogSR, grid scalars, seeds
# ---------------------------------------------------------------------------

def encode_uint16(values: Tensor) -> Tensor:
    """functional.py:24-26 -- unsigned [0, 65535] stored as int16 bits."""
    return values.to(torch.int16)


def decode_uint16(q: Tensor) -> Tensor:
    """functional.py:29-31."""
    return (q.to(torch.int32) & 0xFFFF).float()


def log_sr_threshold(y: Tensor, delta: float, z_denom: float, math_mode="torch"):
    """functional.py:61-64 -- ``floor(y)`` and the round-up probability
    ``p* = expm1(frac(y) * delta) / z_denom`` of LogSR (delta > 0)."""
    M = _m(math_mode)
    fl = y.floor()
    frac = y - fl
    return fl, M.expm1(frac * delta) / z_denom


def log_sr(y: Tensor, delta: float, z_denom: float, rand: Tensor, k_max: int,
           math_mode="torch") -> Tensor:
    """functional.py:38-67 -- log-to-linear corrected stochastic rounding."""
    if delta <= 0.0:
        return torch.zeros_like(y)
    fl, p_star = log_sr_threshold(y, delta, z_denom, math_mode)
    return (fl + (rand < p_star).to(y.dtype)).clamp(0, k_max)


def momentum_bin(m: Tensor, S_m: float, delta_m: float, math_mode="torch"):
    """functional.py:142-143 -- the clamped momentum and its continuous bin
    index ``y = log1p(|clamp(m, +-S_m)|) / delta_m``."""
    M = _m(math_mode)
    m_clip = m.clamp(-S_m, S_m)
    return m_clip, M.log1p(m_clip.abs()) / delta_m


def preconditioner_bin(v: Tensor, eps: float, w_min: float, delta_w: float,
                       math_mode="torch") -> Tensor:
    """functional.py:163-169 -- the continuous bin index of ``w = 1/(sqrt(v)+eps)``
    on the preconditioner grid (0 when delta_w <= 0)."""
    M = _m(math_mode)
    w = 1.0 / (M.sqrt(v.clamp_min(0)) + eps)
    w_clip = w.clamp(w_min, 1.0 / eps)
    if delta_w > 0.0:
        return M.log(w_clip / w_min) / delta_w
    return torch.zeros_like(w_clip)


def precompute(S_m: float, S_v: float, eps: float):
    """functional.py:74-92 -- grid scalars in Python double.

    Returns ``(w_min, delta_m, z_m, delta_w, z_w)``.
    """
    w_min = 1.0 / (math.sqrt(S_v) + eps)
    delta_m = math.log1p(S_m) / K_M
    z_m = math.expm1(delta_m)
    ratio = 1.0 / (eps * w_min)
    delta_w = math.log(ratio) / K_W if ratio > 1.0 else 0.0
    z_w = math.expm1(delta_w) if delta_w > 0.0 else 1.0
    return w_min, delta_m, z_m, delta_w, z_w


def make_step_seed(base_seed: int, step: int, param_id: int) -> int:
    """functional.py:99-106."""
    return ((step << 32) | (param_id * 2)) ^ base_seed


def decode_momentum(Q_m: Tensor, delta_m: float, math_mode="torch") -> Tensor:
    """functional.py:113-116: ``m = sgn(q) * expm1(|q| * delta_m)``."""
    M = _m(math_mode)
    q = Q_m.float()
    return q.sign() * M.expm1(q.abs() * delta_m)


def decode_preconditioner(Q_w: Tensor, w_min: float, delta_w: float,
                          math_mode="torch") -> Tensor:
    """functional.py:119-126: ``w = w_min * exp(u16(q) * delta_w)``."""
    M = _m(math_mode)
    return w_min * M.exp(decode_uint16(Q_w) * delta_w)


def decode_second_moment(Q_w: Tensor, w_min: float, delta_w: float, eps: float,
                         math_mode="torch") -> Tensor:
    """functional.py:269-270 (and optimizer.py:234-235): ``v = (1/w - eps)_+^2``."""
    w = decode_preconditioner(Q_w, w_min, delta_w, math_mode)
    return (1.0 / w - eps).clamp_min(0).square()


def quantize_momentum(m: Tensor, S_m: float, delta_m: float, z_m: float,
                      rand: Tensor, math_mode="torch") -> Tensor:
    """functional.py:133-150 (the uniforms are passed in instead of drawn)."""
    M = _m(math_mode)
    m_clip, y = momentum_bin(m, S_m, delta_m, M)
    q_mag = log_sr(y, delta_m, z_m, rand, K_M, M)
    return (m_clip.sign() * q_mag).to(torch.int16)


def quantize_preconditioner(v: Tensor, eps: float, w_min: float, delta_w: float,
                            z_w: float, rand: Tensor, math_mode="torch") -> Tensor:
    """functional.py:153-176 (the uniforms are passed in instead of drawn)."""
    M = _m(math_mode)
    y = preconditioner_bin(v, eps, w_min, delta_w, M)
    q = log_sr(y, delta_w, z_w, rand, K_W, M)
    return encode_uint16(q.to(torch.int32))


# ---------------------------------------------------------------------------
#  Draws
# ---------------------------------------------------------------------------

Draw = Callable[[torch.Size], Tensor]


def generator_draw(seed: int) -> Draw:
    """optimizer.py:389-393 + functional.py:144,170.

    One CPU generator per (param, step); every call draws the next uniforms.
    ``manual_seed`` takes the signed 64-bit seed and uses its two's-complement
    bits, which is what the reference relies on for negative seeds.
    """
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)

    def draw(shape):
        return torch.rand(shape, dtype=torch.float32, generator=gen)

    return draw


class RecordingDraw:
    """Wraps a draw and keeps what it returned (momentum first, then w)."""

    def __init__(self, inner: Draw):
        self.inner = inner
        self.draws = []

    def __call__(self, shape):
        u = self.inner(shape)
        self.draws.append(u.clone())
        return u


def injected_draw(u_m: Tensor, u_w: Tensor) -> Draw:
    """Hands out ``u_m`` then ``u_w`` (shapes must match the tensor)."""
    seq = [u_m, u_w]

    def draw(shape):
        u = seq.pop(0)
        assert tuple(u.shape) == tuple(shape)
        return u

    return draw


# ---------------------------------------------------------------------------
#  Step functions (functional.py:183-298)
# ---------------------------------------------------------------------------

def init_moments(grad: Tensor, beta1: float, beta2: float):
    """functional.py:200-204 -- the first step's moments ``m = (1-b1) g``,
    ``v = (1-b2) g^2`` (float32, the scalar cast once)."""
    g = grad.float()
    return (1.0 - beta1) * g, (1.0 - beta2) * g.square()


def init_step(param: Tensor, grad: Tensor, beta1: float, beta2: float, eps: float,
              lr: float, weight_decay: float, draw: Draw, math_mode="torch"):
    """functional.py:183-228.  Mutates ``param``; returns (Q_m, Q_w, S_m, S_v)."""
    M = _m(math_mode)
    m, v = init_moments(grad, beta1, beta2)
    bc1 = 1.0 - beta1
    bc2 = 1.0 - beta2
    eta_t = lr / bc1
    param.mul_(1.0 - lr * weight_decay)
    param.addcdiv_(m, M.sqrt(v / bc2).add_(eps), value=-eta_t)
    S_m_t, S_v_t = torch.stack([m.abs().max(), v.max()]).tolist()
    S_m = max(S_m_t, SCALE_FLOOR_M)
    S_v = max(S_v_t, 0.0)
    w_min, delta_m, z_m, delta_w, z_w = precompute(S_m, S_v, eps)
    Q_m = quantize_momentum(m, S_m, delta_m, z_m, draw(m.shape), M)
    Q_w = quantize_preconditioner(v, eps, w_min, delta_w, z_w, draw(v.shape), M)
    return Q_m, Q_w, S_m, S_v


def ema(Q_m: Tensor, Q_w: Tensor, grad: Tensor, S_m: float, S_v: float,
        beta1: float, beta2: float, eps: float, math_mode="torch"):
    """functional.py:259,265-275 -- decode the stored codes and apply the EMA.

    Returns ``(m_new, v_new)`` as float32 tensors.
    """
    M = _m(math_mode)
    g = grad.float()
    w_min, delta_m, _, delta_w, _ = precompute(S_m, S_v, eps)
    m = decode_momentum(Q_m, delta_m, M)
    v = decode_second_moment(Q_w, w_min, delta_w, eps, M)
    m_new = beta1 * m + (1.0 - beta1) * g
    v_new = beta2 * v + (1.0 - beta2) * g.square()
    return m_new, v_new


def update_step(param: Tensor, grad: Tensor, Q_m: Tensor, Q_w: Tensor, S_m: float,
                S_v: float, step: int, beta1: float, beta2: float, eps: float,
                lr: float, weight_decay: float, draw: Draw, math_mode="torch"):
    """functional.py:231-298.  Mutates param/Q_m/Q_w; returns (S_m', S_v')."""
    M = _m(math_mode)
    bc1 = 1.0 - beta1 ** step
    bc2 = 1.0 - beta2 ** step
    eta_t = lr / bc1
    m_new, v_new = ema(Q_m, Q_w, grad, S_m, S_v, beta1, beta2, eps, M)
    param.mul_(1.0 - weight_decay * lr)
    param.addcdiv_(m_new, M.sqrt(v_new / bc2).add_(eps), value=-eta_t)
    S_m_t, S_v_t = torch.stack([m_new.abs().max(), v_new.max()]).tolist()
    S_m_next = max(S_m_t, SCALE_FLOOR_M)
    S_v_next = max(S_v_t, 0.0)
    w_min, delta_m, z_m, delta_w, z_w = precompute(S_m_next, S_v_next, eps)
    Q_m.copy_(quantize_momentum(m_new, S_m_next, delta_m, z_m, draw(m_new.shape), M))
    Q_w.copy_(quantize_preconditioner(v_new, eps, w_min, delta_w, z_w,
                                      draw(v_new.shape), M))
    return S_m_next, S_v_next


def quantize_states(m: Tensor, v: Tensor, eps: float, draw: Draw, math_mode="torch"):
    """optimizer.py:307-321 -- the import_adamw_state quantisation of given m, v."""
    M = _m(math_mode)
    m = m.float()
    v = v.float().clamp(min=0.0)
    S_m = max(m.abs().max().item(), SCALE_FLOOR_M)
    S_v = max(v.max().item(), 0.0)
    w_min, delta_m, z_m, delta_w, z_w = precompute(S_m, S_v, eps)
    Q_m = quantize_momentum(m, S_m, delta_m, z_m, draw(m.shape), M)
    Q_w = quantize_preconditioner(v, eps, w_min, delta_w, z_w, draw(v.shape), M)
    return Q_m, Q_w, S_m, S_v


# ---------------------------------------------------------------------------
#  Optimizer bookkeeping (optimizer.py, PyTorch backend only)
# ---------------------------------------------------------------------------

class OracleLUMA:
    """The reference optimizer's PyTorch-backend path over CPU tensors.

    ``params`` is a list of param-group dicts (each with ``params``, ``lr``,
    ``betas``, ``eps``, ``weight_decay``) of CPU float32 tensors whose
    ``.grad`` the caller sets.  ``base_seed`` plays the role of
    ``LUMA._base_seed`` (optimizer.py:94-96).  ``draw_factory(seed, pid, t)``
    returns the Draw for one (param, step); by default the reference's seeded
    generator.  After each ``step()`` the uniforms used are in
    ``last_draws[param_id] = (u_m, u_w)``.
    """

    def __init__(self, groups, base_seed: int, math_mode="torch",
                 draw_factory: Optional[Callable[[int, int, int], Draw]] = None):
        self.param_groups = groups
        self.base_seed = base_seed
        self.math_mode = math_mode
        self.state: Dict[int, dict] = {}
        self.draw_factory = draw_factory
        self.last_draws: Dict[int, Tuple[Tensor, Tensor]] = {}

    def _draw(self, seed, pid, t):
        if self.draw_factory is not None:
            return RecordingDraw(self.draw_factory(seed, pid, t))
        return RecordingDraw(generator_draw(seed))

    @torch.no_grad()
    def step(self):
        """optimizer.py:413-524 (PyTorch branch)."""
        self.last_draws = {}
        param_idx = 0
        for group in self.param_groups:
            beta1, beta2 = group["betas"]
            eps, lr, wd = group["eps"], group["lr"], group["weight_decay"]
            for p in group["params"]:
                param_idx += 1
                if p.grad is None:
                    continue
                if p.numel() == 0:
                    continue
                if p.grad.is_sparse:
                    raise RuntimeError("LUMA does not support sparse gradients")
                if p.dtype != torch.float32:
                    raise ValueError(f"LUMA requires float32 parameters (got {p.dtype}).")
                st = self.state.setdefault(id(p), {})
                if len(st) == 0:
                    st["step"] = 0
                    st["param_id"] = param_idx - 1
                st["step"] += 1
                t = st["step"]
                seed = make_step_seed(self.base_seed, t, st["param_id"])
                draw = self._draw(seed, st["param_id"], t)
                if t == 1:
                    Q_m, Q_w, S_m, S_v = init_step(p, p.grad, beta1, beta2, eps, lr, wd,
                                                   draw, self.math_mode)
                    st["Q_m"], st["Q_w"], st["S_m"], st["S_v"] = Q_m, Q_w, S_m, S_v
                else:
                    S_m, S_v = update_step(p, p.grad, st["Q_m"], st["Q_w"], st["S_m"],
                                           st["S_v"], t, beta1, beta2, eps, lr, wd,
                                           draw, self.math_mode)
                    st["S_m"], st["S_v"] = S_m, S_v
                self.last_draws[st["param_id"]] = tuple(draw.draws)

    def export_adamw_state(self) -> dict:
        """optimizer.py:189-250."""
        index = {}
        for group in self.param_groups:
            for p in group["params"]:
                index[id(p)] = len(index)
        out = {}
        for group in self.param_groups:
            eps = group["eps"]
            for p in group["params"]:
                st = self.state.get(id(p))
                if not st:
                    continue
                w_min, delta_m, _, delta_w, _ = precompute(st["S_m"], st["S_v"], eps)
                exp_avg = decode_momentum(st["Q_m"], delta_m, self.math_mode)
                w = decode_preconditioner(st["Q_w"], w_min, delta_w, self.math_mode)
                exp_avg_sq = (1.0 / w - eps).clamp(min=0).square()
                out[index[id(p)]] = {"step": torch.tensor(float(st["step"])),
                                     "exp_avg": exp_avg, "exp_avg_sq": exp_avg_sq}
        groups = []
        for group in self.param_groups:
            pg = {k: v for k, v in group.items() if k != "params"}
            pg["params"] = [index[id(p)] for p in group["params"]]
            groups.append(pg)
        return {"state": out, "param_groups": groups}

    def import_adamw_state(self, adamw_sd: dict) -> None:
        """optimizer.py:256-335 (PyTorch branch): step-0 seed per param index."""
        flat = []
        for group in self.param_groups:
            for p in group["params"]:
                flat.append((p, group))
        for key, s in adamw_sd["state"].items():
            idx = int(key)
            if idx >= len(flat):
                raise ValueError(f"AdamW state has index {idx} but LUMA only has "
                                 f"{len(flat)} parameters")
            p, group = flat[idx]
            step_val = s["step"]
            step = int(step_val.item() if isinstance(step_val, Tensor) else step_val)
            draw = self._draw(make_step_seed(self.base_seed, 0, idx), idx, 0)
            Q_m, Q_w, S_m, S_v = quantize_states(s["exp_avg"], s["exp_avg_sq"],
                                                 group["eps"], draw, self.math_mode)
            self.state[id(p)] = {"step": step, "param_id": idx, "Q_m": Q_m,
                                 "Q_w": Q_w, "S_m": S_m, "S_v": S_v}
            self.last_draws[idx] = tuple(draw.draws)
