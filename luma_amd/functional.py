"""Per-tensor functional form of the HIP step, as ``torch.library`` custom ops.

The reference exposes its Triton pipeline as two per-tensor functions,
``luma_triton_init_step`` and ``luma_triton_step`` (triton_kernel.py:409-492),
that take every piece of state as a tensor (``new_grid``, ``old_scalars``,
``step_tensor``, ...) so that ``torch.compile(fullgraph=True)`` traces them
without graph breaks and CUDA graphs replay them (tests/test_compile.py).
Here one op covers both: a tensor's state is ``Q_m``, ``Q_w`` and its
``slot`` (a ``LUMA_SLOT_BYTES`` uint8 tensor holding the step count, S_m,
S_v and the grids).  A fresh slot (``new_slot``) has step count 0, so the
next ``luma_step`` is the init step; each call advances the count on the
device.  ``torch.compile`` records each call as one opaque op
(``torch.ops.luma_amd.luma_step``) that mutates ``param``, ``Q_m``, ``Q_w``
and ``slot``.

The op launches through ``luma_step_tensor`` of the C ABI (include/luma.h):
no device tables, no host synchronisation.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import numpy as np
import torch

from . import _lib as L

_GRAD_CODES = {torch.float32: L.GRAD_F32, torch.bfloat16: L.GRAD_BF16, torch.float16: L.GRAD_F16}
_MASK64 = (1 << 64) - 1

__all__ = ["luma_step", "new_slot", "init_slot", "slot_state"]


def new_slot(device) -> torch.Tensor:
    """A fresh slot for one tensor: zero-filled, step count 0."""
    return torch.zeros(L.SLOT_BYTES, dtype=torch.uint8, device=device)


def _check(param, grad, Q_m, Q_w, slot, u_m, u_w):
    if not param.is_cuda:
        raise RuntimeError(f"luma_step: tensors must be on a ROCm GPU; got {param.device}")
    # triton_kernel.py:392-401
    if param.dtype != torch.float32:
        raise ValueError(f"LUMA HIP kernel requires float32 parameters (got {param.dtype})")
    if not param.is_contiguous():
        raise ValueError("LUMA HIP kernel requires contiguous parameters")
    if not grad.is_contiguous():
        raise ValueError("LUMA HIP kernel requires contiguous gradients")
    if grad.dtype not in _GRAD_CODES:
        raise ValueError(f"luma_step: gradient dtype {grad.dtype} is not float32/bfloat16/float16")
    if Q_m.dtype != torch.int16 or Q_w.dtype != torch.int16:
        raise ValueError("luma_step: Q_m and Q_w must be int16")
    if slot.dtype != torch.uint8 or slot.numel() != L.SLOT_BYTES or not slot.is_contiguous():
        raise ValueError(f"luma_step: slot must be a contiguous uint8 tensor of {L.SLOT_BYTES} "
                         "elements (see new_slot)")
    if slot.data_ptr() % 16:
        raise ValueError("luma_step: slot must be 16-byte aligned")
    n = param.numel()
    for name, t in (("grad", grad), ("Q_m", Q_m), ("Q_w", Q_w), ("u_m", u_m), ("u_w", u_w)):
        if t is None:
            continue
        if t.device != param.device:
            raise ValueError(f"luma_step: {name} is on {t.device}, param on {param.device}")
        if t.numel() != n:
            raise ValueError(f"luma_step: {name} has {t.numel()} elements, param {n}")
    # one flat element order for all operands
    for name, t in (("Q_m", Q_m), ("Q_w", Q_w), ("u_m", u_m), ("u_w", u_w)):
        if t is not None and not t.is_contiguous():
            raise ValueError(f"LUMA HIP kernel requires contiguous {name}")
    if (u_m is None) != (u_w is None):
        raise ValueError("luma_step: pass both u_m and u_w, or neither")
    for name, t in (("u_m", u_m), ("u_w", u_w)):
        if t is not None and t.dtype != torch.float32:
            raise ValueError(f"luma_step: {name} must be float32")


@torch.library.custom_op("luma_amd::luma_step", mutates_args=("param", "Q_m", "Q_w", "slot"),
                         device_types="cuda")
def _luma_step_op(param: torch.Tensor, grad: torch.Tensor, Q_m: torch.Tensor,
                  Q_w: torch.Tensor, slot: torch.Tensor, beta1: float, beta2: float, eps: float,
                  lr: float, weight_decay: float, param_id: int, base_seed: int,
                  u_m: Optional[torch.Tensor] = None, u_w: Optional[torch.Tensor] = None,
                  exact: bool = False, grad_scale: Optional[torch.Tensor] = None,
                  found_inf: Optional[torch.Tensor] = None, elem_offset: int = 0) -> None:
    _check(param, grad, Q_m, Q_w, slot, u_m, u_w)
    if elem_offset < 0:
        raise ValueError("luma_step: elem_offset must be >= 0")
    for name, t in (("grad_scale", grad_scale), ("found_inf", found_inf)):
        if t is not None and (t.numel() != 1 or t.dtype != torch.float32
                              or t.device != param.device):
            raise ValueError(f"luma_step: {name} must be a one-element float32 tensor on "
                             f"{param.device}")
    n = param.numel()
    if n == 0:
        return
    lib = L.load()
    tt = np.zeros(1, dtype=L.TENSOR_DTYPE)
    tt["param"] = param.data_ptr()
    tt["grad"] = grad.data_ptr()
    tt["q_m"] = Q_m.data_ptr()
    tt["q_w"] = Q_w.data_ptr()
    tt["u_m"] = 0 if u_m is None else u_m.data_ptr()
    tt["u_w"] = 0 if u_w is None else u_w.data_ptr()
    tt["slot"] = slot.data_ptr()
    tt["numel"] = n
    tt["param_id"] = param_id
    tt["elem_offset"] = elem_offset
    tt["grad_dtype"] = _GRAD_CODES[grad.dtype]
    gg = np.array([(lr, beta1, beta2, eps, weight_decay, 0.0)], dtype=L.GROUP_DTYPE)
    nch = (n + L.STEP_TENSOR_CHUNK_MIN - 1) // L.STEP_TENSOR_CHUNK_MIN   # at most this many chunks
    partials = torch.empty(max(lib.luma_workspace_bytes(nch) // 4, 4), dtype=torch.float32,
                           device=param.device)
    noise = L.NOISE_PHILOX if u_m is None else L.NOISE_INJECTED
    stream = torch.cuda.current_stream(param.device).cuda_stream
    scaling = L.Scaling(None if grad_scale is None else grad_scale.data_ptr(),
                        None if found_inf is None else found_inf.data_ptr())
    rc = lib.luma_step_tensor(tt.ctypes.data, gg.ctypes.data, partials.data_ptr(),
                              base_seed & _MASK64, noise, L.FLAG_EXACT_ONLY if exact else 0,
                              ctypes.byref(scaling), stream)
    L.check(rc, "luma_step_tensor")


@_luma_step_op.register_fake
def _luma_step_fake(param, grad, Q_m, Q_w, slot, beta1, beta2, eps, lr, weight_decay, param_id,
                    base_seed, u_m=None, u_w=None, exact=False, grad_scale=None,
                    found_inf=None, elem_offset=0) -> None:
    return None


def luma_step(param: torch.Tensor, grad: torch.Tensor, Q_m: torch.Tensor, Q_w: torch.Tensor,
              slot: torch.Tensor, beta1: float, beta2: float, eps: float, lr: float,
              weight_decay: float, param_id: int, base_seed: int,
              u_m: Optional[torch.Tensor] = None, u_w: Optional[torch.Tensor] = None,
              exact: bool = False, grad_scale: Optional[torch.Tensor] = None,
              found_inf: Optional[torch.Tensor] = None, elem_offset: int = 0) -> None:
    """One LUMA step of one tensor, in place.

    The init step (functional.py:183-228) when ``slot`` holds step count 0,
    else the update step (functional.py:231-298) at t = count + 1.  Uniforms
    come from Philox keyed by ``((t << 32) | 2*param_id) ^ base_seed``, or from
    ``u_m`` / ``u_w`` (float32 in [0, 1), the parameter's shape) when given.
    ``exact`` forces the exact per-element path (same results, slower).
    ``grad_scale`` / ``found_inf`` (one-element float32 device tensors) are
    GradScaler's: the gradient is unscaled in the kernel as ``unscale_``
    would store it, and a nonzero ``found_inf`` skips the step on the device.
    ``elem_offset``: when ``param`` is one shard of a larger parameter, the
    index of its first element in the whole (flattened) parameter; the Philox
    counters follow that index, so shards draw independent uniforms (and a
    shard whose offset is a multiple of 8 draws exactly the uniforms of the
    same elements of the unsharded parameter).
    """
    torch.ops.luma_amd.luma_step(param, grad, Q_m, Q_w, slot, beta1, beta2, eps, lr,
                                 weight_decay, param_id, base_seed, u_m, u_w, exact, grad_scale,
                                 found_inf, elem_offset)


def init_slot(slot: torch.Tensor, step: int, S_m: float, S_v: float, eps: float) -> None:
    """Write a slot's step count and scales (the slot half of loading saved
    state, optimizer.py:146-183 and 341-387)."""
    lib = L.load()
    arr = np.zeros(1, dtype=L.SCALE_INIT_DTYPE)
    arr[0] = (slot.data_ptr(), int(step), float(S_m), float(S_v), float(eps))
    d = torch.from_numpy(arr.view(np.uint8)).to(slot.device)
    L.check(lib.luma_set_scales(d.data_ptr(), 1,
                                torch.cuda.current_stream(slot.device).cuda_stream),
            "luma_set_scales")


def slot_state(slot: torch.Tensor) -> Tuple[int, float, float]:
    """(step count, S_m, S_v) held by a slot (synchronises)."""
    lib = L.load()
    ptrs = torch.tensor([slot.data_ptr()], dtype=torch.int64, device=slot.device)
    scales = torch.empty(2, dtype=torch.float64, device=slot.device)
    steps = torch.empty(1, dtype=torch.int64, device=slot.device)
    L.check(lib.luma_get_scales(ptrs.data_ptr(), 1, scales.data_ptr(), steps.data_ptr(),
                                torch.cuda.current_stream(slot.device).cuda_stream),
            "luma_get_scales")
    sc = scales.cpu().tolist()
    return int(steps.item()), sc[0], sc[1]
