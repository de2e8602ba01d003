"""ctypes binding of libluma_hip.so (C ABI in include/luma.h).

The table layouts below mirror the C structs byte for byte; ``check_layout``
compares them with the sizes the library reports.  Loading fails loudly: there
is no fallback implementation of the step.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_NAME = "libluma_hip.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)

CHUNK_ELEMS = 131072         # LUMA_CHUNK_ELEMS (default and largest chunk length)
CHUNK_ELEMS_MIN = 2048       # LUMA_CHUNK_ELEMS_MIN
SMALL_TENSOR = 256           # LUMA_SMALL_TENSOR
MEDIUM_TENSOR = 8192         # LUMA_MEDIUM_TENSOR
STEP_TENSOR_CHUNK_MIN = 16384  # LUMA_STEP_TENSOR_CHUNK_MIN
SLOT_BYTES = 512             # LUMA_SLOT_BYTES
NOALLOC_MAX_CHUNKS = 262144  # LUMA_NOALLOC_MAX_CHUNKS
SUMMARY_WORDS = 256          # LUMA_SUMMARY_WORDS (per chunk)
ABI_VERSION = 9              # LUMA_ABI_VERSION

GRAD_F32, GRAD_BF16, GRAD_F16 = 0, 1, 2
NOISE_PHILOX, NOISE_INJECTED = 0, 1
FLAG_EXACT_ONLY = 1

TENSOR_DTYPE = np.dtype([
    ("param", "<u8"), ("grad", "<u8"), ("q_m", "<u8"), ("q_w", "<u8"),
    ("u_m", "<u8"), ("u_w", "<u8"), ("slot", "<u8"), ("summary", "<u8"), ("summary_words", "<i8"),
    ("numel", "<i8"), ("param_id", "<i8"), ("elem_offset", "<i8"),
    ("grad_dtype", "<i4"), ("group", "<i4"), ("first_chunk", "<i4"), ("reserved", "<i4"),
])
CHUNK_DTYPE = np.dtype([("tensor", "<i4"), ("index", "<i4")])
GROUP_DTYPE = np.dtype([
    ("lr", "<f8"), ("beta1", "<f8"), ("beta2", "<f8"), ("eps", "<f8"),
    ("weight_decay", "<f8"), ("reserved", "<f8"),
])
SCALE_INIT_DTYPE = np.dtype([
    ("slot", "<u8"), ("step", "<i8"), ("s_m", "<f8"), ("s_v", "<f8"), ("eps", "<f8"),
])
# luma_hyper_rows output columns
HYPER_ROW_FIELDS = ("beta1", "omb1", "beta2", "omb2", "decay", "neg_eta", "bc2", "eps")


class Scaling(ctypes.Structure):
    """LumaScaling: GradScaler's scale and found_inf device scalars (or NULL)."""
    _fields_ = [("grad_scale", ctypes.c_void_p), ("found_inf", ctypes.c_void_p)]


class StepArgs(ctypes.Structure):
    _fields_ = [
        ("tensors", ctypes.c_void_p),
        ("n_tensors", ctypes.c_int32),
        ("n_chunks", ctypes.c_int32),
        ("chunks", ctypes.c_void_p),
        ("groups", ctypes.c_void_p),
        ("partials", ctypes.c_void_p),
        ("base_seed", ctypes.c_uint64),
        ("noise_mode", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("chunk_elems", ctypes.c_int32),
        ("small_chunks", ctypes.c_int32),
        ("medium_chunks", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("scaling", Scaling),
    ]


class LumaLibraryError(RuntimeError):
    pass


_lib = None

_VP = ctypes.c_void_p
_SIGNATURES = {
    "luma_abi_version": (ctypes.c_int, []),
    "luma_last_error": (ctypes.c_char_p, []),
    "luma_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int32]),
    "luma_summary_words": (ctypes.c_int64, [ctypes.c_int64, ctypes.c_int32]),
    "luma_layout": (None, [ctypes.POINTER(ctypes.c_int32)]),
    "luma_step": (ctypes.c_int, [ctypes.POINTER(StepArgs), _VP]),
    "luma_step_noalloc": (ctypes.c_int, [ctypes.POINTER(StepArgs), _VP]),
    "luma_step_profiled": (ctypes.c_int, [ctypes.POINTER(StepArgs), _VP,
                                          ctypes.POINTER(ctypes.c_void_p)]),
    "luma_step_tensor": (ctypes.c_int, [_VP, _VP, _VP, ctypes.c_uint64, ctypes.c_int32,
                                        ctypes.c_int32, ctypes.POINTER(Scaling), _VP]),
    "luma_set_scales": (ctypes.c_int, [_VP, ctypes.c_int32, _VP]),
    "luma_get_scales": (ctypes.c_int, [_VP, ctypes.c_int32, _VP, _VP, _VP]),
    "luma_decode": (ctypes.c_int, [_VP, _VP, ctypes.c_int64, _VP, ctypes.c_double, _VP, _VP,
                                   _VP]),
    "luma_quantize": (ctypes.c_int, [_VP, _VP, ctypes.c_int64, _VP, _VP, _VP, ctypes.c_int64,
                                     ctypes.c_double, ctypes.c_uint64, ctypes.c_int32, _VP, _VP,
                                     _VP, _VP]),
    "luma_hyper_rows": (ctypes.c_int, [_VP, ctypes.c_int64, ctypes.c_int32, _VP, _VP]),
    "luma_philox4x32": (None, [ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint32),
                               ctypes.POINTER(ctypes.c_uint32)]),
}


def load(path: str = LIB_PATH):
    """Load the HIP library (once) and bind every entry point."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise LumaLibraryError(
            f"{LIB_NAME} not found at {path}; build it with "
            "`python -c 'import luma_amd.build as b; b.build()'` (needs hipcc)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.luma_abi_version() != ABI_VERSION:
        raise LumaLibraryError(f"{LIB_NAME} ABI {lib.luma_abi_version()} != {ABI_VERSION}")
    check_layout(lib)
    _lib = lib
    return lib


def load_host():
    """The host bookkeeping module (luma_amd/_luma_host*.so, built with the
    library): pointer refresh of a re-used step table and the step counts.
    None (with a warning) when it is missing or was built against another
    torch (it reads tensor fields in its build's layout): the optimizer then
    rebuilds its step table on every step, which is slower for large
    parameter lists but gives the same results."""
    import warnings

    import torch

    try:
        from . import _luma_host
    except ImportError as e:
        warnings.warn(f"luma_amd._luma_host not loadable ({e}); LUMA rebuilds its step table "
                      "every step.  Build it with `python -m luma_amd.build`.")
        return None
    built = getattr(_luma_host, "torch_version", None)
    if built != torch.__version__:
        warnings.warn(f"luma_amd._luma_host was built against torch {built}, this is torch "
                      f"{torch.__version__}: not used (LUMA rebuilds its step table every "
                      "step).  Rebuild it with `python -m luma_amd.build`.")
        return None
    return _luma_host


def check_layout(lib) -> None:
    out = (ctypes.c_int32 * 8)()
    lib.luma_layout(out)
    want = [TENSOR_DTYPE.itemsize, CHUNK_DTYPE.itemsize, GROUP_DTYPE.itemsize,
            SCALE_INIT_DTYPE.itemsize, ctypes.sizeof(StepArgs), SLOT_BYTES, CHUNK_ELEMS]
    got = list(out)[:7]
    if got != want:
        raise LumaLibraryError(f"struct layout mismatch: library {got} vs python {want}")


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = _lib.luma_last_error().decode() if _lib is not None else ""
        raise LumaLibraryError(f"{what} failed ({rc}): {msg}")


def philox4x32(ctr, key):
    """Host Philox4x32-10 block from the library (no GPU needed)."""
    lib = load()
    c = (ctypes.c_uint32 * 4)(*[int(x) & 0xFFFFFFFF for x in ctr])
    k = (ctypes.c_uint32 * 2)(*[int(x) & 0xFFFFFFFF for x in key])
    o = (ctypes.c_uint32 * 4)()
    lib.luma_philox4x32(c, k, o)
    return [int(x) for x in o]
