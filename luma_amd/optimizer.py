"""``LUMA`` -- ``torch.optim.Optimizer`` front end over the HIP step.

Same public surface as the reference (src/luma_optimizer/optimizer.py:39-524):
``LUMA(params, lr, betas, eps, weight_decay, backend)``, ``step(closure)``,
``state_dict()`` / ``load_state_dict()``, ``export_adamw_state()``,
``import_adamw_state()`` and ``_base_seed``.  Per parameter the state holds
``step``, ``param_id``, ``Q_m`` and ``Q_w`` (int16, the parameter's shape);
the step count, ``S_m`` and ``S_v`` live on the device in the parameter's
slot (a private 512-byte buffer, the counterpart of the reference's
``_step_tensor`` / ``_new_grid``, optimizer.py:341-387) and appear in
``state_dict()``.

One ``step()`` is one multi-tensor launch sequence on the current stream
(luma_step in include/luma.h) with no host synchronisation.  Every per-step
quantity is derived on the device, so ``step()`` can be captured into a CUDA
(HIP) graph after one eager step and replayed: each replay is one more step.
``state[p]["step"]`` counts eager calls; ``state_dict()`` and
``export_adamw_state()`` read the device counts (and refresh it).  The stochastic
rounding draws come from Philox4x32-10 keyed by the reference's per-step seed
``((t << 32) | 2*param_id) ^ _base_seed`` (functional.py:99-106), or from
uniforms injected with ``inject_noise`` (used to compare against the
reference's own draws).
"""

from __future__ import annotations

import ctypes
from typing import Dict, Optional, Tuple

import numpy as np
import torch
from torch.optim import Optimizer

from . import _lib as L

from .config import SCALE_FLOOR_M  # noqa: F401  (re-exported constant)
from .config import STEP_CHUNK_MIN, STEP_TARGET_CHUNKS

_GRAD_CODES = {torch.float32: L.GRAD_F32, torch.bfloat16: L.GRAD_BF16, torch.float16: L.GRAD_F16}
_MASK64 = (1 << 64) - 1


def make_step_seed(base_seed: int, step: int, param_id: int) -> int:
    """functional.py:99-106 -- the per-(step, param) seed."""
    return ((step << 32) | (param_id * 2)) ^ base_seed


def _is_dense(t: torch.Tensor) -> bool:
    return (t.is_contiguous() or t.is_contiguous(memory_format=torch.channels_last)
            or t.is_contiguous(memory_format=torch.channels_last_3d))


def _ptr(t: Optional[torch.Tensor]) -> int:
    return 0 if t is None else t.data_ptr()


def shard_offset(t) -> int:
    """Index, in the whole parameter's flattened (row-major) elements, of the
    first element of a DTensor's local shard, when that shard is one
    contiguous range of the whole parameter (a ``Shard(0)`` placement, as
    FSDP2 uses, or any placement that leaves the shard whole); 0 for plain
    tensors.  The step keys its Philox counters on ``offset + local index``,
    so the shards of one parameter draw independent uniforms.  A shard that
    is not one contiguous range (e.g. ``Shard(1)`` of a matrix) keys on its
    local index, as the reference's Triton path does for every shard
    (triton_kernel.py:296-301)."""
    if not hasattr(t, "_local_tensor") or not hasattr(t, "device_mesh"):
        return 0
    try:
        from torch.distributed.tensor._utils import compute_local_shape_and_global_offset
    except ImportError:   # pragma: no cover - older torch
        return 0
    gshape = tuple(t.shape)
    lshape, goff = compute_local_shape_and_global_offset(gshape, t.device_mesh, t.placements)
    lshape, goff = tuple(lshape), tuple(goff)
    diff = [d for d in range(len(gshape)) if lshape[d] != gshape[d]]
    if diff:
        d0 = diff[0]
        # contiguous: every dim before d0 has extent 1, every dim after d0 is whole
        if any(gshape[d] != 1 for d in range(d0)) or any(lshape[d] != gshape[d]
                                                           for d in range(d0 + 1, len(gshape))):
            return 0
    off, stride = 0, 1
    for d in range(len(gshape) - 1, -1, -1):
        off += goff[d] * stride
        stride *= gshape[d]
    return int(off)


_ARENA_ALIGN = 128   # int16 elements: every Q tensor starts on a 256-byte boundary
# Smallest tensor given code summaries: pass 1 reads them only in whole
# iterations of a workgroup (256 threads x 8 elements).
_SUMMARY_MIN = 2048


def state_arena(params, device):
    """Q_m and Q_w for the given (dense) parameters as views of ONE int16
    allocation: parameter i's Q_m, then its Q_w, each 256-byte aligned and
    with the parameter's shape and strides.  Two allocations replace two
    per parameter, and a checkpoint of the state serialises one storage."""
    sizes = [-(-p.numel() // _ARENA_ALIGN) * _ARENA_ALIGN for p in params]
    arena = torch.empty(max(2 * sum(sizes), 1), dtype=torch.int16, device=device)
    storage = arena.untyped_storage()
    views, off = [], 0
    for p, n in zip(params, sizes):
        qm = torch.empty(0, dtype=torch.int16, device=device).set_(storage, off, p.shape, p.stride())
        qw = torch.empty(0, dtype=torch.int16, device=device).set_(storage, off + n, p.shape,
                                                                 p.stride())
        views.append((qm, qw))
        off += 2 * n
    return views


def summary_arena(params, device, chunk):
    """One code-summary array per parameter (int32, SUMMARY_WORDS words per
    chunk of `chunk` elements), as views of one allocation.  The step's pass 2
    writes them; the next step's pass 1 reads them to skip the codes of groups
    that cannot hold the tensor's maximum."""
    sizes = [-(-p.numel() // chunk) * L.SUMMARY_WORDS for p in params]
    arena = torch.empty(max(sum(sizes), 1), dtype=torch.int32, device=device)
    return list(arena.split(sizes)) if params else []


class _Engine:
    """Device-side tables of one optimizer: tensor, chunk and group tables and
    the chunk-maxima workspace.  Tables are uploaded only when their contents
    change, so a step whose parameters, gradients and hyper-parameters are
    those of the previous step launches with no host-to-device copy (and may
    be captured into a CUDA/HIP graph)."""

    TABLE_CACHE = 4   # device tensor tables kept for re-use

    def __init__(self, device: torch.device):
        self.lib = L.load()
        self.host = L.load_host()
        self.device = device
        self._tensor_key = None      # bytes of the uploaded tensor table
        self._tensor_src = None      # (table array, chunk setting) last uploaded or matched
        self._numel_key = None       # bytes of its numel column and chunk layout (chunk table)
        self._first = None           # first_chunk column of that layout
        self._chunk = L.CHUNK_ELEMS  # chunk length of the uploaded chunk table
        self.chunk_elems = 0         # fixed chunk length (a power of two), 0: chunk_for's choice
        self.small_tensors = True    # step tensors of <= SMALL_TENSOR elements a wavefront each
        self._small_chunks = 0       # trailing chunk records of such tensors (uploaded table)
        self.medium_tensors = True   # step tensors of <= MEDIUM_TENSOR elements one wavefront
                                     # each (inside the fast kernels' launches)
        self._medium_chunks = 0      # the records of such tensors, before the small ones
        self._d_tensors = None
        self._table_cache = {}       # tensor-table bytes -> device copy (most recent last)
        self._ptr_cache = {}         # sequence number -> (table, (n, 2) grad and param
                                     # pointers, device copy), least recent first
        self._ptr_seq = 0
        self._d_chunks = None
        self._n_chunks = 0
        self._group_key = None
        self._d_groups = None
        self._partials = None
        self._captured = []          # tables that a captured graph may read
        # torch.cuda.Event x4 (already recorded once) -> per-kernel timing
        self.profile_events = None

    # -- helpers ------------------------------------------------------------
    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def _upload(self, arr: np.ndarray) -> torch.Tensor:
        host = torch.from_numpy(arr.view(np.uint8).reshape(-1)).pin_memory()
        return host.to(self.device, non_blocking=True)

    def new_slots(self, n: int):
        """n zero-filled slots (step count 0) as views of one allocation."""
        block = torch.zeros((n, L.SLOT_BYTES), dtype=torch.uint8, device=self.device)
        return list(block.unbind(0))

    @staticmethod
    def _capture_error(what: str) -> RuntimeError:
        return RuntimeError(
            f"LUMA.step() under graph capture: {what} changed since the last eager step(). "
            "Run one eager step() with the same parameters, gradient tensors and "
            "hyper-parameters before capturing.")

    # -- entry points -------------------------------------------------------
    def chunk_for(self, numels: np.ndarray) -> int:
        """Chunk length of a step over tensors of these sizes: the largest power
        of two from CHUNK_ELEMS down to STEP_CHUNK_MIN with STEP_TARGET_CHUNKS
        chunks of it at most the set's total size.  Small sets get shorter
        chunks; so do sets of many tensors whose total is small, where one
        chunk per tensor in parameter order would leave the largest tensors'
        workgroups running alone at the end of the launch.  A set with at least
        STEP_TARGET_CHUNKS tensors above the wavefront-per-tensor limit fills
        the chip with one chunk per tensor: it takes a chunk as long as its
        largest tensor (at most CHUNK_ELEMS), and chunk_layout puts the
        largest tensors first.  The result does not depend on the length:
        every element is computed alone and the per-tensor maxima are exact."""
        if self.chunk_elems:
            return self.chunk_elems
        total = int(numels.sum())
        c = L.CHUNK_ELEMS
        while c > STEP_CHUNK_MIN and c * STEP_TARGET_CHUNKS > total:
            c //= 2
        big = numels[numels > self._wave_limit()]
        if len(big) >= STEP_TARGET_CHUNKS:
            while c < L.CHUNK_ELEMS and c < int(big.max()):
                c *= 2
        return c

    def table(self, rows) -> np.ndarray:
        """Tensor table of rows: (param, grad, q_m, q_w, u_m, u_w, slot, param_id,
        grad_code, group, elem_offset, summary) per tensor, chunks numbered
        consecutively."""
        n = len(rows)
        tt = np.zeros(n, dtype=L.TENSOR_DTYPE)
        numels = np.fromiter((r[0].numel() for r in rows), dtype=np.int64, count=n)
        c = self.chunk_for(numels)
        nch = (numels + c - 1) // c
        first = np.zeros(n, dtype=np.int64)
        np.cumsum(nch[:-1], out=first[1:])
        if int(nch.sum()) >= 2**31:
            raise ValueError("LUMA: too many chunks for one launch")
        tt["param"] = [r[0].data_ptr() for r in rows]
        tt["grad"] = [r[1].data_ptr() for r in rows]
        tt["q_m"] = [r[2].data_ptr() for r in rows]
        tt["q_w"] = [r[3].data_ptr() for r in rows]
        tt["u_m"] = [_ptr(r[4]) for r in rows]
        tt["u_w"] = [_ptr(r[5]) for r in rows]
        tt["slot"] = [r[6].data_ptr() for r in rows]
        tt["summary"] = [_ptr(r[11]) for r in rows]
        tt["summary_words"] = [0 if r[11] is None else r[11].numel() for r in rows]
        tt["numel"] = numels
        tt["param_id"] = [r[7] for r in rows]
        tt["elem_offset"] = [r[10] for r in rows]
        tt["grad_dtype"] = [r[8] for r in rows]
        tt["group"] = [r[9] for r in rows]
        tt["first_chunk"] = first
        return tt

    def launch(self, tt: np.ndarray, groups: np.ndarray, base_seed: int, noise_mode: int,
               flags: int = 0, scaling: Tuple[int, int] = (0, 0), same_table: bool = False,
               moved: bool = False, ptr_match=None):
        """One step over the tensors of table tt (luma_step), uploading only the
        tables whose contents changed since the previous launch.  With
        ``same_table`` the caller vouches that tt is the array of the previous
        launch, unchanged since: the comparison of its contents is skipped.
        With ``moved`` it vouches that tt is that array with only its gradient
        and parameter pointers rewritten: the device tables of earlier pointer
        sets are looked up by those two columns alone, and ``ptr_match`` (a
        key of pointer_candidates(tt)) names the set they equal when the
        caller has compared them already."""
        capturing = torch.cuda.is_current_stream_capturing()
        n = len(tt)
        setting = (self.chunk_elems, self._small_limit(), self._medium_limit())
        same_src = (self._tensor_src is not None and self._tensor_src[0] is tt
                    and self._tensor_src[1] == setting)
        if moved and same_src:
            self._match_pointers(tt, capturing, match=ptr_match)
        elif not (same_table and same_src):
            self._tensor_src = None     # stays unset if the upload fails
            self._match_table(tt, capturing)
            self._tensor_src = (tt, setting)
        n_chunks = self._n_chunks
        gkey = groups.tobytes()
        if gkey != self._group_key:
            if capturing:
                raise self._capture_error("a param group's hyper-parameters")
            self._d_groups = self._upload(groups)
            self._group_key = gkey
        need = max(self.lib.luma_workspace_bytes(n_chunks) // 4, 4)
        if self._partials is None or self._partials.numel() < need:
            if capturing:
                raise self._capture_error("the chunk count")
            self._partials = torch.empty(need, dtype=torch.float32, device=self.device)
        if capturing:
            tables = (self._d_tensors, self._d_chunks, self._d_groups, self._partials)
            if not self._captured or any(x is not y for x, y in zip(self._captured[-1], tables)):
                self._captured.append(tables)
        args = L.StepArgs(
            tensors=self._d_tensors.data_ptr(), n_tensors=n, n_chunks=n_chunks,
            chunks=self._d_chunks.data_ptr(), groups=self._d_groups.data_ptr(),
            partials=self._partials.data_ptr(),
            base_seed=base_seed & _MASK64, noise_mode=noise_mode, flags=flags,
            chunk_elems=self._chunk, small_chunks=self._small_chunks,
            medium_chunks=self._medium_chunks,
            scaling=L.Scaling(scaling[0] or None, scaling[1] or None))
        if self.profile_events is None:
            L.check(self.lib.luma_step(ctypes.byref(args), self._stream()), "luma_step")
        else:
            evs = (ctypes.c_void_p * 4)(*[e.cuda_event for e in self.profile_events])
            L.check(self.lib.luma_step_profiled(ctypes.byref(args), self._stream(), evs),
                    "luma_step_profiled")

    def _small_limit(self) -> int:
        """Largest tensor stepped a wavefront each by the exact kernels (0: none)."""
        return int(L.SMALL_TENSOR) if self.small_tensors else 0

    def _medium_limit(self) -> int:
        """Largest tensor stepped one wavefront each by the fast kernels (0: none)."""
        return int(L.MEDIUM_TENSOR) if self.medium_tensors else 0

    def _wave_limit(self) -> int:
        """Largest tensor stepped by a single wavefront, either route."""
        return max(self._small_limit(), self._medium_limit())

    def chunk_layout(self, numels: np.ndarray, c: int):
        """Chunk table layout of tensors of these sizes at chunk length c: the
        first chunk of every tensor, the chunk records (tensor, index), and
        the number of records of medium and of small tensors, which come last
        in that order (luma.h, LumaStepArgs.medium_chunks / small_chunks).
        Tensors of at most SMALL_TENSOR elements are stepped a wavefront per
        chunk by the exact kernels, and those above it and of at most
        MEDIUM_TENSOR elements (and one chunk) one wavefront each by the fast
        kernels, four to a workgroup; each run is ordered largest first, so the four
        wavefronts of a small-tensor workgroup step tensors of about one size
        and every launch ends on its shortest work.  The others keep their
        order, unless there are STEP_TARGET_CHUNKS of them or more (chunk_for
        gives such a set one chunk per tensor): then the largest come first.
        Ties keep their order."""
        n = len(numels)
        nch = (numels + c - 1) // c
        small = numels <= self._small_limit()
        medium = ~small & (numels <= min(self._medium_limit(), c))
        big = np.nonzero(~small & ~medium)[0]
        if len(big) >= STEP_TARGET_CHUNKS:
            big = big[np.argsort(-numels[big], kind="stable")]
        mid = np.nonzero(medium)[0]
        mid = mid[np.argsort(-numels[mid], kind="stable")]
        little = np.nonzero(small)[0]
        little = little[np.argsort(-numels[little], kind="stable")]
        order = np.concatenate([big, mid, little])
        n_small = int(nch[small].sum())
        n_medium = int(nch[medium].sum())
        nch_o = nch[order]
        first_o = np.zeros(n, dtype=np.int64)
        np.cumsum(nch_o[:-1], out=first_o[1:])
        first = np.empty(n, dtype=np.int64)
        first[order] = first_o
        n_chunks = int(nch.sum())
        ch = np.empty(n_chunks, dtype=L.CHUNK_DTYPE)
        ch["tensor"] = np.repeat(order.astype(np.int32), nch_o)
        ch["index"] = np.arange(n_chunks, dtype=np.int64) - np.repeat(first_o, nch_o)
        return first, ch, n_small, n_medium

    def _match_table(self, tt: np.ndarray, capturing: bool):
        """Upload tt (and its chunk table) unless the device holds it already."""
        # first_chunk follows the chunk length and layout of this launch (a
        # cached table may have been built for another)
        numels = tt["numel"]
        c = self.chunk_for(numels)
        nkey = (numels.tobytes() + c.to_bytes(4, "little")
                + self._small_limit().to_bytes(8, "little")
                + self._medium_limit().to_bytes(8, "little"))
        if nkey != self._numel_key:
            if capturing:
                raise self._capture_error("the parameter or gradient set")
            first, ch, n_small, n_medium = self.chunk_layout(numels, c)
            tt["first_chunk"] = first
            key = tt.tobytes()
            self._d_chunks = self._upload(ch)
            self._n_chunks = len(ch)
            self._small_chunks = n_small
            self._medium_chunks = n_medium
            self._chunk = c
            self._numel_key = nkey
            self._first = first
        else:
            tt["first_chunk"] = self._first
            key = tt.tobytes()
        if key != self._tensor_key:
            # the last few uploaded tables stay on the device: a loop whose
            # gradients alternate between buffers re-uses them, no upload
            cached = self._table_cache.pop(key, None)
            if cached is None:
                if capturing:
                    raise self._capture_error("the parameter or gradient set")
                cached = self._upload(tt)
            self._table_cache[key] = cached
            while len(self._table_cache) > self.TABLE_CACHE:
                self._table_cache.pop(next(iter(self._table_cache)))
            self._d_tensors = cached
            self._tensor_key = key

    def _same_pointers(self, tt: np.ndarray, cols: np.ndarray) -> bool:
        """Whether tt's gradient and parameter columns equal cols ((n, 2))."""
        if len(cols) != len(tt):
            return False
        if self.host is not None:
            return self.host.same_pointers(tt.ctypes.data, tt.dtype.itemsize,
                                           tt.dtype.fields["grad"][1],
                                           tt.dtype.fields["param"][1], cols)
        return bool(np.array_equal(cols[:, 0], tt["grad"])
                    and np.array_equal(cols[:, 1], tt["param"]))

    def pointer_candidates(self, tt: np.ndarray):
        """(key, (n, 2) pointer array) of the cached pointer sets of tt, most
        recent first (at most eight): what a planned step's refresh compares
        the new pointers with while it writes them."""
        out = []
        for k in reversed(self._ptr_cache):
            ent = self._ptr_cache[k]
            if ent[0] is tt:
                out.append((k, ent[1]))
                if len(out) == 8:
                    break
        return out

    def _match_pointers(self, tt: np.ndarray, capturing: bool, match=None):
        """Device table for tt, which differs from the table last matched for
        it in its gradient and parameter pointers only (a planned step whose
        gradients moved, e.g. a loop that alternates gradient buffers): a
        table uploaded for the same pointers is re-used, so such a loop
        uploads each table once.  ``match``: the key of a cached set that the
        caller found equal to tt's two columns (the host module's refresh
        compares them while it writes them).  Otherwise the cached sets of tt
        are compared here, most recent first; the host module's comparison
        stops at the first row that differs, so a set that does not match
        costs about one row."""
        key = None
        if match is not None and match in self._ptr_cache and self._ptr_cache[match][0] is tt:
            key = match
        else:
            for k in reversed(self._ptr_cache):
                ent = self._ptr_cache[k]
                if ent[0] is tt and self._same_pointers(tt, ent[1]):
                    key = k
                    break
        if key is None:
            if capturing:
                raise self._capture_error("the parameter or gradient set")
            cols = np.empty((len(tt), 2), dtype=np.uint64)
            cols[:, 0] = tt["grad"]
            cols[:, 1] = tt["param"]
            self._ptr_seq += 1
            key, ent = self._ptr_seq, (tt, cols, self._upload(tt))
        else:
            ent = self._ptr_cache.pop(key)
        self._ptr_cache[key] = ent
        while len(self._ptr_cache) > self.TABLE_CACHE:
            self._ptr_cache.pop(next(iter(self._ptr_cache)))
        self._d_tensors = ent[2]
        self._tensor_key = None   # (the bytes key of _match_table no longer applies)

    def set_scales(self, items):
        """items: list of (slot tensor, step, S_m, S_v, eps)."""
        arr = np.zeros(len(items), dtype=L.SCALE_INIT_DTYPE)
        arr["slot"] = [i[0].data_ptr() for i in items]
        arr["step"] = [i[1] for i in items]
        arr["s_m"] = [i[2] for i in items]
        arr["s_v"] = [i[3] for i in items]
        arr["eps"] = [i[4] for i in items]
        d = self._upload(arr)
        L.check(self.lib.luma_set_scales(d.data_ptr(), len(items), self._stream()),
                "luma_set_scales")

    def get_scales(self, slots):
        """Returns a list of (step, S_m, S_v) as Python numbers (synchronises)."""
        n = len(slots)
        d_ptrs = self._upload(np.asarray([s.data_ptr() for s in slots], dtype=np.uint64))
        scales = torch.empty(2 * n, dtype=torch.float64, device=self.device)
        steps = torch.empty(n, dtype=torch.int64, device=self.device)
        L.check(self.lib.luma_get_scales(d_ptrs.data_ptr(), n, scales.data_ptr(),
                                         steps.data_ptr(), self._stream()), "luma_get_scales")
        sc = scales.cpu().tolist()
        st = steps.cpu().tolist()
        return [(st[i], sc[2 * i], sc[2 * i + 1]) for i in range(n)]

    def decode(self, q_m, q_w, slot, eps, m_out, v_out):
        L.check(self.lib.luma_decode(q_m.data_ptr(), q_w.data_ptr(), q_m.numel(),
                                     slot.data_ptr(), float(eps), m_out.data_ptr(),
                                     v_out.data_ptr(), self._stream()), "luma_decode")

    def quantize(self, m, v, q_m, q_w, slot, step, eps, seed, noise_mode, u_m, u_w):
        n = m.numel()
        nch = (n + L.CHUNK_ELEMS - 1) // L.CHUNK_ELEMS
        ws = torch.empty(max(2 * nch, 2), dtype=torch.float32, device=self.device)
        L.check(self.lib.luma_quantize(m.data_ptr(), v.data_ptr(), n, q_m.data_ptr(),
                                       q_w.data_ptr(), slot.data_ptr(), step, float(eps),
                                       seed & _MASK64, noise_mode, _ptr(u_m), _ptr(u_w),
                                       ws.data_ptr(), self._stream()), "luma_quantize")


class _Plan:
    """The tensor table of the previous step, for re-use.

    A step may re-use it when the parameter list is the same objects, the
    same parameters have a gradient, and every gradient is a plain dense
    tensor of the planned dtype, strides and device.  Then only the gradient
    and parameter pointers are re-read, by the host module (_luma_host.refresh),
    and nothing is uploaded unless they moved.
    Invalidated by load_state_dict, import_adamw_state and add_param_group.
    """

    __slots__ = ("all_params", "has_grad", "work_idx", "layout_at", "layout", "gdtypes",
                 "device_index", "states", "tt", "host", "chunk_setting")

    _FIELDS = (L.TENSOR_DTYPE.itemsize, L.TENSOR_DTYPE.fields["grad"][1],
               L.TENSOR_DTYPE.fields["param"][1])

    def __init__(self, param_groups, work, rows, states, tt, host):
        self.all_params = [p for g in param_groups for p in g["params"]]
        self.has_grad = np.fromiter((p.grad is not None for p in self.all_params),
                                    dtype=np.uint8, count=len(self.all_params))
        self.work_idx = np.fromiter((w[4] for w in work), dtype=np.int64, count=len(work))
        # per row [ndim, sizes..., strides...] of the parameter (and of its
        # gradient and Q_m, which the step checked against it)
        lay, at = [], []
        for r in rows:
            at.append(len(lay))
            lay.append(r[0].dim())
            lay.extend(r[0].shape)
            lay.extend(r[0].stride())
        self.layout_at = np.asarray(at, dtype=np.int64)
        self.layout = np.asarray(lay, dtype=np.int64)
        self.gdtypes = np.ascontiguousarray(tt["grad_dtype"], dtype=np.int32)
        self.device_index = rows[0][0].get_device()
        self.states = states
        self.tt = tt
        self.host = host
        # the engine's fixed chunk length when planned: the code summaries in
        # tt were sized for the chunk length it gave
        self.chunk_setting = None

    @staticmethod
    def usable(work, rows) -> bool:
        """Whether the step just built from `work` can be re-used: every
        gradient went in as the parameter's own .grad tensor (no dtype or
        layout conversion, no DTensor unwrapping)."""
        return all(type(w[1]) is torch.nn.Parameter or type(w[1]) is torch.Tensor
                   for w in work) and all(
            r[1] is w[1].grad and type(r[1]) is torch.Tensor for w, r in zip(work, rows))

    def refresh(self, param_groups, cands=None) -> int:
        """0: the plan no longer applies; 1: it applies and the table is
        unchanged; 2: it applies with new gradient or parameter pointers
        (written into the table).  With cands (a list of (n, 2) pointer
        arrays), bit 2 + k of the result is set when the new pointers equal
        cands[k]'s."""
        return self.host.refresh(param_groups, self.all_params, self.has_grad, self.work_idx,
                                 self.layout_at, self.layout, self.gdtypes, self.tt.ctypes.data,
                                 *self._FIELDS, self.device_index, cands)


class LUMA(Optimizer):
    r"""LUMA: Log-space Unbiased Momentum AdamW on the MI355X HIP backend.

    Stores two int16 tensors per parameter (signed log-grid momentum ``Q_m``,
    unsigned log-grid preconditioner ``Q_w``): 4 bytes/param of state.

    ``backend`` accepts the reference's names ``"auto"``, ``"triton"`` and
    ``"pytorch"`` (optimizer.py:98-113), and ``"hip"``; every name selects the
    HIP library, whose stochastic rounding draws from Philox (as the
    reference's GPU backend does) rather than from the CPU generator of its
    PyTorch backend.  Parameters must be float32 and live on a ROCm GPU;
    gradients may be float32, bfloat16 or float16 (others are promoted to
    float32 first).
    """

    _BACKENDS = ("auto", "triton", "pytorch", "hip")

    # torch.amp.GradScaler: instead of unscaling the gradients and checking
    # them on the host before calling step(), the scaler sets
    # self.grad_scale / self.found_inf (device tensors) and calls step();
    # the kernels unscale each gradient as unscale_ would store it and skip
    # the whole step on the device when found_inf is nonzero.
    _step_supports_amp_scaling = True

    def __init__(self, params, lr: float = 1e-3, betas: Tuple[float, float] = (0.9, 0.999),
                 eps: float = 1e-8, weight_decay: float = 0.01, backend: str = "auto"):
        # optimizer.py:80-89
        if lr < 0.0:
            raise ValueError(f"Invalid learning rate: {lr}")
        if eps <= 0.0:
            raise ValueError(f"Invalid epsilon: {eps}")
        if not 0.0 <= betas[0] < 1.0:
            raise ValueError(f"Invalid beta1: {betas[0]}")
        if not 0.0 <= betas[1] < 1.0:
            raise ValueError(f"Invalid beta2: {betas[1]}")
        if weight_decay < 0.0:
            raise ValueError(f"Invalid weight_decay: {weight_decay}")
        defaults = dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay)
        super().__init__(params, defaults)
        # optimizer.py:94-96: one int64 draw from the global CPU generator
        self._base_seed: int = int(
            torch.randint(-(2**63), 2**63 - 1, (1,), dtype=torch.int64).item())
        if backend not in self._BACKENDS:
            raise ValueError(f"Invalid backend: {backend}. Expected one of "
                             "{'auto', 'triton', 'pytorch', 'hip'} (every name selects the HIP "
                             "library).")
        self._engine: Optional[_Engine] = None
        self._noise: Optional[Dict[int, Tuple[torch.Tensor, torch.Tensor]]] = None
        self._noise_strict = True
        self._flags = 0
        self._summaries = True   # pass per-parameter code summaries to the step
        self._plan: Optional[_Plan] = None
        self._scaling_keep = []

    # ------------------------------------------------------------------
    #  Helpers
    # ------------------------------------------------------------------
    @staticmethod
    def _unwrap_tensor(t):
        """optimizer.py:399-407: DTensor -> local shard."""
        if t is None:
            return None
        return t._local_tensor if hasattr(t, "_local_tensor") else t

    def _get_engine(self, device: torch.device) -> _Engine:
        if self._engine is None:
            if device.type != "cuda":
                raise RuntimeError(f"LUMA (HIP) steps parameters on a ROCm GPU; got device {device}")
            self._engine = _Engine(device)
        elif self._engine.device != device:
            raise RuntimeError("LUMA (HIP): all parameters must be on one device "
                               f"({self._engine.device} vs {device})")
        return self._engine

    def inject_noise(self, noise: Dict[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]],
                     strict: bool = True):
        """Use the given uniforms (u_m, u_w), float32 in [0, 1) with each parameter's
        shape and device, for the next ``step()`` or ``import_adamw_state()``
        instead of Philox draws.  With ``strict`` every parameter updated by
        that call needs an entry; otherwise parameters without one draw from
        Philox as usual."""
        self._noise = {id(p): (u_m, u_w) for p, (u_m, u_w) in noise.items()}
        self._noise_strict = strict

    def _take_noise(self, p, like):
        if self._noise is None:
            return None, None
        if id(p) not in self._noise:
            if not self._noise_strict:
                return None, None
            raise ValueError("LUMA.inject_noise: missing uniforms for a parameter")
        u_m, u_w = self._noise[id(p)]
        out = []
        for u in (u_m, u_w):
            u = u.to(device=like.device, dtype=torch.float32)
            if u.shape != like.shape:
                raise ValueError("LUMA.inject_noise: uniform shape mismatch")
            if u.stride() != like.stride():
                u = torch.empty_like(like, dtype=torch.float32).copy_(u)
            out.append(u)
        return out[0], out[1]

    def _scaling(self, device) -> Tuple[int, int]:
        """Device pointers of GradScaler's grad_scale / found_inf (0 if unset).
        The tensors are kept on self until the next step so that they outlive
        the launch."""
        keep = []
        ptrs = []
        for name in ("grad_scale", "found_inf"):
            t = getattr(self, name, None)
            if t is None:
                ptrs.append(0)
                continue
            if not isinstance(t, torch.Tensor) or t.numel() != 1:
                raise ValueError(f"LUMA: {name} must be a one-element tensor")
            if t.dtype != torch.float32 or t.device != device:
                t = t.to(device=device, dtype=torch.float32)
            keep.append(t)
            ptrs.append(t.data_ptr())
        self._scaling_keep = keep
        return ptrs[0], ptrs[1]

    def _group_table(self) -> np.ndarray:
        """Hyper-parameters of every param group as the Python doubles the
        reference computes with (optimizer.py:80-92); the device derives the
        per-step scalars from them."""
        arr = np.zeros(len(self.param_groups), dtype=L.GROUP_DTYPE)
        for i, g in enumerate(self.param_groups):
            b1, b2 = g["betas"]
            arr[i] = (float(g["lr"]), float(b1), float(b2), float(g["eps"]),
                      float(g["weight_decay"]), 0.0)
        return arr

    # ------------------------------------------------------------------
    #  Checkpoint: portable save / load  (optimizer.py:119-183)
    # ------------------------------------------------------------------
    def _read_slots(self, states):
        """Device step counts and scales of the given states (one sync); also
        refreshes each state's host ``step``."""
        vals = self._engine.get_scales([s["_slot"] for s in states])
        for s, (step, _, _) in zip(states, vals):
            s["step"] = step
        return vals

    def state_dict(self) -> dict:
        raw = super().state_dict()
        keys = [idx for idx, s in raw["state"].items() if "_slot" in s]
        vals = self._read_slots([raw["state"][k] for k in keys]) if keys else []
        clean = {idx: {k: v for k, v in s.items() if not k.startswith("_")}
                 for idx, s in raw["state"].items()}
        for idx, (step, sm, sv) in zip(keys, vals):
            clean[idx]["step"] = step
            clean[idx]["S_m"] = sm
            clean[idx]["S_v"] = sv
        raw["state"] = clean
        raw["_base_seed"] = self._base_seed
        return raw

    def add_param_group(self, param_group: dict) -> None:
        self._plan = None
        super().add_param_group(param_group)

    def load_state_dict(self, state_dict: dict) -> None:
        self._plan = None
        self._base_seed = state_dict.get("_base_seed", self._base_seed)
        super().load_state_dict(state_dict)
        pending = []
        for group in self.param_groups:
            for p in group["params"]:
                state = self.state[p]
                if len(state) == 0:
                    continue
                param = self._unwrap_tensor(p)
                for key in ("Q_m", "Q_w"):
                    # torch's load casts state tensors of a float parameter to the
                    # parameter's dtype (Optimizer._process_value_according_to_param_policy);
                    # the codes are exact integers, so restore int16 in the param's layout.
                    if key in state:
                        q = state[key]
                        if (q.dtype != torch.int16 or q.device != param.device
                                or q.stride() != param.stride()):
                            fixed = torch.empty_like(param, dtype=torch.int16)
                            fixed.copy_(q.reshape(param.shape))
                            state[key] = fixed
                if "S_m" not in state:
                    raise ValueError("LUMA.load_state_dict: state without S_m/S_v")
                pending.append((p, param, state, group["eps"]))
        if not pending:
            return
        engine = self._get_engine(pending[0][1].device)
        items = []
        for (_, param, state, eps), slot in zip(pending, engine.new_slots(len(pending))):
            self._get_engine(param.device)
            state["_slot"] = slot
            state["step"] = int(state["step"])
            items.append((slot, state["step"], float(state.pop("S_m")),
                          float(state.pop("S_v")), eps))
        engine.set_scales(items)

    # ------------------------------------------------------------------
    #  AdamW interop  (optimizer.py:189-335)
    # ------------------------------------------------------------------
    def export_adamw_state(self) -> dict:
        param_to_idx: Dict[int, int] = {}
        for group in self.param_groups:
            for p in group["params"]:
                param_to_idx[id(p)] = len(param_to_idx)
        adamw_state: dict = {}
        live = [self.state[p] for g in self.param_groups for p in g["params"]
                if "_slot" in self.state[p]]
        if live:
            self._read_slots(live)
        for group in self.param_groups:
            eps = group["eps"]
            for p in group["params"]:
                state = self.state[p]
                if len(state) == 0:
                    continue
                param = self._unwrap_tensor(p)
                engine = self._get_engine(param.device)
                if state["Q_m"].shape != param.shape or state["Q_w"].shape != param.shape:
                    raise ValueError("LUMA.export_adamw_state: the codes do not match their "
                                     f"parameter ({tuple(state['Q_m'].shape)} vs "
                                     f"{tuple(param.shape)})")
                exp_avg = torch.empty_like(param, dtype=torch.float32)
                exp_avg_sq = torch.empty_like(param, dtype=torch.float32)
                engine.decode(state["Q_m"], state["Q_w"], state["_slot"], eps,
                              exp_avg, exp_avg_sq)
                adamw_state[param_to_idx[id(p)]] = {
                    "step": torch.tensor(float(state["step"])),
                    "exp_avg": exp_avg,
                    "exp_avg_sq": exp_avg_sq,
                }
        param_groups = []
        for group in self.param_groups:
            pg = {k: v for k, v in group.items() if k != "params"}
            pg["params"] = [param_to_idx[id(p)] for p in group["params"]]
            param_groups.append(pg)
        return {"state": adamw_state, "param_groups": param_groups}

    def import_adamw_state(self, adamw_sd: dict) -> None:
        self._plan = None
        all_params = []
        group_of = {}
        for group in self.param_groups:
            for p in group["params"]:
                group_of[len(all_params)] = group
                all_params.append(p)
        for idx_key, s in adamw_sd["state"].items():
            idx = int(idx_key) if isinstance(idx_key, str) else idx_key
            if idx >= len(all_params):
                raise ValueError(f"AdamW state has index {idx} but LUMA only has "
                                 f"{len(all_params)} parameters")
            p = all_params[idx]
            group = group_of[idx]
            step_val = s["step"]
            step = int(step_val.item() if isinstance(step_val, torch.Tensor) else step_val)
            param = self._unwrap_tensor(p)
            engine = self._get_engine(param.device)
            m = torch.empty_like(param, dtype=torch.float32).copy_(s["exp_avg"])
            v = torch.empty_like(param, dtype=torch.float32).copy_(s["exp_avg_sq"])
            q_m = torch.empty_like(param, dtype=torch.int16)
            q_w = torch.empty_like(param, dtype=torch.int16)
            state = self.state[p]
            slot = state["_slot"] if "_slot" in state else engine.new_slots(1)[0]
            u_m, u_w = self._take_noise(p, param)
            noise_mode = L.NOISE_PHILOX if u_m is None else L.NOISE_INJECTED
            seed = make_step_seed(self._base_seed, 0, idx)   # optimizer.py:315-317
            engine.quantize(m, v, q_m, q_w, slot, step, group["eps"], seed, noise_mode, u_m, u_w)
            state["step"] = step
            state["param_id"] = idx
            state["Q_m"] = q_m
            state["Q_w"] = q_w
            state["_slot"] = slot
        self._noise = None

    # ------------------------------------------------------------------
    #  Main entry point  (optimizer.py:413-524)
    # ------------------------------------------------------------------
    # Not traced by dynamo: under torch.compile the call is a graph break and
    # runs as is (table bookkeeping in Python, then three kernel launches).
    @torch.compiler.disable
    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()

        plan = self._plan
        if (plan is not None and self._noise is None
                and plan.chunk_setting == self._engine.chunk_elems):
            eng = self._engine
            cands = eng.pointer_candidates(plan.tt)
            res = plan.refresh(self.param_groups, [c for _, c in cands] if cands else None)
            r, same = res & 3, res >> 2
            match = next((k for i, (k, _) in enumerate(cands) if (same >> i) & 1), None)
            if r:
                self._engine.launch(plan.tt, self._group_table(), self._base_seed,
                                    L.NOISE_PHILOX, self._flags,
                                    self._scaling(self._engine.device), same_table=(r == 1),
                                    moved=(r == 2), ptr_match=match)
                plan.host.bump_steps(plan.states)
                return loss
        self._plan = None

        work = []
        param_idx = 0
        for gi, group in enumerate(self.param_groups):
            for p in group["params"]:
                param_idx += 1
                if p.grad is None:
                    continue
                param = self._unwrap_tensor(p)
                grad = self._unwrap_tensor(p.grad)
                if param.numel() == 0:
                    continue
                if grad.is_sparse:
                    raise RuntimeError("LUMA does not support sparse gradients")
                if param.dtype != torch.float32:
                    raise ValueError(
                        f"LUMA requires float32 parameters (got {param.dtype}). "
                        f"Use torch.amp.autocast() or FSDP MixedPrecision "
                        f"instead of casting model weights to a reduced dtype.")
                if not param.is_cuda:
                    raise RuntimeError(
                        f"LUMA (HIP) steps parameters on a ROCm GPU; got device {param.device}")
                if not _is_dense(param):
                    raise ValueError("LUMA requires dense (contiguous) parameters")
                work.append((gi, p, param, grad, param_idx - 1))
        if not work:
            self._noise = None
            return loss

        engine = self._get_engine(work[0][2].device)
        noise_mode = L.NOISE_INJECTED if self._noise is not None else L.NOISE_PHILOX
        capturing = torch.cuda.is_current_stream_capturing()
        fresh = [self.state[w[1]] for w in work if "_slot" not in self.state[w[1]]]
        if fresh:
            if capturing:
                raise engine._capture_error("the set of parameters with optimizer state")
            for state, slot in zip(fresh, engine.new_slots(len(fresh))):
                state["_slot"] = slot
        no_q = [(self.state[w[1]], w[2]) for w in work if "Q_m" not in self.state[w[1]]]
        if no_q:
            if capturing:
                raise engine._capture_error("the set of parameters with optimizer state")
            for (state, _), (qm, qw) in zip(no_q, state_arena([p for _, p in no_q],
                                                              engine.device)):
                state["Q_m"] = qm
                state["Q_w"] = qw
        # code summaries: SUMMARY_WORDS words per chunk at this step's chunk length
        chunk = engine.chunk_for(np.fromiter((w[2].numel() for w in work), dtype=np.int64,
                                             count=len(work)))
        # (a tensor below one whole 2048-element iteration, or stepped by a
        # single wavefront, never reads a summary: it gets none)
        least = max(_SUMMARY_MIN, engine._wave_limit() + 1)
        no_summ = [(self.state[w[1]], w[2]) for w in work
                   if w[2].numel() >= least and (
                       self.state[w[1]].get("_summary") is None
                       or self.state[w[1]]["_summary"].numel() < -(-w[2].numel() // chunk)
                       * L.SUMMARY_WORDS)]
        if no_summ and not capturing:   # (under capture, a short array is only used less)
            for (state, _), sm in zip(no_summ, summary_arena([p for _, p in no_summ],
                                                             engine.device, chunk)):
                state["_summary"] = sm
        rows, states = [], []
        for gi, p, param, grad, pidx in work:
            self._get_engine(param.device)   # one device for all parameters
            state = self.state[p]
            if "step" not in state:
                state["step"] = 0
                state["param_id"] = pidx
            states.append(state)
            for key in ("Q_m", "Q_w"):
                q = state[key]
                if (q.dtype != torch.int16 or q.shape != param.shape
                        or q.stride() != param.stride() or q.device != param.device):
                    raise ValueError(
                        f"LUMA: state {key!r} ({tuple(q.shape)}, {q.dtype}) does not match its "
                        f"parameter ({tuple(param.shape)}); was the parameter replaced after "
                        "the optimizer state was created?")
            code = _GRAD_CODES.get(grad.dtype)
            if code is None:
                grad = grad.float()
                code = L.GRAD_F32
            if grad.device != param.device:
                grad = grad.to(param.device)
            if grad.stride() != param.stride() or not _is_dense(grad):
                grad = torch.empty_like(param, dtype=grad.dtype).copy_(grad)
            u_m, u_w = self._take_noise(p, param)
            summ = (state.get("_summary") if self._summaries and param.numel() >= least
                    else None)
            rows.append((param, grad, state["Q_m"], state["Q_w"], u_m, u_w, state["_slot"],
                         state["param_id"], code, gi, shard_offset(p), summ))
        tt = engine.table(rows)
        engine.launch(tt, self._group_table(), self._base_seed, noise_mode, self._flags,
                      self._scaling(engine.device))
        # host count of step() calls; the kernels use the slot's device count
        for state in states:
            state["step"] += 1
        if noise_mode == L.NOISE_PHILOX and engine.host is not None and _Plan.usable(work, rows):
            self._plan = _Plan(self.param_groups, work, rows, states, tt, engine.host)
            self._plan.chunk_setting = engine.chunk_elems
        self._noise = None
        return loss
