"""The host bookkeeping module (luma_amd._luma_host) on the CPU: the step
counts and the plan checks that need no device tensors."""

import numpy as np
import pytest
import torch

from luma_amd import _lib as L

H = L.load_host()


def test_bump_steps_counts_every_state():
    states = [{"step": 5, "param_id": i} for i in range(1000)]
    states += [{"step": 0}, {"step": 2**40}, {"step": 5}]
    H.bump_steps(states)
    H.bump_steps(states)
    assert [s["step"] for s in states[:1000]] == [7] * 1000
    assert [s["step"] for s in states[1000:]] == [2, 2**40 + 2, 7]
    assert [s["param_id"] for s in states[:1000]] == list(range(1000))
    # the same state dict twice in the list is counted twice, as a Python loop would
    d = {"step": 1}
    H.bump_steps([d, d])
    assert d["step"] == 3


def test_bump_steps_rejects_missing_count():
    states = [{"step": 1}, {"param_id": 0}]
    with pytest.raises(KeyError):
        H.bump_steps(states)
    assert states[0]["step"] == 2   # dicts before the bad one were counted
    with pytest.raises(TypeError):
        H.bump_steps([{"step": 1}, [1]])


def _layout(ps):
    lay, at = [], []
    for p in ps:
        at.append(len(lay))
        lay += [p.dim(), *p.shape, *p.stride()]
    return at, lay


def _refresh(groups, planned, has_grad, work_idx, gdtypes, tt, layout=None, device=0):
    f = L.TENSOR_DTYPE.fields
    at, lay = layout or _layout([planned[j] for j in work_idx])
    return H.refresh(groups, planned, np.asarray(has_grad, dtype=np.uint8),
                     np.asarray(work_idx, dtype=np.int64), np.asarray(at, dtype=np.int64),
                     np.asarray(lay, dtype=np.int64), np.asarray(gdtypes, dtype=np.int32),
                     tt.ctypes.data, L.TENSOR_DTYPE.itemsize, f["grad"][1], f["param"][1],
                     device)


def test_refresh_rejects_a_changed_parameter_list():
    ps = [torch.zeros(4, requires_grad=True) for _ in range(3)]
    tt = np.zeros(3, dtype=L.TENSOR_DTYPE)
    groups = [{"params": ps}]
    # planned list of other objects, or of another length
    assert _refresh(groups, list(reversed(ps)), [0, 0, 0], [], [], tt) == 0
    assert _refresh(groups, ps[:2], [0, 0], [], [], tt) == 0
    assert _refresh(groups + [{"params": [torch.zeros(1)]}], ps, [0, 0, 0], [], [], tt) == 0
    assert _refresh([{"params": tuple(ps)}], ps, [0, 0, 0], [], [], tt) == 0
    # malformed plans: rows out of range or not increasing, bad layouts,
    # arrays of the wrong length
    assert _refresh(groups, ps, [0, 0, 0], [7], [0], tt, layout=([0], [1, 4, 1])) == 0
    assert _refresh(groups, ps, [0, 0, 0], [1, 0], [0, 0], tt) == 0
    assert _refresh(groups, ps, [0, 0, 0], [0], [0], tt, layout=([2], [1, 4, 1])) == 0
    assert _refresh(groups, ps, [0, 0, 0], [0], [0], tt, layout=([0], [5, 4, 1])) == 0
    assert _refresh(groups, ps, [0, 0], [], [], tt) == 0
    assert not tt["grad"].any() and not tt["param"].any()


def test_refresh_checks_the_gradient_pattern():
    ps = [torch.zeros(4, requires_grad=True) for _ in range(3)]
    tt = np.zeros(3, dtype=L.TENSOR_DTYPE)
    groups = [{"params": ps}]
    # no gradients, as planned: a valid plan with no rows
    assert _refresh(groups, ps, [0, 0, 0], [], [], tt) == 1
    # a gradient appeared
    ps[1].grad = torch.zeros(4)
    assert _refresh(groups, ps, [0, 0, 0], [], [], tt) == 0
    # a planned gradient is missing
    assert _refresh(groups, ps, [1, 1, 0], [], [], tt) == 0
    # an object of another type in the planned place
    assert _refresh([{"params": [ps[0], [1], ps[2]]}], [ps[0], [1], ps[2]], [0, 0, 0], [], [],
                    tt) == 0
    assert _refresh([{"params": []}], [], [], [], [], tt) == 1


def test_refresh_rejects_host_tensors():
    """The step runs on the GPU: a CPU parameter never matches a plan."""
    ps = [torch.zeros(4, requires_grad=True)]
    ps[0].grad = torch.ones(4)
    tt = np.zeros(1, dtype=L.TENSOR_DTYPE)
    assert _refresh([{"params": ps}], ps, [1], [0], [L.GRAD_F32], tt) == 0


def test_module_records_its_torch():
    """The module was compiled against this torch (load_host refuses another)."""
    assert H is not None and H.torch_version == torch.__version__


class _Recording(torch.Tensor):
    """A wrapper subclass with a custom device policy: asking its impl for
    is_cuda() or device() goes through __torch_dispatch__ (Python)."""
    calls = 0

    @staticmethod
    def __new__(cls, elem):
        return torch.Tensor._make_wrapper_subclass(cls, elem.shape, dtype=elem.dtype,
                                                   device=elem.device, dispatch_device=True)

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        cls.calls += 1
        if func is torch.ops.prim.device.default:   # the .grad setter asks for it
            return torch.device("cpu")
        raise RuntimeError(f"unexpected {func}")


def test_refresh_rejects_a_subclass_gradient_without_python():
    """With 4096 or more parameters the check runs on worker threads while the
    caller holds the GIL; a gradient subclass with a custom device policy
    must be rejected from its dispatch keys, before anything that would call
    into Python."""
    n = 3 * 4096
    ps = [torch.zeros(2, requires_grad=True) for _ in range(n)]
    for p in ps:
        p.grad = torch.zeros(2)
    tt = np.zeros(n, dtype=L.TENSOR_DTYPE)
    groups = [{"params": ps}]
    ps[-5].grad = _Recording(torch.zeros(2))
    _Recording.calls = 0
    assert _refresh(groups, ps, [1] * n, list(range(n)), [L.GRAD_F32] * n, tt) == 0
    assert _Recording.calls == 0


def test_refresh_candidates_of_any_shape():
    """Candidate pointer arrays of the wrong shape are ignored (never read);
    a plan that does not apply returns 0 whatever the candidates."""
    ps = [torch.zeros(3, requires_grad=True) for _ in range(3)]
    for p in ps:
        p.grad = torch.zeros(3)
    tt = np.zeros(3, dtype=L.TENSOR_DTYPE)
    groups = [{"params": ps}]
    args = (groups, ps, np.ones(3, dtype=np.uint8), np.arange(3, dtype=np.int64),
            np.array([0, 3, 6], dtype=np.int64), np.array([1, 3, 1] * 3, dtype=np.int64),
            np.zeros(3, dtype=np.int32), tt.ctypes.data, tt.dtype.itemsize,
            tt.dtype.fields["grad"][1], tt.dtype.fields["param"][1], 0)
    cands = [np.zeros((2, 2), dtype=np.uint64), np.zeros((3, 2), dtype=np.uint64),
             np.zeros(6, dtype=np.uint64)]
    # CPU tensors: the plan does not apply (not on the planned GPU)
    assert H.refresh(*args, cands) == 0
    assert H.refresh(*args) == 0


def test_refresh_pool_after_fork():
    """The check's worker threads belong to the process that made them: a
    forked child (a DataLoader worker, say) that steps makes its own."""
    import multiprocessing as mp
    n = 4 * 2048
    ps = [torch.zeros(2, requires_grad=True) for _ in range(n)]
    for p in ps:
        p.grad = torch.zeros(2)
    tt = np.zeros(n, dtype=L.TENSOR_DTYPE)
    groups = [{"params": ps}]
    args = (groups, ps, [1] * n, list(range(n)), [L.GRAD_F32] * n, tt)
    for _ in range(3):   # the parent's pool, used more than once
        assert _refresh(*args) == 0
    ctx = mp.get_context("fork")
    q = ctx.Queue()
    child = ctx.Process(target=lambda: q.put([_refresh(*args) for _ in range(3)]))
    child.start()
    child.join(60)
    alive = child.is_alive()
    if alive:
        child.kill()
    assert not alive and child.exitcode == 0
    assert q.get(timeout=5) == [0, 0, 0]
    assert _refresh(*args) == 0
