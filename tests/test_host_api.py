"""Host-side checks that need no GPU: the C ABI library, Philox, API contract."""

import ctypes
import os
import re

import numpy as np
import pytest
import torch
import torch.nn as nn

import luma_amd
from luma_amd import LUMA
from luma_amd import _lib as L
from luma_amd.optimizer import make_step_seed

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _engine_stub(chunk_elems=0, small_tensors=True, medium_tensors=False):
    """The attributes _Engine.chunk_for and _Engine.chunk_layout read."""
    import types
    from luma_amd.optimizer import _Engine
    eng = types.SimpleNamespace(chunk_elems=chunk_elems, small_tensors=small_tensors,
                                medium_tensors=medium_tensors)
    eng._small_limit = lambda: _Engine._small_limit(eng)
    eng._medium_limit = lambda: _Engine._medium_limit(eng)
    eng._wave_limit = lambda: _Engine._wave_limit(eng)
    return eng


def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "luma.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(luma_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = L.load()
    names = _declared_symbols()
    assert "luma_step" in names and len(names) >= 9
    for name in names:
        assert hasattr(lib, name), name
        assert ctypes.cast(getattr(lib, name), ctypes.c_void_p).value


def test_layout_and_version():
    lib = L.load()
    assert lib.luma_abi_version() == L.ABI_VERSION
    L.check_layout(lib)
    assert lib.luma_workspace_bytes(10) == 160


# Random123 known-answer vectors for philox4x32_10 (kat_vectors).
PHILOX_KAT = [
    ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
    ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
    ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
     [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
]

# The same block function as computed by Triton's tl.randint4x (an independent
# implementation) for key = 0x123456789abcdef0 and counters (i, 0, 0, 0).
PHILOX_TRITON = [
    (0, [0x092C9B44, 0x78384BC0, 0xC9FB80BE, 0x2B3BE4DD]),
    (3, [0xF708969C, 0x62778C12, 0xE11922B4, 0x6D6AF8E0]),
    (7, [0x2A23B679, 0x84C69006, 0x0481A097, 0x0AE2270E]),
]


@pytest.mark.parametrize("ctr,key,out", PHILOX_KAT)
def test_philox_known_answers(ctr, key, out):
    assert L.philox4x32(ctr, key) == out


@pytest.mark.parametrize("i,out", PHILOX_TRITON)
def test_philox_matches_triton(i, out):
    seed = 0x123456789ABCDEF0
    assert L.philox4x32([i, 0, 0, 0], [seed & 0xFFFFFFFF, seed >> 32]) == out


def test_step_seed_matches_reference_formula():
    # functional.py:99-106
    for base in [0, 12345, -(2**63), 2**63 - 1, -987654321]:
        for t in [0, 1, 2, 1000]:
            for pid in [0, 1, 77]:
                assert make_step_seed(base, t, pid) == ((t << 32) | (2 * pid)) ^ base


# ── API contract (optimizer.py:71-113), no GPU needed ────────────────────────

def test_default_params():
    assert LUMA(nn.Linear(8, 4).parameters()) is not None


def test_custom_params():
    opt = LUMA(nn.Linear(8, 4).parameters(), lr=5e-4, betas=(0.95, 0.98), eps=1e-6,
               weight_decay=0.1)
    assert opt.defaults["lr"] == 5e-4


def test_invalid_backend():
    with pytest.raises(ValueError, match="Invalid backend"):
        LUMA(nn.Linear(8, 4).parameters(), backend="tritonn")


@pytest.mark.parametrize("kwargs", [{"lr": -1}, {"eps": -1}, {"eps": 0}, {"betas": (1.0, 0.999)},
                                    {"betas": (0.9, -0.1)}, {"weight_decay": -0.01}])
def test_invalid_hyperparams(kwargs):
    with pytest.raises(ValueError):
        LUMA(nn.Linear(4, 2).parameters(), **kwargs)


def test_base_seed_from_global_generator():
    torch.manual_seed(42)
    a = LUMA([torch.zeros(3, requires_grad=True)])._base_seed
    torch.manual_seed(42)
    b = int(torch.randint(-(2**63), 2**63 - 1, (1,), dtype=torch.int64).item())
    assert a == b


def test_step_without_grads_is_noop():
    opt = LUMA(nn.Linear(8, 4).parameters())
    assert opt.step() is None


def test_cpu_params_fail_loudly():
    """No CPU fallback: the step refuses parameters that are not on the GPU."""
    model = nn.Linear(8, 4)
    opt = LUMA(model.parameters())
    model(torch.randn(2, 8)).sum().backward()
    with pytest.raises(RuntimeError, match="GPU"):
        opt.step()


def test_rejects_reduced_precision_params():
    model = nn.Linear(16, 8).to(torch.bfloat16)
    opt = LUMA(model.parameters())
    for p in model.parameters():
        p.grad = torch.randn_like(p)
    with pytest.raises(ValueError, match="float32"):
        opt.step()


def test_sparse_grad_rejected():
    emb = nn.Embedding(10, 4, sparse=True)
    opt = LUMA(emb.parameters())
    emb(torch.tensor([1, 2])).sum().backward()
    with pytest.raises(RuntimeError, match="sparse"):
        opt.step()


def test_step_chunk_policy():
    """The step's chunk length: 131072 while 2048 chunks of it fit in the
    set's total size, else halved down to 16384; a fixed length overrides it."""
    import types
    import numpy as np
    from luma_amd.optimizer import _Engine
    pick = _Engine.chunk_for
    auto = _engine_stub(chunk_elems=0)
    assert pick(auto, np.array([4096 * 4096], dtype=np.int64)) == 16384
    # (fewer than 2048 tensors above the wavefront limit in these)
    assert pick(auto, np.array([65536] * 1024 + [1] * 3000, dtype=np.int64)) == 32768
    assert pick(auto, np.array([131072] * 2047, dtype=np.int64)) == 65536
    assert pick(auto, np.array([131072] * 1024, dtype=np.int64)) == 65536
    assert pick(auto, np.array([65536] * 2047, dtype=np.int64)) == 32768
    assert pick(auto, np.array([65536] * 1024, dtype=np.int64)) == 32768
    assert pick(auto, np.array([65536] * 1023, dtype=np.int64)) == 16384
    assert pick(auto, np.array([1] * 20000, dtype=np.int64)) == 16384
    assert pick(auto, np.array([65536] * 1000 + [1] * 20000, dtype=np.int64)) == 16384
    assert pick(_engine_stub(chunk_elems=2048), np.array([10], dtype=np.int64)) == 2048
    # 2048 or more tensors above the wavefront limit: one chunk per tensor,
    # as long as the largest of them (at most 131072)
    assert pick(auto, np.array([65536] * 2048, dtype=np.int64)) == 65536
    assert pick(auto, np.array([65536] * 4096, dtype=np.int64)) == 131072
    assert pick(auto, np.array([600] * 2047 + [40000], dtype=np.int64)) == 65536
    assert pick(auto, np.array([600] * 2048 + [300000], dtype=np.int64)) == 131072
    assert pick(auto, np.array([600] * 2047 + [40000] + [1] * 10, dtype=np.int64)) == 65536
    assert pick(auto, np.array([600] * 2047 + [1] * 10, dtype=np.int64)) == 16384
    assert pick(_engine_stub(small_tensors=False),
                np.array([600] * 2047 + [1] * 10, dtype=np.int64)) == 16384


def test_step_rejects_bad_chunk_length():
    """luma_step validates chunk_elems before any launch."""
    lib = L.load()
    for bad in (1000, 1024, 262144, 3 * 4096):
        args = L.StepArgs(tensors=16, n_tensors=1, n_chunks=1, chunks=16, groups=16, partials=16,
                          base_seed=0, noise_mode=L.NOISE_PHILOX, flags=0, chunk_elems=bad,
                          small_chunks=0, medium_chunks=0, scaling=L.Scaling(None, None))
        assert lib.luma_step(ctypes.byref(args), None) != 0
        assert b"chunk_elems" in lib.luma_last_error()


def test_step_rejects_bad_small_chunks():
    """luma_step validates small_chunks (0 .. n_chunks) before any launch."""
    lib = L.load()
    for bad in (-1, 3):
        args = L.StepArgs(tensors=16, n_tensors=1, n_chunks=2, chunks=16, groups=16, partials=16,
                          base_seed=0, noise_mode=L.NOISE_PHILOX, flags=0, chunk_elems=0,
                          small_chunks=bad, scaling=L.Scaling(None, None))
        assert lib.luma_step(ctypes.byref(args), None) != 0
        assert b"small_chunks" in lib.luma_last_error()
    for small, bad in ((0, -1), (0, 3), (1, 2)):
        args = L.StepArgs(tensors=16, n_tensors=1, n_chunks=2, chunks=16, groups=16, partials=16,
                          base_seed=0, noise_mode=L.NOISE_PHILOX, flags=0, chunk_elems=0,
                          small_chunks=small, medium_chunks=bad, scaling=L.Scaling(None, None))
        assert lib.luma_step(ctypes.byref(args), None) != 0
        assert b"medium_chunks" in lib.luma_last_error()


def test_step_args_fields():
    """The ctypes binding has exactly the header's LumaStepArgs fields (a
    misspelt keyword would otherwise become a plain Python attribute)."""
    names = [f[0] for f in L.StepArgs._fields_]
    assert names == ["tensors", "n_tensors", "n_chunks", "chunks", "groups", "partials",
                     "base_seed", "noise_mode", "flags", "chunk_elems", "small_chunks",
                     "medium_chunks", "reserved", "scaling"]


def test_package_exports():
    assert luma_amd.__all__ == ["LUMA", "get_kernel_config"]
    assert "CHUNK_ELEMS" in luma_amd.get_kernel_config()


def test_state_arena_layout():
    """Q_m / Q_w views of one allocation: parameter shapes and strides
    (channels_last included), 256-byte aligned offsets, no overlap."""
    from luma_amd.optimizer import state_arena
    ps = [torch.zeros(3, 5), torch.zeros(1), torch.zeros(2, 3, 4, 5).to(memory_format=torch.channels_last),
          torch.zeros(300)]
    views = state_arena(ps, torch.device("cpu"))
    base = views[0][0].untyped_storage().data_ptr()
    for p, (qm, qw) in zip(ps, views):
        for q in (qm, qw):
            assert q.dtype == torch.int16 and q.shape == p.shape and q.stride() == p.stride()
            assert q.untyped_storage().data_ptr() == base
            assert (q.data_ptr() - base) % 256 == 0
    for i, (qm, qw) in enumerate(views):
        qm.fill_(i + 1)
        qw.fill_(-(i + 1))
    for i, (qm, qw) in enumerate(views):
        assert (qm == i + 1).all() and (qw == -(i + 1)).all()


def test_chunk_layout_small_tensors_last():
    """Tensors of at most SMALL_TENSOR elements take the last chunk records
    (one each, largest first); the others keep their order; first_chunk
    points at each tensor's records."""
    import types
    import numpy as np
    from luma_amd.optimizer import _Engine
    S = L.SMALL_TENSOR
    numels = np.array([5000, 3, S, S + 1, 40000, 1, 20000], dtype=np.int64)
    eng = _engine_stub(small_tensors=True)
    first, ch, n_small, n_med = _Engine.chunk_layout(eng, numels, 16384)
    assert n_small == 3
    assert ch["tensor"].tolist() == [0, 3, 4, 4, 4, 6, 6, 2, 1, 5]
    assert ch["index"].tolist() == [0, 0, 0, 1, 2, 0, 1, 0, 0, 0]
    assert first.tolist() == [0, 8, 7, 1, 2, 9, 5]
    for t in range(len(numels)):
        assert ch["tensor"][first[t]] == t and ch["index"][first[t]] == 0
    eng.small_tensors = False
    first, ch, n_small, n_med = _Engine.chunk_layout(eng, numels, 16384)
    assert n_small == 0
    assert ch["tensor"].tolist() == [0, 1, 2, 3, 4, 4, 4, 5, 6, 6]
    assert first.tolist() == [0, 1, 2, 3, 4, 7, 8]


def test_chunk_layout_many_tensors_largest_first(monkeypatch):
    """With STEP_TARGET_CHUNKS or more tensors above the wavefront limit, their
    chunk records come largest tensor first (ties in parameter order), the
    small tensors still last; first_chunk points at each tensor's records."""
    import numpy as np
    import luma_amd.optimizer as O
    S = L.SMALL_TENSOR
    numels = np.array([5000, 3, S, S + 1, 40000, 1, 20000, 5000], dtype=np.int64)
    eng = _engine_stub()
    monkeypatch.setattr(O, "STEP_TARGET_CHUNKS", 5)
    assert O._Engine.chunk_for(eng, numels) == 65536
    first, ch, n_small, n_med = O._Engine.chunk_layout(eng, numels, 65536)
    assert n_small == 3
    assert ch["tensor"].tolist() == [4, 6, 0, 7, 3, 2, 1, 5]
    assert ch["index"].tolist() == [0] * 8
    for t in range(len(numels)):
        assert ch["tensor"][first[t]] == t
    # chunks of 16384: the 40000-element tensor's three records stay together
    first, ch, n_small, n_med = O._Engine.chunk_layout(eng, numels, 16384)
    assert ch["tensor"].tolist() == [4, 4, 4, 6, 6, 0, 7, 3, 2, 1, 5]
    assert ch["index"].tolist() == [0, 1, 2, 0, 1, 0, 0, 0, 0, 0, 0]
    assert first.tolist() == [5, 9, 8, 7, 0, 10, 3, 6]
    # one tensor fewer above the limit: parameter order
    monkeypatch.setattr(O, "STEP_TARGET_CHUNKS", 6)
    first, ch, n_small, n_med = O._Engine.chunk_layout(eng, numels, 65536)
    assert ch["tensor"].tolist() == [0, 3, 4, 6, 7, 2, 1, 5]


def test_chunk_layout_medium_tensors():
    """Tensors above SMALL_TENSOR and of at most MEDIUM_TENSOR elements (and
    one chunk) take the records before the small ones, largest first; the
    workgroup tensors keep their order and come first."""
    import numpy as np
    from luma_amd.optimizer import _Engine
    M = L.MEDIUM_TENSOR
    S = L.SMALL_TENSOR
    numels = np.array([M + 904, 3, S, S + 1, 40000, 1, 20000, M, 2000], dtype=np.int64)
    eng = _engine_stub(medium_tensors=True)
    first, ch, n_small, n_med = _Engine.chunk_layout(eng, numels, 16384)
    assert (n_med, n_small) == (3, 3)
    assert ch["tensor"].tolist() == [0, 4, 4, 4, 6, 6, 7, 8, 3, 2, 1, 5]
    assert ch["index"].tolist() == [0, 0, 1, 2, 0, 1, 0, 0, 0, 0, 0, 0]
    for t in range(len(numels)):
        assert ch["tensor"][first[t]] == t and ch["index"][first[t]] == 0
    # a chunk shorter than the medium limit: only tensors of one chunk qualify
    first, ch, n_small, n_med = _Engine.chunk_layout(eng, numels, 2048)
    assert (n_med, n_small) == (2, 3)
    assert ch["tensor"].tolist()[-5:] == [8, 3, 2, 1, 5]
    # the tensors above the medium limit decide the one-chunk-per-tensor rule
    # (2048 or more of them)
    assert _Engine.chunk_for(eng, np.array([3000] * 5000 + [40000], dtype=np.int64)) == 16384
    assert _Engine.chunk_for(eng, np.array([M + 904] * 2048 + [40000], dtype=np.int64)) == 65536


@pytest.mark.parametrize("with_host", [True, False])
def test_moved_pointer_tables_are_reused(with_host):
    """A planned step whose gradients alternate between buffers uploads each
    pointer set's table once (_Engine._match_pointers), and a cached set
    whose pointers differ, or another table object, never returns a wrong
    table; the host module's comparison and numpy's agree."""
    from luma_amd.optimizer import _Engine
    eng = _Engine.__new__(_Engine)
    eng.host = L.load_host() if with_host else None
    if with_host and eng.host is None:
        pytest.skip("host module not built")
    eng._ptr_cache = {}
    eng._ptr_seq = 0
    eng._tensor_key = b""
    uploads = []
    eng._upload = lambda arr: uploads.append(arr.copy()) or len(uploads)
    tt = np.zeros(5, dtype=L.TENSOR_DTYPE)
    tt["param"] = np.arange(5) * 4096 + (1 << 40)
    sets = [np.arange(5, dtype=np.uint64) * 512 + (k + 1) * (1 << 36) for k in range(2)]
    for i in range(6):
        tt["grad"] = sets[i % 2]
        eng._match_pointers(tt, capturing=False)
        assert eng._d_tensors == 1 + (i % 2)          # one upload per pointer set
        assert np.array_equal(uploads[eng._d_tensors - 1]["grad"], sets[i % 2])
    assert len(uploads) == 2 and eng._tensor_key is None
    # the same pointers in another table object: not re-used
    tt2 = tt.copy()
    eng._match_pointers(tt2, capturing=False)
    assert len(uploads) == 3
    # two gradients swapped, and the last parameter moved: new tables
    tt["grad"] = sets[0][[1, 0, 2, 3, 4]]
    eng._match_pointers(tt, capturing=False)
    assert len(uploads) == 4
    tt["grad"] = sets[0]
    tt["param"][4] += 256
    eng._match_pointers(tt, capturing=False)
    assert len(uploads) == 5 and eng._d_tensors == 5
    assert len(eng._ptr_cache) == _Engine.TABLE_CACHE
    # a cached entry whose columns differ from the table's: uploaded afresh
    key = list(eng._ptr_cache)[-1]
    ent = eng._ptr_cache[key]
    assert ent[0] is tt
    eng._ptr_cache = {key: (ent[0], ent[1] + 1, ent[2])}
    with pytest.raises(RuntimeError):
        eng._match_pointers(ent[0], capturing=True)   # would need an upload under capture


def test_pointer_match_named_by_the_caller():
    """_match_pointers takes a cached set named by the caller (the host
    module's refresh compared it) without comparing; a key that names no
    set of this table falls back to the comparison."""
    from luma_amd.optimizer import _Engine
    eng = _Engine.__new__(_Engine)
    eng.host = None
    eng._ptr_cache = {}
    eng._ptr_seq = 0
    eng._tensor_key = b""
    uploads = []
    eng._upload = lambda arr: uploads.append(arr.copy()) or len(uploads)
    tt = np.zeros(3, dtype=L.TENSOR_DTYPE)
    tt["param"] = np.arange(3) * 4096 + (1 << 40)
    sets = [np.arange(3, dtype=np.uint64) * 512 + (k + 1) * (1 << 36) for k in range(2)]
    for k in range(2):
        tt["grad"] = sets[k]
        eng._match_pointers(tt, capturing=False)
    cands = eng.pointer_candidates(tt)
    assert [c[1][:, 0].tolist() for c in cands] == [sets[1].tolist(), sets[0].tolist()]
    compared = []
    eng._same_pointers = lambda t, cols: compared.append(1) or _Engine._same_pointers(eng, t, cols)
    tt["grad"] = sets[0]
    eng._match_pointers(tt, capturing=True, match=cands[1][0])   # no upload, no comparison
    assert eng._d_tensors == 1 and not compared
    tt["grad"] = sets[1]
    eng._match_pointers(tt, capturing=False, match=-5)           # unknown key: compared
    assert eng._d_tensors == 2 and compared and len(uploads) == 2
    # another table's key is not taken
    tt2 = tt.copy()
    eng._match_pointers(tt2, capturing=False, match=cands[0][0])
    assert len(uploads) == 3
