"""The five benchmark workloads against the CPU oracle, on the GPU at full size.

Each test builds one configuration's parameter set on the GPU, steps it with
the HIP optimizer, and steps the same tensors (all of them, or a sample for
the 8B-parameter sets) with the correctly rounded oracle on the CPU, the
oracle's uniforms injected into the sampled tensors.  After every step the
sampled tensors' codes and scales must be identical and their parameters
within 1e-6 (the reference's own parity tests, tests/test_correctness.py:
247-381, run its two backends on the same inputs; the configurations are
those of the reference's headline benchmark set):

  cfg1  one 4096x4096 fp32 tensor, fp32 grads N(0, 1e-3)             6 steps
  cfg2  the GPT-2-small list (148 tensors, 124M params), bf16 grads  3 steps
  cfg3  20,000 tensors of log-uniform size in [1, 65536], fp32 grads
        N(0, 1e-4) with 1% exact zeros (one chunk per tensor)        3 steps
  cfg4  the Llama-3-8B set (291 tensors, 8.03G params), bf16 grads with
        0.1% x100 outliers; seven tensors sampled, one of each shape
        (the 525M-element embedding included)                        3 steps
  cfg5  the same set, per-tensor grad std log-uniform in [1e-7, 1e-1],
        fp16 grads scaled by 2^16 and unscaled in the kernel by
        torch.amp.GradScaler, resumed from a state_dict after 2 steps;
        five tensors sampled                                         2+2 steps
"""

import gc
import math

import pytest
import torch

import bench
from luma_amd import _lib as L
from config_util import SampledPair, normal_grad, numel

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _gen(seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    return g


@pytest.fixture(autouse=True)
def _free_memory():
    yield
    gc.collect()
    torch.cuda.empty_cache()


@pytest.mark.timeout(600)
def test_cfg1_single_4096():
    p = torch.randn(4096, 4096, device=DEV, generator=_gen(0)) * 0.02
    pair = SampledPair([p], [0])
    for t in range(1, 7):
        g = normal_grad((4096, 4096), 1e-3, _gen(1000 + t), DEV, torch.float32)
        pair.step([g], {0: g.cpu()})
        pair.check()


def _gpt2_params():
    """GPT-2-small: weights N(0, 0.02); LayerNorm weights 1, biases 0."""
    shapes = bench.gpt2_small_shapes()
    gen = _gen(0)
    params = []
    block = len(shapes[2:-2]) // 12
    for k, s in enumerate(shapes):
        if len(s) == 2:
            params.append(torch.randn(s, device=DEV, generator=gen) * 0.02)
            continue
        j = (k - 2) % block if 2 <= k < len(shapes) - 2 else (0 if k == len(shapes) - 2 else 1)
        # in a block: 0 ln_1.w, 1 ln_1.b, 3 c_attn.b, 5 c_proj.b, 6 ln_2.w, 7 ln_2.b, ...
        params.append(torch.full(s, 1.0 if j in (0, 6) else 0.0, device=DEV))
    return params


@pytest.mark.timeout(600)
def test_cfg2_gpt2_small():
    params = _gpt2_params()
    assert len(params) == 148 and sum(p.numel() for p in params) == 124_439_808
    pair = SampledPair(params, range(len(params)))
    for t in range(1, 4):
        gen = _gen(2000 + t)
        gd = [normal_grad(p.shape, 1e-3, gen, DEV, torch.bfloat16) for p in params]
        pair.step(gd, {i: g.cpu() for i, g in enumerate(gd)})
        pair.check()


@pytest.mark.timeout(600)
def test_cfg3_many_small():
    shapes = bench.many_small_shapes()
    assert len(shapes) == 20000
    gen = _gen(3)
    params = [torch.randn(s, device=DEV, generator=gen) * 0.02 for s in shapes]
    total = sum(p.numel() for p in params)
    print(f"cfg3: {len(params)} tensors, {total} params", flush=True)
    pair = SampledPair(params, range(len(params)))
    for t in range(1, 4):
        gen = _gen(3000 + t)
        gd = [normal_grad(p.shape, 1e-4, gen, DEV, torch.float32, zeros=0.01) for p in params]
        pair.step(gd, {i: g.cpu() for i, g in enumerate(gd)})
        # more than 2048 tensors above the single-wavefront routes: one
        # chunk per tensor (the largest has 32769 to 65536 elements),
        # largest first; tensors of 513 to 8192 elements a wavefront each
        # in the fast kernels, those of at most 256 the exact wavefront kernels
        eng = pair.opt._engine
        assert 32768 < max(p.numel() for p in params) <= 65536
        assert eng._chunk == 65536 and eng._n_chunks == len(params)
        assert eng._small_chunks == sum(1 for p in params if p.numel() <= L.SMALL_TENSOR)
        assert eng._medium_chunks == sum(1 for p in params
                                         if L.SMALL_TENSOR < p.numel() <= L.MEDIUM_TENSOR)
        rows = pair.check()
        assert sum(r["n"] for r in rows) == total


# Llama-3-8B (bench.llama3_8b_shapes order: embed, 32 x [q, k, v, o, gate, up,
# down, norm, norm], final norm, lm_head)
def _llama_index(layer, which):
    return 1 + 9 * layer + ["q", "k", "v", "o", "gate", "up", "down", "n1", "n2"].index(which)


def _llama_params():
    shapes = bench.llama3_8b_shapes()
    gen = _gen(0)
    params = []
    for s in shapes:
        params.append(torch.full(s, 1.0, device=DEV) if len(s) == 1
                      else torch.randn(s, device=DEV, generator=gen) * 0.02)
    assert len(params) == 291 and sum(p.numel() for p in params) == 8_030_261_248
    return params


@pytest.mark.timeout(900)
def test_cfg4_llama3_8b_sampled():
    params = _llama_params()
    sample = [0, _llama_index(0, "q"), _llama_index(5, "k"), _llama_index(17, "gate"),
              _llama_index(31, "down"), _llama_index(31, "n2"), 289]
    assert [tuple(params[i].shape) for i in sample] == [
        (128256, 4096), (4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336), (4096,),
        (4096,)]
    pair = SampledPair(params, sample)
    for t in range(1, 4):
        gen = _gen(4000 + t)
        gd = []
        for i, p in enumerate(params):
            gd.append(normal_grad(p.shape, 1e-3, gen, DEV, torch.bfloat16, outliers=1e-3))
            params[i].grad = None
        pair.step(gd, {i: gd[i].cpu() for i in sample})
        del gd
        pair.check()
    # every tensor advanced, sampled or not
    assert all(s["step"] == 3 for s in pair.opt.state_dict()["state"].values())


@pytest.mark.timeout(900)
def test_cfg5_hetero_fp16_gradscaler_restored():
    params = _llama_params()
    shapes = [tuple(p.shape) for p in params]
    gen5 = torch.Generator().manual_seed(5)
    stds = torch.exp(torch.empty(len(shapes), dtype=torch.float64)
                     .uniform_(math.log(1e-7), math.log(1e-1), generator=gen5)).tolist()
    sample = [_llama_index(0, "q"), _llama_index(9, "k"), _llama_index(30, "down"),
              _llama_index(30, "n1"), 289]
    pair = SampledPair(params, sample)
    scaler = torch.amp.GradScaler(DEV, init_scale=2.0 ** 16, growth_interval=10 ** 9)
    scaler.scale(torch.ones((), device=DEV))   # creates the scale tensor

    def through_scaler(opt):
        scaler.step(opt)      # the kernels unscale; found_inf is checked on the device
        scaler.update()

    for t in range(1, 5):
        if t == 3:
            pair.restore()    # resume from the checkpoint of step 2
        gen = _gen(5000 + t)
        gd, gc_ = [], {}
        for i, p in enumerate(params):
            g = torch.randn(p.shape, device=DEV, generator=gen) * stds[i]
            g16 = (g * 2.0 ** 16).half()           # what backward produces under the scaler
            gd.append(g16)
            if i in sample:                        # what GradScaler.unscale_ would store
                gc_[i] = (g16.float() * 2.0 ** -16).half().cpu()
            params[i].grad = None
        pair.step(gd, gc_, driver=through_scaler)
        del gd
        assert scaler.get_scale() == 2.0 ** 16    # no overflow: every step was taken
        rows = pair.check()
        print(" ".join(f"[{r['i']}] dq={r['dq']} p_rel={r['p_rel']:.1e}" for r in rows), flush=True)
