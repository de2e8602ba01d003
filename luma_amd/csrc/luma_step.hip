// LUMA optimizer step for MI355X (gfx950): multi-tensor passes behind the C ABI
// of include/luma.h.
//
// One step over every parameter is three launches on the caller's stream:
//   pass 1   (grid = chunks)  decode Q_m/Q_w with the old grid, EMA with the
//                             gradient, max |m'| and max v' per chunk;
//   finalize (grid = tensors) reduce the chunk maxima to S_m', S_v' and derive
//                             the new grid in float64 (functional.py:282-292);
//   pass 2   (grid = chunks)  recompute m', v' bit-identically, AdamW update of
//                             the parameter, LogSR re-quantisation on the new
//                             grid (functional.py:278-279, 293-295).
// Nothing is materialised between the passes except 8 bytes per chunk.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <stdio.h>
#include <string.h>

#include "../../include/luma.h"
#include "luma_exact.h"
#include "luma_philox.h"

namespace luma {

constexpr int kThreads = 256;     // 4 wave64 per workgroup
constexpr int kVec = 8;           // consecutive elements per thread per iteration
constexpr int64_t kChunk = LUMA_CHUNK_ELEMS;
static_assert(kChunk % (kThreads * kVec) == 0, "chunk must be a whole number of iterations");
static_assert(sizeof(LumaHyper) == sizeof(Hyper), "hyper layout");

struct Tensor {  // mirror of LumaTensor
  float *param;
  const void *grad;
  int16_t *q_m;
  int16_t *q_w;
  const float *u_m;
  const float *u_w;
  int64_t numel;
  int64_t step;
  int64_t param_id;
  int32_t grad_dtype;
  int32_t hyper;
  int32_t slot;
  int32_t first_chunk;
};
static_assert(sizeof(Tensor) == sizeof(LumaTensor), "tensor layout");

__device__ __forceinline__ float load_grad(const void *g, int64_t i, int dt) {
  if (dt == LUMA_GRAD_F32) return static_cast<const float *>(g)[i];
  const uint16_t b = static_cast<const uint16_t *>(g)[i];
  if (dt == LUMA_GRAD_BF16) return __uint_as_float((uint32_t)b << 16);
  return __half2float(__ushort_as_half(b));
}

// Key of the (param, step) uniform stream: the reference's step seed
// ((t << 32) | 2*pid) ^ base_seed (functional.py:99-106) as 64 bits.
__device__ __forceinline__ void step_key(uint64_t base, int64_t t, int64_t pid, uint32_t &k0,
                                         uint32_t &k1) {
  const uint64_t s = (((uint64_t)t << 32) | (uint64_t)(2 * pid)) ^ base;
  k0 = (uint32_t)s;
  k1 = (uint32_t)(s >> 32);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = nan_max(v, __shfl_xor(v, off, 64));
  return v;
}

// Block-wide NaN-propagating max of two values; result valid in thread 0.
__device__ __forceinline__ void block_max2(float &a, float &b) {
  __shared__ float sa[kThreads / 64], sb[kThreads / 64];
  a = wave_max(a);
  b = wave_max(b);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  if (l == 0) {
    sa[w] = a;
    sb[w] = b;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < kThreads / 64; ++i) {
      a = nan_max(a, sa[i]);
      b = nan_max(b, sb[i]);
    }
  }
}

// m', v' of element i of tensor T (exact path).
__device__ __forceinline__ void element_ema(const Tensor &T, const Hyper &h, const Grid *old,
                                            int64_t i, float &mn, float &vn) {
  const float g = load_grad(T.grad, i, T.grad_dtype);
  float m = 0.0f, v = 0.0f;
  if (old) {  // t >= 2: decode the stored codes on the old grid
    m = exact_decode_m(T.q_m[i], old->dm);
    v = exact_decode_v(T.q_w[i], old->wmin, old->dw, h.eps);
  }
  exact_ema(m, v, g, h, mn, vn);
}

__global__ __launch_bounds__(kThreads) void pass1_kernel(const Tensor *__restrict__ tensors,
                                                         const LumaChunk *__restrict__ chunks,
                                                         const Hyper *__restrict__ hypers,
                                                         const Slot *__restrict__ slots,
                                                         float *__restrict__ partials) {
  const LumaChunk c = chunks[blockIdx.x];
  const Tensor T = tensors[c.tensor];
  const Hyper h = hypers[T.hyper];
  const Grid *old = T.step >= 2 ? &slots[T.slot].grid[(T.step - 1) & 1] : nullptr;
  const int64_t beg = (int64_t)c.index * kChunk;
  const int64_t end = beg + kChunk < T.numel ? beg + kChunk : T.numel;

  float am = 0.0f, av = 0.0f;
  for (int64_t e0 = beg + (int64_t)threadIdx.x * kVec; e0 < end; e0 += (int64_t)kThreads * kVec) {
    for (int j = 0; j < kVec; ++j) {
      const int64_t i = e0 + j;
      if (i >= end) break;
      float mn, vn;
      element_ema(T, h, old, i, mn, vn);
      am = nan_max(am, fabsf(mn));
      av = nan_max(av, vn);
    }
  }
  block_max2(am, av);
  if (threadIdx.x == 0) {
    partials[2 * (int64_t)blockIdx.x] = am;
    partials[2 * (int64_t)blockIdx.x + 1] = av;
  }
}

// S' = max(max, floor) with Python's max() semantics (a NaN maximum stays NaN).
__device__ __forceinline__ double py_max(double a, double floor_) { return floor_ > a ? floor_ : a; }

__global__ __launch_bounds__(64) void finalize_kernel(const Tensor *__restrict__ tensors,
                                                      const Hyper *__restrict__ hypers,
                                                      Slot *__restrict__ slots,
                                                      const float *__restrict__ partials) {
  const Tensor T = tensors[blockIdx.x];
  const int nch = (int)((T.numel + kChunk - 1) / kChunk);
  float am = 0.0f, av = 0.0f;
  for (int i = threadIdx.x; i < nch; i += 64) {
    const int64_t c = (int64_t)T.first_chunk + i;
    am = nan_max(am, partials[2 * c]);
    av = nan_max(av, partials[2 * c + 1]);
  }
  am = wave_max(am);
  av = wave_max(av);
  if (threadIdx.x == 0) {
    const double s_m = py_max((double)am, 1e-9);  // SCALE_FLOOR_M (config.py:25)
    const double s_v = py_max((double)av, 0.0);
    Slot &s = slots[T.slot];
    const int par = (int)(T.step & 1);
    s.s_m[par] = s_m;
    s.s_v[par] = s_v;
    make_grid(s_m, s_v, hypers[T.hyper].eps_d, s.grid[par]);
  }
}

__global__ __launch_bounds__(kThreads) void pass2_kernel(const Tensor *__restrict__ tensors,
                                                         const LumaChunk *__restrict__ chunks,
                                                         const Hyper *__restrict__ hypers,
                                                         const Slot *__restrict__ slots,
                                                         uint64_t base_seed, int noise_mode) {
  const LumaChunk c = chunks[blockIdx.x];
  const Tensor T = tensors[c.tensor];
  const Hyper h = hypers[T.hyper];
  const Slot &S = slots[T.slot];
  const Grid *old = T.step >= 2 ? &S.grid[(T.step - 1) & 1] : nullptr;
  const Grid G = S.grid[T.step & 1];
  const int64_t beg = (int64_t)c.index * kChunk;
  const int64_t end = beg + kChunk < T.numel ? beg + kChunk : T.numel;
  uint32_t k0, k1;
  step_key(base_seed, T.step, T.param_id, k0, k1);

  for (int64_t e0 = beg + (int64_t)threadIdx.x * kVec; e0 < end; e0 += (int64_t)kThreads * kVec) {
    U4 coarse{}, fine0{}, fine1{};
    if (noise_mode == LUMA_NOISE_PHILOX) {
      coarse = philox_coarse_block((uint64_t)e0, k0, k1);
      fine0 = philox_fine_block((uint64_t)e0, k0, k1);
      fine1 = philox_fine_block((uint64_t)e0 + 4, k0, k1);
    }
    for (int j = 0; j < kVec; ++j) {
      const int64_t i = e0 + j;
      if (i >= end) break;
      float mn, vn;
      element_ema(T, h, old, i, mn, vn);
      T.param[i] = exact_param_update(T.param[i], mn, vn, h);
      float um, uw;
      if (noise_mode == LUMA_NOISE_PHILOX) {
        uint32_t bm, bw;
        philox_uniform_bits(coarse, j < 4 ? fine0 : fine1, (uint64_t)i, bm, bw);
        um = (float)bm * 0x1p-24f;
        uw = (float)bw * 0x1p-24f;
      } else {
        um = T.u_m[i];
        uw = T.u_w[i];
      }
      T.q_m[i] = (int16_t)exact_quant_m(mn, G, um);
      T.q_w[i] = (int16_t)(uint16_t)exact_quant_w(vn, G, h.eps, uw);
    }
  }
}

// ---------------------------------------------------------------------------
//  Scale slots, decode (export) and quantise (import)
// ---------------------------------------------------------------------------

__global__ void set_scales_kernel(Slot *__restrict__ slots, const LumaScaleInit *__restrict__ items,
                                  int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const LumaScaleInit it = items[i];
  Slot &s = slots[it.slot];
  const int par = (int)(it.step & 1);
  s.s_m[par] = it.s_m;
  s.s_v[par] = it.s_v;
  make_grid(it.s_m, it.s_v, it.eps, s.grid[par]);
}

__global__ void get_scales_kernel(const Slot *__restrict__ slots, const int32_t *__restrict__ idx,
                                  const int64_t *__restrict__ steps, int n, double *__restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const Slot &s = slots[idx[i]];
  const int par = (int)(steps[i] & 1);
  out[2 * i] = s.s_m[par];
  out[2 * i + 1] = s.s_v[par];
}

__global__ __launch_bounds__(kThreads) void decode_kernel(const int16_t *__restrict__ q_m,
                                                          const int16_t *__restrict__ q_w,
                                                          int64_t n, const Slot *__restrict__ slots,
                                                          int slot, int par, double eps,
                                                          float *__restrict__ m_out,
                                                          float *__restrict__ v_out) {
  __shared__ Grid g;
  if (threadIdx.x == 0) make_grid(slots[slot].s_m[par], slots[slot].s_v[par], eps, g);
  __syncthreads();
  const float epsf = (float)eps;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads) {
    m_out[i] = exact_decode_m(q_m[i], g.dm);
    v_out[i] = exact_decode_v(q_w[i], g.wmin, g.dw, epsf);
  }
}

__global__ __launch_bounds__(kThreads) void quant_max_kernel(const float *__restrict__ m,
                                                             const float *__restrict__ v, int64_t n,
                                                             float *__restrict__ partials) {
  const int64_t beg = (int64_t)blockIdx.x * kChunk;
  const int64_t end = beg + kChunk < n ? beg + kChunk : n;
  float am = 0.0f, av = 0.0f;
  for (int64_t i = beg + threadIdx.x; i < end; i += kThreads) {
    const float vi = v[i];
    am = nan_max(am, fabsf(m[i]));
    av = nan_max(av, (vi != vi || vi > 0.0f) ? vi : 0.0f);
  }
  block_max2(am, av);
  if (threadIdx.x == 0) {
    partials[2 * (int64_t)blockIdx.x] = am;
    partials[2 * (int64_t)blockIdx.x + 1] = av;
  }
}

__global__ __launch_bounds__(64) void quant_finalize_kernel(const float *__restrict__ partials,
                                                            int nch, Slot *__restrict__ slots,
                                                            int slot, int par, double eps) {
  float am = 0.0f, av = 0.0f;
  for (int i = threadIdx.x; i < nch; i += 64) {
    am = nan_max(am, partials[2 * i]);
    av = nan_max(av, partials[2 * i + 1]);
  }
  am = wave_max(am);
  av = wave_max(av);
  if (threadIdx.x == 0) {
    Slot &s = slots[slot];
    s.s_m[par] = py_max((double)am, 1e-9);
    s.s_v[par] = py_max((double)av, 0.0);
    make_grid(s.s_m[par], s.s_v[par], eps, s.grid[par]);
  }
}

__global__ __launch_bounds__(kThreads) void quant_kernel(const float *__restrict__ m,
                                                         const float *__restrict__ v, int64_t n,
                                                         int16_t *__restrict__ q_m,
                                                         int16_t *__restrict__ q_w,
                                                         const Slot *__restrict__ slots, int slot,
                                                         int par, double eps, uint64_t seed,
                                                         int noise_mode, const float *__restrict__ u_m,
                                                         const float *__restrict__ u_w) {
  const Grid G = slots[slot].grid[par];
  const float epsf = (float)eps;
  const uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
  const int64_t beg = (int64_t)blockIdx.x * kChunk;
  const int64_t end = beg + kChunk < n ? beg + kChunk : n;
  for (int64_t e0 = beg + (int64_t)threadIdx.x * kVec; e0 < end; e0 += (int64_t)kThreads * kVec) {
    U4 coarse{}, fine0{}, fine1{};
    if (noise_mode == LUMA_NOISE_PHILOX) {
      coarse = philox_coarse_block((uint64_t)e0, k0, k1);
      fine0 = philox_fine_block((uint64_t)e0, k0, k1);
      fine1 = philox_fine_block((uint64_t)e0 + 4, k0, k1);
    }
    for (int j = 0; j < kVec; ++j) {
      const int64_t i = e0 + j;
      if (i >= end) break;
      float um, uw;
      if (noise_mode == LUMA_NOISE_PHILOX) {
        uint32_t bm, bw;
        philox_uniform_bits(coarse, j < 4 ? fine0 : fine1, (uint64_t)i, bm, bw);
        um = (float)bm * 0x1p-24f;
        uw = (float)bw * 0x1p-24f;
      } else {
        um = u_m[i];
        uw = u_w[i];
      }
      q_m[i] = (int16_t)exact_quant_m(m[i], G, um);
      q_w[i] = (int16_t)(uint16_t)exact_quant_w(v[i], G, epsf, uw);
    }
  }
}

}  // namespace luma

// ---------------------------------------------------------------------------
//  C ABI
// ---------------------------------------------------------------------------

using namespace luma;

static thread_local char g_err[512] = "";

static int fail(const char *msg, hipError_t e = hipSuccess) {
  if (e != hipSuccess)
    snprintf(g_err, sizeof(g_err), "%s: %s", msg, hipGetErrorString(e));
  else
    snprintf(g_err, sizeof(g_err), "%s", msg);
  return e != hipSuccess ? (int)e : -1;
}

static int check_launch(const char *what) {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : fail(what, e);
}

extern "C" {

int luma_abi_version(void) { return LUMA_ABI_VERSION; }

const char *luma_last_error(void) { return g_err; }

size_t luma_workspace_bytes(int32_t n_chunks) { return (size_t)(n_chunks > 0 ? n_chunks : 0) * 2 * sizeof(float); }

void luma_layout(int32_t out[8]) {
  out[0] = (int32_t)sizeof(LumaTensor);
  out[1] = (int32_t)sizeof(LumaChunk);
  out[2] = (int32_t)sizeof(LumaHyper);
  out[3] = (int32_t)sizeof(LumaScaleInit);
  out[4] = (int32_t)sizeof(LumaStepArgs);
  out[5] = (int32_t)sizeof(Slot);
  out[6] = (int32_t)LUMA_CHUNK_ELEMS;
  out[7] = 0;
}

static int step_impl(const LumaStepArgs *a, void *stream, void *const *events) {
  if (!a) return fail("luma_step: null args");
  if (a->n_tensors <= 0 || a->n_chunks <= 0) return 0;
  if (!a->tensors || !a->chunks || !a->hypers || !a->slots || !a->partials)
    return fail("luma_step: null table pointer");
  if (a->noise_mode != LUMA_NOISE_PHILOX && a->noise_mode != LUMA_NOISE_INJECTED)
    return fail("luma_step: unknown noise_mode");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const Tensor *T = reinterpret_cast<const Tensor *>(a->tensors);
  const Hyper *H = reinterpret_cast<const Hyper *>(a->hypers);
  Slot *S = static_cast<Slot *>(a->slots);
  auto mark = [&](int i) -> int {
    if (!events || !events[i]) return 0;
    const hipError_t e = hipEventRecord(static_cast<hipEvent_t>(events[i]), s);
    return e == hipSuccess ? 0 : fail("luma_step: event record", e);
  };
  if (int r = mark(0)) return r;
  hipLaunchKernelGGL(pass1_kernel, dim3(a->n_chunks), dim3(kThreads), 0, s, T, a->chunks, H, S,
                     a->partials);
  if (int r = check_launch("luma_step: pass 1 launch")) return r;
  if (int r = mark(1)) return r;
  hipLaunchKernelGGL(finalize_kernel, dim3(a->n_tensors), dim3(64), 0, s, T, H, S, a->partials);
  if (int r = check_launch("luma_step: finalize launch")) return r;
  if (int r = mark(2)) return r;
  hipLaunchKernelGGL(pass2_kernel, dim3(a->n_chunks), dim3(kThreads), 0, s, T, a->chunks, H, S,
                     a->base_seed, a->noise_mode);
  if (int r = check_launch("luma_step: pass 2 launch")) return r;
  return mark(3);
}

int luma_step(const LumaStepArgs *a, void *stream) { return step_impl(a, stream, nullptr); }

int luma_step_profiled(const LumaStepArgs *a, void *stream, void *const events[4]) {
  return step_impl(a, stream, events);
}

int luma_set_scales(void *slots, const LumaScaleInit *items, int32_t n, void *stream) {
  if (n <= 0) return 0;
  if (!slots || !items) return fail("luma_set_scales: null pointer");
  hipLaunchKernelGGL(set_scales_kernel, dim3((n + 63) / 64), dim3(64), 0,
                     static_cast<hipStream_t>(stream), static_cast<Slot *>(slots), items, n);
  return check_launch("luma_set_scales: launch");
}

int luma_get_scales(const void *slots, const int32_t *slot_idx, const int64_t *steps, int32_t n,
                    double *out, void *stream) {
  if (n <= 0) return 0;
  if (!slots || !slot_idx || !steps || !out) return fail("luma_get_scales: null pointer");
  hipLaunchKernelGGL(get_scales_kernel, dim3((n + 63) / 64), dim3(64), 0,
                     static_cast<hipStream_t>(stream), static_cast<const Slot *>(slots), slot_idx,
                     steps, n, out);
  return check_launch("luma_get_scales: launch");
}

int luma_decode(const int16_t *q_m, const int16_t *q_w, int64_t numel, const void *slots,
                int32_t slot, int64_t step, double eps, float *m_out, float *v_out, void *stream) {
  if (numel <= 0) return 0;
  if (!q_m || !q_w || !slots || !m_out || !v_out) return fail("luma_decode: null pointer");
  int64_t blocks = (numel + kThreads * 8 - 1) / (kThreads * 8);
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(decode_kernel, dim3((unsigned)blocks), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), q_m, q_w, numel,
                     static_cast<const Slot *>(slots), slot, (int)(step & 1), eps, m_out, v_out);
  return check_launch("luma_decode: launch");
}

int luma_quantize(const float *m, const float *v, int64_t numel, int16_t *q_m, int16_t *q_w,
                  void *slots, int32_t slot, int64_t step, double eps, uint64_t seed,
                  int32_t noise_mode, const float *u_m, const float *u_w, float *partials,
                  void *stream) {
  if (numel <= 0) return 0;
  if (!m || !v || !q_m || !q_w || !slots || !partials) return fail("luma_quantize: null pointer");
  if (noise_mode == LUMA_NOISE_INJECTED && (!u_m || !u_w))
    return fail("luma_quantize: injected noise needs u_m and u_w");
  if (noise_mode != LUMA_NOISE_PHILOX && noise_mode != LUMA_NOISE_INJECTED)
    return fail("luma_quantize: unknown noise_mode");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t nch = (numel + kChunk - 1) / kChunk;
  if (nch > 0x7fffffff) return fail("luma_quantize: tensor too large");
  Slot *S = static_cast<Slot *>(slots);
  const int par = (int)(step & 1);
  hipLaunchKernelGGL(quant_max_kernel, dim3((unsigned)nch), dim3(kThreads), 0, s, m, v, numel,
                     partials);
  if (int r = check_launch("luma_quantize: max launch")) return r;
  hipLaunchKernelGGL(quant_finalize_kernel, dim3(1), dim3(64), 0, s, partials, (int)nch, S, slot,
                     par, eps);
  if (int r = check_launch("luma_quantize: finalize launch")) return r;
  hipLaunchKernelGGL(quant_kernel, dim3((unsigned)nch), dim3(kThreads), 0, s, m, v, numel, q_m, q_w,
                     S, slot, par, eps, seed, noise_mode, u_m, u_w);
  return check_launch("luma_quantize: launch");
}

void luma_philox4x32(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
  const U4 o = philox4x32_10(ctr[0], ctr[1], ctr[2], ctr[3], key[0], key[1]);
  out[0] = o.x;
  out[1] = o.y;
  out[2] = o.z;
  out[3] = o.w;
}

}  // extern "C"
