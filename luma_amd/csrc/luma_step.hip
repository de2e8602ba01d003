// LUMA optimizer step for MI355X (gfx950): multi-tensor passes behind the C ABI
// of include/luma.h.
//
// One step over every parameter is three launches on the caller's stream:
//   pass 1   (grid = chunks)  decode Q_m/Q_w with the old grid, EMA with the
//                             gradient, max |m'| and max v' per chunk;
//   finalize (grid = tensors) reduce the chunk maxima to S_m', S_v', derive
//                             the new grid in float64 (functional.py:282-292),
//                             advance the tensor's step count and derive the
//                             step's scalars (functional.py:209-213, 262-264);
//   pass 2   (grid = chunks)  recompute m', v' bit-identically, AdamW update of
//                             the parameter, LogSR re-quantisation on the new
//                             grid (functional.py:278-279, 293-295).
// A chunk takes a workgroup; a medium tensor's one chunk takes a wavefront of
// the same launches (four to a workgroup).  Tensors of at most
// LUMA_SMALL_TENSOR elements take a kernel of their own in each pass (a
// wavefront per tensor, the exact path).  Nothing is materialised between the
// passes except 16 bytes per chunk.  With GradScaler's scaling (LumaScaling)
// every kernel unscales the gradients as it loads them, and returns at once
// when the overflow flag is set.
//
// Both passes take each rounding decision from fast float32 arithmetic when an
// error bound proves it equal to the exact path's (luma_fast.h), and queue
// the other elements for the exact path, 64 at a time.  Pass 2 keeps each
// wave's new preconditioner codes in LDS for a few iterations so that the
// exact codes land there before the codes go to HBM, and it streams the
// gradients, parameters and preconditioner codes non-temporally so that L2
// holds the momentum code lines.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <mutex>
#include <stdio.h>
#include <string.h>

#include "../../include/luma.h"
#include "luma_exact.h"
#include "luma_fast.h"
#include "luma_philox.h"

namespace luma {

constexpr int kThreads = 256;     // 4 wave64 per workgroup
constexpr int kVec = 8;           // consecutive elements per thread per iteration
constexpr int kItShift = 11;      // log2(kThreads * kVec): elements per workgroup iteration
static_assert((1 << kItShift) == kThreads * kVec, "kItShift");
constexpr int64_t kChunk = LUMA_CHUNK_ELEMS;
static_assert(kChunk % (kThreads * kVec) == 0, "chunk must be a whole number of iterations");
static_assert(kChunk <= (1 << 20), "chunk offsets fit the 32-bit word of a pass-2 queue entry");
static_assert(LUMA_CHUNK_ELEMS_MIN % (kThreads * kVec) == 0,
              "every chunk length must be a whole number of iterations");

// Device view of LumaTensor.  The pointer fields are declared in the global
// address space so loads and stores through them compile to global_* (not
// flat_*) instructions.
#if defined(__HIP_DEVICE_COMPILE__)
#define LUMA_GLOBAL __attribute__((address_space(1)))
#else
#define LUMA_GLOBAL
#endif
typedef float vf4 __attribute__((ext_vector_type(4)));
typedef uint32_t vu4 __attribute__((ext_vector_type(4)));

struct Tensor {
  LUMA_GLOBAL float *param;
  const LUMA_GLOBAL void *grad;
  LUMA_GLOBAL int16_t *q_m;
  LUMA_GLOBAL int16_t *q_w;
  const LUMA_GLOBAL float *u_m;
  const LUMA_GLOBAL float *u_w;
  LUMA_GLOBAL Slot *slot;
  LUMA_GLOBAL uint32_t *summary;
  int64_t summary_words;
  int64_t numel;
  int64_t param_id;
  int64_t elem_offset;
  int32_t grad_dtype;
  int32_t group;
  int32_t first_chunk;
  int32_t reserved;
};
static_assert(sizeof(Tensor) == sizeof(LumaTensor), "tensor layout");

// Where a launch finds its tensors: the device tables of luma_step, or (when
// `tensors` is null) the single tensor and group passed by value by
// luma_step_tensor, whose chunks are then the workgroups in order.  The
// chunk records come in three runs: [0, medium_from) take a workgroup each,
// [medium_from, small_from) a wavefront each (medium tensors: the pass
// kernels' workgroups from medium_from on step four such records, one per
// wavefront, through the same code), [small_from, n_chunks) the
// wavefront-per-tensor exact kernels (small tensors).
struct StepSrc {
  const Tensor *tensors;
  const LumaChunk *chunks;
  const LumaGroup *groups;
  Tensor one;
  LumaGroup group;
  LumaScaling scaling;
  int32_t chunk_shift;   // log2 of the launch's chunk length
  int32_t summaries;     // this launch's pass 2 writes the code summaries
  int32_t small_from;    // chunks from here on: small tensors, one wavefront each
  int32_t n_chunks;
  int32_t medium_from;   // chunks from here on (to small_from): medium tensors
  int32_t reserved;
};

// How a chunk's elements are shared out: among nt threads (kThreads, a whole
// workgroup; or 64, one wavefront of a medium record), tid this thread's
// index among them.  An iteration covers nt * kVec consecutive elements.
// The thread index is recomputed from threadIdx.x where it is used rather
// than held: a register live across a whole pass body costs spills.
struct Share {
  int nt;
  __device__ __forceinline__ uint32_t tid() const {
    return nt == kThreads ? threadIdx.x : threadIdx.x & 63u;
  }
};

// Elements [beg, end) of chunk ci of tensor T.
__device__ __forceinline__ void chunk_range(const StepSrc &src, const Tensor &T, int64_t ci,
                                            int64_t &beg, int64_t &end) {
  const int64_t len = (int64_t)1 << src.chunk_shift;
  beg = ci << src.chunk_shift;
  end = beg + len < T.numel ? beg + len : T.numel;
}

// GradScaler's found_inf: a nonzero value makes the whole step a no-op.
__device__ __forceinline__ bool skip_step(const StepSrc &src) {
  return src.scaling.found_inf != nullptr && *src.scaling.found_inf != 0.0f;
}

// f32(1 / (double)scale), as GradScaler computes the inverse scale.
__device__ __forceinline__ float inv_scale(const StepSrc &src) {
  return src.scaling.grad_scale ? (float)(1.0 / (double)*src.scaling.grad_scale) : 1.0f;
}

// A scaled gradient element as GradScaler.unscale_ stores it: the float32
// product with the inverse scale, rounded to nearest even in the gradient's
// own dtype (a NaN becomes the canonical bfloat16 NaN, as torch's cast does).
__device__ __forceinline__ float round_bf16(float x) {
  if (x != x) return __uint_as_float(0x7FC00000u);
  const uint32_t u = __float_as_uint(x);
  return __uint_as_float((u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u);
}

template <int GD>
__device__ __forceinline__ float unscale(float g, float inv) {
  float x = g * inv;
  // Round the product to float32 first, as torch does: left alone, the
  // compiler fuses the product and the half conversion into one
  // v_fma_mixlo_f16, which rounds once instead of twice.
  asm("" : "+v"(x));
  if (GD == LUMA_GRAD_F32) return x;
  if (GD == LUMA_GRAD_F16) return __half2float(__float2half_rn(x));
  return round_bf16(x);
}

__device__ __forceinline__ float unscale_rt(float g, float inv, int dt) {
  if (dt == LUMA_GRAD_F32) return unscale<LUMA_GRAD_F32>(g, inv);
  if (dt == LUMA_GRAD_F16) return unscale<LUMA_GRAD_F16>(g, inv);
  return unscale<LUMA_GRAD_BF16>(g, inv);
}

// The chunk of this workgroup, or from medium_from on of this wavefront:
// its record, tensor, group, chunk index and thread share.  False: the
// wavefront has no record (the last workgroup of the wavefront run, which
// ends at small_from, or with to_end at the table's end).
__device__ __forceinline__ bool chunk_job(const StepSrc &src, Tensor &T, LumaGroup &g,
                                          int64_t &index, int64_t &rec, Share &sh,
                                          bool to_end = false) {
  if (src.tensors) {
    if ((int32_t)blockIdx.x < src.medium_from) {
      rec = blockIdx.x;
      sh = Share{kThreads};
    } else {
      // wave-uniform (readfirstlane): the record and the tensor it names
      // then load through the scalar cache into scalar registers
      rec = __builtin_amdgcn_readfirstlane(
          src.medium_from + (int32_t)(blockIdx.x - (uint32_t)src.medium_from) * (kThreads / 64) +
          (int32_t)(threadIdx.x >> 6));
      if (rec >= (to_end ? src.n_chunks : src.small_from)) return false;
      sh = Share{64};
    }
    const LumaChunk c = src.chunks[rec];
    T = src.tensors[c.tensor];
    g = src.groups[T.group];
    index = c.index;
  } else {
    T = src.one;
    g = src.group;
    index = rec = blockIdx.x;
    sh = Share{kThreads};
  }
  return true;
}

// Workgroups of a pass-kernel launch: one per workgroup record, one per
// four medium records.
__device__ __host__ __forceinline__ int32_t pass_blocks(int32_t medium_from, int32_t small_from) {
  return medium_from + (small_from - medium_from + kThreads / 64 - 1) / (kThreads / 64);
}

// The tensor of this workgroup (one workgroup per tensor).
__device__ __forceinline__ void tensor_job(const StepSrc &src, Tensor &T, LumaGroup &g) {
  if (src.tensors) {
    T = src.tensors[blockIdx.x];
    g = src.groups[T.group];
  } else {
    T = src.one;
    g = src.group;
  }
}

__device__ __forceinline__ float load_grad(const LUMA_GLOBAL void *g, int64_t i, int dt) {
  if (dt == LUMA_GRAD_F32) return ((const LUMA_GLOBAL float *)g)[i];
  const uint16_t b = ((const LUMA_GLOBAL uint16_t *)g)[i];
  if (dt == LUMA_GRAD_BF16) return __uint_as_float((uint32_t)b << 16);
  return __half2float(__ushort_as_half(b));
}

// Whether tensor T takes injected uniforms: the launch asks for them and T
// has both arrays (a tensor without them draws from Philox).
__device__ __forceinline__ bool injected(const Tensor &T, int noise_mode) {
  return noise_mode == LUMA_NOISE_INJECTED && T.u_m != nullptr && T.u_w != nullptr;
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
    for (int i = 1; i < (int)(blockDim.x >> 6); ++i) {
      a = nan_max(a, sa[i]);
      b = nan_max(b, sb[i]);
    }
  }
}

// Pass 1's record of one chunk (the step's workspace, kPartialWords words
// per chunk): the exact max |m'| and max v' of the chunk and the offsets in
// the chunk of the elements that hold them (kNoArg: not known).
constexpr int kPartialWords = 4;
constexpr uint32_t kNoArg = 0xFFFFFFFFu;

__device__ __forceinline__ uint32_t lane_id() {
  return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}

__device__ __forceinline__ void put_partial(float *partials, int64_t chunk, float am, float av,
                                            uint32_t im, uint32_t iv) {
  float *p = partials + kPartialWords * chunk;
  p[0] = am;
  p[1] = av;
  p[2] = __uint_as_float(im);
  p[3] = __uint_as_float(iv);
}

// Whether (a, ia) should replace (b, ib) in a NaN-propagating max: a is
// NaN and b is not, or a > b.
__device__ __forceinline__ bool beats(float a, float b) {
  return (a != a && b == b) || a > b;
}

// Wave-wide (value, index) max; the result in every lane.
__device__ __forceinline__ void wave_argmax(float &v, uint32_t &i) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(v, off, 64);
    const uint32_t oi = (uint32_t)__shfl_xor((int)i, off, 64);
    if (beats(ov, v) || (__float_as_uint(ov) == __float_as_uint(v) && oi < i)) {
      v = ov;
      i = oi;
    }
  }
}

// Block-wide argmax of two (value, index) pairs; result valid in thread 0.
__device__ __forceinline__ void block_argmax2(float &a, uint32_t &ia, float &b, uint32_t &ib) {
  __shared__ float sa[kThreads / 64], sb[kThreads / 64];
  __shared__ uint32_t sia[kThreads / 64], sib[kThreads / 64];
  wave_argmax(a, ia);
  wave_argmax(b, ib);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  if (l == 0) {
    sa[w] = a;
    sb[w] = b;
    sia[w] = ia;
    sib[w] = ib;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < (int)(blockDim.x >> 6); ++k) {
      if (beats(sa[k], a)) {
        a = sa[k];
        ia = sia[k];
      }
      if (beats(sb[k], b)) {
        b = sb[k];
        ib = sib[k];
      }
    }
  }
}

// S' = max(max, floor) with Python's max() semantics (a NaN maximum stays NaN).
__device__ __forceinline__ double py_max(double a, double floor_) { return floor_ > a ? floor_ : a; }

// The per-tensor stage of a step, after pass 1: reduce the tensor's chunk
// records to S_m', S_v' (functional.py:282-284; init 217-219), derive the
// new grid in float64 (functional.py:74-92), advance the step count, derive
// the step's scalars (functional.py:209-213, 262-264), and keep the maxima's
// elements as the next step's seeds.
//
// The tail, by one lane: from the tensor's maxima and the elements holding
// them (-1: none), everything after the reduction.
__device__ __forceinline__ void finalize_tail(const StepSrc &src, const Tensor &T,
                                              const LumaGroup &grp, int64_t prev, float am,
                                              float av, int64_t seed_m, int64_t seed_v) {
  const double s_m = py_max((double)am, 1e-9);  // SCALE_FLOOR_M (config.py:25)
  const double s_v = py_max((double)av, 0.0);
  LUMA_GLOBAL Slot &s = *T.slot;
  const int64_t t = prev + 1;
  const int par = (int)(t & 1);
  const Hyper h = step_hyper(grp, t);
  s.s_m[par] = s_m;
  s.s_v[par] = s_v;
  Grid g;
  make_grid(s_m, s_v, grp.eps, g);
  make_fast(g, h.eps);
  s.grid[par] = g;
  s.hyp = h;
  s.step = t;
  // (only the kThreads-workgroup route writes summaries)
  s.summ_step = (src.summaries && T.summary && T.first_chunk < src.medium_from) ? t : 0;
  s.summ_shift = src.chunk_shift;
  s.seed_m = seed_m;
  s.seed_v = seed_v;
}

// The element a chunk record's offset word names (-1: none).
__device__ __forceinline__ int64_t seed_at(uint32_t chunk, uint32_t off, int32_t shift) {
  return (chunk == kNoArg || off == kNoArg) ? -1 : ((int64_t)chunk << shift) + off;
}

// One wavefront for tensor T (wave-uniform): each lane folds every 64th of
// the tensor's records, 16 loads in flight (a tensor of a few thousand
// chunks reads them in a few round trips), keeping the offset word of its
// best record, which the winning lane then hands out.
__device__ __forceinline__ void finalize_wave(const StepSrc &src, const Tensor &T,
                                              const LumaGroup &grp, const float *partials) {
  const int64_t prev = T.slot->step;   // (loaded while the records stream in)
  const uint32_t lane = lane_id();
  const int nch = (int)(((T.numel - 1) >> src.chunk_shift) + 1);
  float am = 0.0f, av = 0.0f;
  uint32_t cm = kNoArg, cv = kNoArg;   // chunk (within the tensor) of each maximum
  uint32_t om = kNoArg, ov = kNoArg;   // its offset word
  const vf4 *rec = (const vf4 *)(partials + kPartialWords * (int64_t)T.first_chunk);
  auto fold = [&](const vf4 &r, int i) {
    if (beats(r.x, am)) {
      am = r.x;
      cm = (uint32_t)i;
      om = __float_as_uint(r.z);
    }
    if (beats(r.y, av)) {
      av = r.y;
      cv = (uint32_t)i;
      ov = __float_as_uint(r.w);
    }
  };
  constexpr int kInFlight = 16;
  int i = (int)lane;
  for (; i + (kInFlight - 1) * 64 < nch; i += kInFlight * 64) {
    vf4 r[kInFlight];
#pragma unroll
    for (int k = 0; k < kInFlight; ++k) r[k] = rec[i + 64 * k];
#pragma unroll
    for (int k = 0; k < kInFlight; ++k) fold(r[k], i + 64 * k);
  }
  for (; i < nch; i += 64) fold(rec[i], i);
  // the lane that read chunk c is c % 64; wave_argmax keeps the smallest
  // chunk among equal maxima, which is that lane's own first best
  wave_argmax(am, cm);
  wave_argmax(av, cv);
  om = (uint32_t)__shfl((int)om, (int)(cm & 63u), 64);
  ov = (uint32_t)__shfl((int)ov, (int)(cv & 63u), 64);
  if (lane == 0)
    finalize_tail(src, T, grp, prev, am, av, seed_at(cm, om, src.chunk_shift),
                  seed_at(cv, ov, src.chunk_shift));
}

// Tensors of at most kLaneChunks chunks take a lane each: 64 to a wavefront,
// the float64 tail of 64 tensors side by side.  The others take a wavefront.
constexpr int kLaneChunks = 4;

__device__ __forceinline__ int tensor_chunks(const Tensor &T, int32_t shift) {
  return (int)(((T.numel - 1) >> shift) + 1);
}

// Waves [0, n_tensors): one tensor each (those of more than kLaneChunks
// chunks; the others return at once); then, from a tensor table, one lane
// per chunk record: the lane of a tensor's first record steps a tensor of at
// most kLaneChunks chunks.
__device__ __host__ inline int32_t finalize_waves(const StepSrc &src, int32_t n_tensors) {
  return n_tensors + (src.tensors ? (src.n_chunks + 63) / 64 : 0);
}

__global__ __launch_bounds__(kThreads) void finalize_kernel(StepSrc src,
                                                            const float *__restrict__ partials,
                                                            int32_t n_tensors) {
  if (skip_step(src)) return;
  const int32_t w = __builtin_amdgcn_readfirstlane((int32_t)blockIdx.x * (kThreads / 64) +
                                                   (int32_t)(threadIdx.x >> 6));
  if (w < n_tensors) {
    if (!src.tensors) {
      finalize_wave(src, src.one, src.group, partials);
      return;
    }
    const Tensor T = src.tensors[w];
    if (tensor_chunks(T, src.chunk_shift) <= kLaneChunks) return;   // a lane's (below)
    finalize_wave(src, T, src.groups[T.group], partials);
    return;
  }
  if (!src.tensors) return;
  const int64_t r = (int64_t)(w - n_tensors) * 64 + lane_id();
  if (r >= src.n_chunks) return;   // (no wave operations below)
  const Tensor T = src.tensors[src.chunks[r].tensor];
  // the tensor's first record, and few enough chunks for one lane
  if (T.first_chunk != r || tensor_chunks(T, src.chunk_shift) > kLaneChunks) return;
  const int64_t prev = T.slot->step;
  const int nch = tensor_chunks(T, src.chunk_shift);
  float am = 0.0f, av = 0.0f;
  uint32_t cm = kNoArg, cv = kNoArg, om = kNoArg, ov = kNoArg;
  for (int c = 0; c < nch; ++c) {
    const vf4 x = ((const vf4 *)partials)[r + c];
    if (beats(x.x, am)) {
      am = x.x;
      cm = (uint32_t)c;
      om = __float_as_uint(x.z);
    }
    if (beats(x.y, av)) {
      av = x.y;
      cv = (uint32_t)c;
      ov = __float_as_uint(x.w);
    }
  }
  finalize_tail(src, T, src.groups[T.group], prev, am, av, seed_at(cm, om, src.chunk_shift),
                seed_at(cv, ov, src.chunk_shift));
}

// The record of a chunk whose threads hold (am, im), (av, iv): the share's
// argmax (a workgroup's, with barriers, or a wavefront's), put by its
// thread 0.
__device__ __forceinline__ void put_chunk(float *partials, int64_t rec, const Share &sh, float am,
                                          float av, uint32_t im, uint32_t iv) {
  if (sh.nt == kThreads) {
    block_argmax2(am, im, av, iv);
  } else {
    wave_argmax(am, im);
    wave_argmax(av, iv);
  }
  if (sh.tid() == 0) put_partial(partials, rec, am, av, im, iv);
}

// m', v' of element i of tensor T (exact path).
__device__ __forceinline__ void element_ema(const Tensor &T, const Hyper &h, const Grid *old,
                                            int64_t i, bool scaled, float inv, float &mn,
                                            float &vn) {
  float g = load_grad(T.grad, i, T.grad_dtype);
  if (scaled) g = unscale_rt(g, inv, T.grad_dtype);
  float m = 0.0f, v = 0.0f;
  if (old) {  // t >= 2: decode the stored codes on the old grid
    m = exact_decode_m(T.q_m[i], old->dm);
    v = exact_decode_v(T.q_w[i], old->wmin, old->dw, h.eps);
  }
  exact_ema(m, v, g, h, mn, vn);
}

__global__ __launch_bounds__(kThreads) void pass1_exact_kernel(StepSrc src,
                                                               float *__restrict__ partials) {
  if (skip_step(src)) return;
  Tensor T;
  LumaGroup grp;
  int64_t ci, rec;
  Share sh;
  if (!chunk_job(src, T, grp, ci, rec, sh)) return;   // (wave mode: no barriers below)
  const Hyper h = group_hyper(grp);
  const bool scaled = src.scaling.grad_scale != nullptr;
  const float inv = inv_scale(src);
  // this step is t = step + 1; its decode reads the grid of step t - 1
  const int64_t prev = T.slot->step;
  const Grid *old = prev >= 1 ? (const Grid *)&T.slot->grid[prev & 1] : nullptr;
  int64_t beg, end;
  chunk_range(src, T, ci, beg, end);

  float am = 0.0f, av = 0.0f;
  uint32_t im = kNoArg, iv = kNoArg;
  for (int64_t e0 = beg + (int64_t)sh.tid() * kVec; e0 < end; e0 += (int64_t)sh.nt * kVec) {
    for (int j = 0; j < kVec; ++j) {
      const int64_t i = e0 + j;
      if (i >= end) break;
      float mn, vn;
      element_ema(T, h, old, i, scaled, inv, mn, vn);
      if (beats(fabsf(mn), am)) {
        am = fabsf(mn);
        im = (uint32_t)(i - beg);
      }
      if (beats(vn, av)) {
        av = vn;
        iv = (uint32_t)(i - beg);
      }
    }
  }
  put_chunk(partials, rec, sh, am, av, im, iv);
}

// ---------------------------------------------------------------------------
//  Small tensors: one wavefront per chunk
// ---------------------------------------------------------------------------
// The chunk records from src.small_from on belong to tensors of at most
// LUMA_SMALL_TENSOR elements, one chunk each.  Each is stepped by one
// wavefront (four per workgroup) through the exact path: a workgroup of its
// own would spend most of its time in the fast path's set-up while three of
// its four wavefronts hold the CU with nothing to do.  The exact path's codes
// are the fast path's (which certifies each of its codes against them).  The
// loops cover any chunk length, so a larger tensor routed here is stepped
// correctly, only slowly.

// The chunk of small wavefront w (w-th record from small_from on; false:
// none, the wavefront exits).
__device__ __forceinline__ bool small_job(const StepSrc &src, int64_t w, Tensor &T, LumaGroup &g,
                                          int64_t &ci, int64_t &cidx) {
  cidx = (int64_t)src.small_from + w;
  if (cidx >= src.n_chunks) return false;
  const LumaChunk c = src.chunks[cidx];
  T = src.tensors[c.tensor];
  g = src.groups[T.group];
  ci = c.index;
  return true;
}

// Workgroup b of the small tensors' launches: small wavefronts 4b .. 4b + 3.
__device__ __forceinline__ int64_t small_wave(int64_t b) {
  return b * (kThreads / 64) + (int64_t)(threadIdx.x >> 6);
}

// Pass 1 of small wavefront w.  The fast pass 1 runs it in workgroups past
// its own records (the exact-only mode in a kernel of its own), so that the
// small tensors fill the CUs that its last round of large chunks leaves
// idle.
__device__ __forceinline__ void pass1_small_body(const StepSrc &src, float *partials, int64_t w) {
  Tensor T;
  LumaGroup grp;
  int64_t ci, cidx;
  if (!small_job(src, w, T, grp, ci, cidx)) return;   // no barriers below
  const Hyper h = group_hyper(grp);
  const bool scaled = src.scaling.grad_scale != nullptr;
  const float inv = inv_scale(src);
  const int64_t prev = T.slot->step;
  const Grid *old = prev >= 1 ? (const Grid *)&T.slot->grid[prev & 1] : nullptr;
  int64_t beg, end;
  chunk_range(src, T, ci, beg, end);
  const uint32_t lane = lane_id();
  float am = 0.0f, av = 0.0f;
  uint32_t im = kNoArg, iv = kNoArg;
  // one element per lane and pass: a tensor of n elements takes
  // ceil(n / 64) passes through the exact path
  for (int64_t i = beg + (int64_t)lane; i < end; i += 64) {
    float mn, vn;
    element_ema(T, h, old, i, scaled, inv, mn, vn);
    if (beats(fabsf(mn), am)) {
      am = fabsf(mn);
      im = (uint32_t)(i - beg);
    }
    if (beats(vn, av)) {
      av = vn;
      iv = (uint32_t)(i - beg);
    }
  }
  wave_argmax(am, im);
  wave_argmax(av, iv);
  if (lane == 0) put_partial(partials, cidx, am, av, im, iv);
}

__global__ __launch_bounds__(kThreads) void pass1_small_kernel(StepSrc src,
                                                               float *__restrict__ partials) {
  if (skip_step(src)) return;
  pass1_small_body(src, partials, small_wave(blockIdx.x));
}

// The exact pass 2 of elements e0 .. min(e0 + 8, end) - 1: update, draws
// (Philox or injected), new codes.
__device__ __forceinline__ void exact_group(const Tensor &T, const Hyper &h, const Grid *old,
                                            const Grid &G, int64_t e0, int64_t end, bool scaled,
                                            float inv, bool inj, const PhiloxBase &pb, uint32_t k0,
                                            uint32_t k1) {
  U4 top_m{}, top_w{}, low{};   // e0 is a multiple of 8: one group of blocks
  if (!inj) {
    top_m = philox_block((uint64_t)e0, pb, kBlockTopM, k0, k1);
    top_w = philox_block((uint64_t)e0, pb, kBlockTopW, k0, k1);
    low = philox_block((uint64_t)e0, pb, kBlockLow, k0, k1);
  }
  for (int j = 0; j < kVec; ++j) {
    const int64_t i = e0 + j;
    if (i >= end) break;
    float mn, vn;
    element_ema(T, h, old, i, scaled, inv, mn, vn);
    T.param[i] = exact_param_update(T.param[i], mn, vn, h);
    float um, uw;
    if (!inj) {
      uint32_t bm, bw;
      philox_uniform_bits(top_m, top_w, low, (uint64_t)i, bm, bw);
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

__global__ __launch_bounds__(kThreads) void pass2_exact_kernel(StepSrc src, uint64_t base_seed,
                                                               int noise_mode) {
  if (skip_step(src)) return;
  Tensor T;
  LumaGroup grp;
  int64_t ci, rec;
  Share sh;
  if (!chunk_job(src, T, grp, ci, rec, sh)) return;
  const bool scaled = src.scaling.grad_scale != nullptr;
  const float inv = inv_scale(src);
  const Slot &S = *(const Slot *)T.slot;
  const int64_t t = S.step;   // advanced by finalize
  const Hyper h = S.hyp;
  const Grid *old = t >= 2 ? &S.grid[(t - 1) & 1] : nullptr;
  const Grid G = S.grid[t & 1];
  int64_t beg, end;
  chunk_range(src, T, ci, beg, end);
  uint32_t k0, k1;
  step_key(base_seed, t, T.param_id, k0, k1);
  const PhiloxBase pb = philox_base(T.elem_offset);
  const bool inj = injected(T, noise_mode);

  for (int64_t e0 = beg + (int64_t)sh.tid() * kVec; e0 < end; e0 += (int64_t)sh.nt * kVec)
    exact_group(T, h, old, G, e0, end, scaled, inv, inj, pb, k0, k1);
}

// Pass 2 of small wavefront w through the exact path (the exact-only mode's
// kernel; the fast pass 2 steps small tensors like medium ones).
__device__ __forceinline__ void pass2_small_body(const StepSrc &src, uint64_t base_seed,
                                                 int noise_mode, int64_t w) {
  Tensor T;
  LumaGroup grp;
  int64_t ci, cidx;
  if (!small_job(src, w, T, grp, ci, cidx)) return;
  const bool scaled = src.scaling.grad_scale != nullptr;
  const float inv = inv_scale(src);
  const Slot &S = *(const Slot *)T.slot;
  const int64_t t = S.step;   // advanced by finalize
  const Hyper h = S.hyp;
  const Grid *old = t >= 2 ? &S.grid[(t - 1) & 1] : nullptr;
  const Grid G = S.grid[t & 1];
  int64_t beg, end;
  chunk_range(src, T, ci, beg, end);
  uint32_t k0, k1;
  step_key(base_seed, t, T.param_id, k0, k1);
  const PhiloxBase pb = philox_base(T.elem_offset);
  const bool inj = injected(T, noise_mode);
  // One element per lane and pass (see pass1_small_kernel).  The 8 lanes of
  // a group of elements (beg is a multiple of 8) share its three Philox
  // blocks: lanes 0, 1 and 2 of the group evaluate T_m, L and T_w, and every
  // lane takes the words it needs from them, so each pass costs one block
  // per lane instead of three.  Every lane runs every pass (the blocks are
  // evaluated and exchanged by lanes past the end too); only lanes on an
  // element touch memory.
  const uint32_t lane = lane_id(), r = lane & 7u;
  const int first = (int)(lane & ~7u);   // lane 0 of the group
  const uint32_t stream = r == 1u ? kBlockLow : (r == 2u ? kBlockTopW : kBlockTopM);
  const uint32_t sh = (r & 1u) << 4;
  for (int64_t i0 = beg; i0 < end; i0 += 64) {
    const int64_t i = i0 + (int64_t)lane;
    uint32_t bm = 0u, bw = 0u;
    if (!inj) {
      const U4 blk = philox_block((uint64_t)i, pb, stream, k0, k1);
      // word r >> 1 of the block held by lane first + s
      auto word = [&](int s) -> uint32_t {
        const uint32_t x = (uint32_t)__shfl((int)blk.x, first + s, 64);
        const uint32_t y = (uint32_t)__shfl((int)blk.y, first + s, 64);
        const uint32_t z = (uint32_t)__shfl((int)blk.z, first + s, 64);
        const uint32_t w = (uint32_t)__shfl((int)blk.w, first + s, 64);
        return (r & 4u) ? ((r & 2u) ? w : z) : ((r & 2u) ? y : x);
      };
      const uint32_t wm = word(0), wl = word(1), ww = word(2);
      // philox_uniform_bits: half r of T_m / T_w, bytes 2r and 2r + 1 of L
      bm = (((wm >> sh) & 0xFFFFu) << 8) | ((wl >> sh) & 0xFFu);
      bw = (((ww >> sh) & 0xFFFFu) << 8) | ((wl >> (sh + 8u)) & 0xFFu);
    }
    if (i >= end) continue;
    float mn, vn;
    element_ema(T, h, old, i, scaled, inv, mn, vn);
    T.param[i] = exact_param_update(T.param[i], mn, vn, h);
    const float um = inj ? T.u_m[i] : (float)bm * 0x1p-24f;
    const float uw = inj ? T.u_w[i] : (float)bw * 0x1p-24f;
    T.q_m[i] = (int16_t)exact_quant_m(mn, G, um);
    T.q_w[i] = (int16_t)(uint16_t)exact_quant_w(vn, G, h.eps, uw);
  }
}

__global__ __launch_bounds__(kThreads) void pass2_small_kernel(StepSrc src, uint64_t base_seed,
                                                               int noise_mode) {
  if (skip_step(src)) return;
  pass2_small_body(src, base_seed, noise_mode, small_wave(blockIdx.x));
}

// ---------------------------------------------------------------------------
//  Fast path: 8 consecutive elements per thread per iteration, 16-byte
//  loads/stores, certified decisions, exact fallback for flagged elements.
// ---------------------------------------------------------------------------

struct Group8 {
  int qm[kVec];   // signed momentum codes
  int qw[kVec];   // unsigned preconditioner codes, as kCodeFloat | code
  float g[kVec];  // gradient promoted to float32
};

__device__ __forceinline__ void unpack_i16(uint32_t w, int &lo, int &hi) {
  lo = (int)(int16_t)(w & 0xFFFFu);
  hi = (int)w >> 16;
}

// Preconditioner codes are kept as the bits of the float 2^23 + q
// (kCodeFloat | q): their decode then needs no v_cvt, see fast_ema.  The
// low 16 bits are the code.
constexpr uint32_t kCodeFloat = 0x4B000000u;

__device__ __forceinline__ void unpack_u16(uint32_t w, int &lo, int &hi) {
  lo = (int)((w & 0xFFFFu) | kCodeFloat);
  hi = (int)((w >> 16) | kCodeFloat);
}

template <int GD>
__device__ __forceinline__ float grad_lo(uint32_t w) {
  if (GD == LUMA_GRAD_BF16) return __uint_as_float(w << 16);
  return __half2float(__ushort_as_half((uint16_t)(w & 0xFFFFu)));
}

template <int GD>
__device__ __forceinline__ float grad_hi(uint32_t w) {
  if (GD == LUMA_GRAD_BF16) return __uint_as_float(w & 0xFFFF0000u);
  return __half2float(__ushort_as_half((uint16_t)(w >> 16)));
}

// Cache policy of the streams.  The gradients, and pass 2's parameters, are
// touched once per step: they are loaded (and stored) non-temporally, so that
// they are the first lines L2 evicts.  So are pass 2's preconditioner codes,
// which reach HBM only as whole staged vectors.  The momentum codes keep the
// normal policy: pass 2 overwrites some of its new momentum codes again after
// the exact path has run for them, some iterations later, and those late
// 2-byte stores are cheap while the line is still in L2 but cost a
// partial-line write-back to HBM once it has been evicted.
template <typename V>
__device__ __forceinline__ V load_stream(const LUMA_GLOBAL V *p) {
  return __builtin_nontemporal_load(p);
}

template <typename V>
__device__ __forceinline__ void store_stream(V v, LUMA_GLOBAL V *p) {
  __builtin_nontemporal_store(v, p);
}

// The 16-byte words holding the codes and gradients of 8 consecutive
// elements, as loaded (g1: float32 gradients only).  Pass 1 streams the
// gradients non-temporally (about 8% faster than the normal policy).
struct Raw8 {
  vu4 qm, qw, g0, g1;
};

template <int GD>
__device__ __forceinline__ void load_raw(const Tensor &T, int64_t e0, Raw8 &r) {
  r.qm = *(const LUMA_GLOBAL vu4 *)(T.q_m + e0);
  r.qw = *(const LUMA_GLOBAL vu4 *)(T.q_w + e0);
  if (GD == LUMA_GRAD_F32) {
    r.g0 = load_stream((const LUMA_GLOBAL vu4 *)((const LUMA_GLOBAL float *)T.grad + e0));
    r.g1 = load_stream((const LUMA_GLOBAL vu4 *)((const LUMA_GLOBAL float *)T.grad + e0 + 4));
  } else {
    r.g0 = load_stream((const LUMA_GLOBAL vu4 *)((const LUMA_GLOBAL uint16_t *)T.grad + e0));
  }
}

template <int GD>
__device__ __forceinline__ void unpack_raw(const Raw8 &r, Group8 &G) {
  unpack_i16(r.qm.x, G.qm[0], G.qm[1]);
  unpack_i16(r.qm.y, G.qm[2], G.qm[3]);
  unpack_i16(r.qm.z, G.qm[4], G.qm[5]);
  unpack_i16(r.qm.w, G.qm[6], G.qm[7]);
  unpack_u16(r.qw.x, G.qw[0], G.qw[1]);
  unpack_u16(r.qw.y, G.qw[2], G.qw[3]);
  unpack_u16(r.qw.z, G.qw[4], G.qw[5]);
  unpack_u16(r.qw.w, G.qw[6], G.qw[7]);
  if (GD == LUMA_GRAD_F32) {
    G.g[0] = __uint_as_float(r.g0.x); G.g[1] = __uint_as_float(r.g0.y);
    G.g[2] = __uint_as_float(r.g0.z); G.g[3] = __uint_as_float(r.g0.w);
    G.g[4] = __uint_as_float(r.g1.x); G.g[5] = __uint_as_float(r.g1.y);
    G.g[6] = __uint_as_float(r.g1.z); G.g[7] = __uint_as_float(r.g1.w);
  } else {
    G.g[0] = grad_lo<GD>(r.g0.x); G.g[1] = grad_hi<GD>(r.g0.x);
    G.g[2] = grad_lo<GD>(r.g0.y); G.g[3] = grad_hi<GD>(r.g0.y);
    G.g[4] = grad_lo<GD>(r.g0.z); G.g[5] = grad_hi<GD>(r.g0.z);
    G.g[6] = grad_lo<GD>(r.g0.w); G.g[7] = grad_hi<GD>(r.g0.w);
  }
}

// Load the codes and gradients of elements e0 .. e0+7 (n of them valid).
// STREAM: the gradient and preconditioner-code vectors are loaded non-temporally.
template <int GD, bool STREAM = false>
__device__ __forceinline__ void load_group(const Tensor &T, int64_t e0, int n, bool vec, Group8 &G) {
  if (vec) {
    const vu4 a = *(const LUMA_GLOBAL vu4 *)(T.q_m + e0);
    const vu4 b = STREAM ? load_stream((const LUMA_GLOBAL vu4 *)(T.q_w + e0)) : *(const LUMA_GLOBAL vu4 *)(T.q_w + e0);
    unpack_i16(a.x, G.qm[0], G.qm[1]);
    unpack_i16(a.y, G.qm[2], G.qm[3]);
    unpack_i16(a.z, G.qm[4], G.qm[5]);
    unpack_i16(a.w, G.qm[6], G.qm[7]);
    unpack_u16(b.x, G.qw[0], G.qw[1]);
    unpack_u16(b.y, G.qw[2], G.qw[3]);
    unpack_u16(b.z, G.qw[4], G.qw[5]);
    unpack_u16(b.w, G.qw[6], G.qw[7]);
    if (GD == LUMA_GRAD_F32) {
      const LUMA_GLOBAL vf4 *gp = (const LUMA_GLOBAL vf4 *)((const LUMA_GLOBAL float *)T.grad + e0);
      const vf4 g0 = STREAM ? load_stream(gp) : gp[0];
      const vf4 g1 = STREAM ? load_stream(gp + 1) : gp[1];
      G.g[0] = g0.x; G.g[1] = g0.y; G.g[2] = g0.z; G.g[3] = g0.w;
      G.g[4] = g1.x; G.g[5] = g1.y; G.g[6] = g1.z; G.g[7] = g1.w;
    } else {
      const LUMA_GLOBAL vu4 *gp = (const LUMA_GLOBAL vu4 *)((const LUMA_GLOBAL uint16_t *)T.grad + e0);
      const vu4 gw = STREAM ? load_stream(gp) : gp[0];
      G.g[0] = grad_lo<GD>(gw.x); G.g[1] = grad_hi<GD>(gw.x);
      G.g[2] = grad_lo<GD>(gw.y); G.g[3] = grad_hi<GD>(gw.y);
      G.g[4] = grad_lo<GD>(gw.z); G.g[5] = grad_hi<GD>(gw.z);
      G.g[6] = grad_lo<GD>(gw.w); G.g[7] = grad_hi<GD>(gw.w);
    }
  } else {
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      const bool ok = j < n;
      G.qm[j] = ok ? (int)T.q_m[e0 + j] : 0;
      G.qw[j] = (int)((ok ? (uint32_t)(uint16_t)T.q_w[e0 + j] : 0u) | kCodeFloat);
      G.g[j] = ok ? load_grad(T.grad, e0 + j, GD) : 0.0f;
    }
  }
}

__device__ __forceinline__ bool tensor_vec_ok(const Tensor &T) {
  const uintptr_t bits = (uintptr_t)T.param | (uintptr_t)T.grad | (uintptr_t)T.q_m |
                         (uintptr_t)T.q_w | (uintptr_t)T.u_m | (uintptr_t)T.u_w;
  return (bits & 15u) == 0;
}

// Exact path for one element, kept out of line so that its float64 constants
// are not hoisted into (and do not crowd) the registers of the fast loops.
// Takes the element's old codes and gradient; returns (m', v').
__device__ __noinline__ float2 exact_mv(int qm, int qw, float g, const LUMA_GLOBAL Grid *old,
                                        Hyper h) {
  float m = 0.0f, v = 0.0f;
  if (old) {
    m = exact_decode_m(qm, old->dm);
    v = exact_decode_v(qw, old->wmin, old->dw, h.eps);
  }
  float mn, vn;
  exact_ema(m, v, g, h, mn, vn);
  return make_float2(mn, vn);
}

// New code of one element before its draw is final (exact path): the
// 16-bit code when the uniform u >= p (lo) and when u < p (hi), and the
// argument a of p = exact_sr_prob(a, z).  The caller knows u to an interval
// [ulo, uhi] (the injected u itself, or with Philox the interval of its
// top 16 bits); codes that interval decides come back as lo = hi.  p is first
// bracketed without the double expm1, which then runs only when the bracket
// overlaps the interval.  Returned packed in one 64-bit value (lo | hi << 16
// | bits(a) << 32) so that the call needs no stack.
struct CodePair {
  int lo, hi;
  float a;
};

__device__ __forceinline__ uint64_t pack_pair(int lo, int hi, float a) {
  return (uint64_t)(((uint32_t)lo & 0xFFFFu) | (((uint32_t)hi & 0xFFFFu) << 16)) |
         ((uint64_t)__float_as_uint(a) << 32);
}

__device__ __forceinline__ CodePair unpack_pair(uint64_t v) {
  CodePair c;
  c.lo = (int)(v & 0xFFFFu);
  c.hi = (int)((v >> 16) & 0xFFFFu);
  c.a = __uint_as_float((uint32_t)(v >> 32));
  return c;
}

__device__ __forceinline__ uint64_t sr_resolve(int lo, int hi, float a, float z, float ulo,
                                               float uhi) {
  if (lo == hi) return pack_pair(lo, lo, 0.0f);
  float pl, ph;
  if (!sr_prob_bracket(a, z, pl, ph)) pl = ph = exact_sr_prob(a, z);
  if (uhi < pl) return pack_pair(hi, hi, 0.0f);     // u <= uhi < pl <= p
  if (!(ulo < ph)) return pack_pair(lo, lo, 0.0f);  // u >= ulo >= ph >= p (NaN p: lo)
  if (ulo == uhi) {                                  // u known: p itself decides
    const float p = pl == ph ? pl : exact_sr_prob(a, z);
    return ulo < p ? pack_pair(hi, hi, 0.0f) : pack_pair(lo, lo, 0.0f);
  }
  return pack_pair(lo, hi, a);   // the caller draws u's low bits (sr_below)
}

// u < exact_sr_prob(a, z) for a u known exactly; the double expm1 runs only
// when u falls inside sr_prob_bracket's bracket.  A call, so that the
// streaming loops keep their registers.
template <int KTAG>
__device__ __noinline__ bool sr_below(float a, float z, float u) {
  float pl, ph;
  if (!sr_prob_bracket(a, z, pl, ph)) return u < exact_sr_prob(a, z);
  if (u < pl) return true;
  if (!(u < ph)) return false;
  return u < exact_sr_prob(a, z);
}

// Momentum: the same float32 sequence as exact_mv's m' then exact_quant_m.
template <int KTAG>
__device__ __noinline__ uint64_t exact_pair_m(int qm, float g, const LUMA_GLOBAL Grid *old,
                                              const LUMA_GLOBAL Grid *nw, Hyper h, float ulo,
                                              float uhi) {
  const float m = old ? exact_decode_m(qm, old->dm) : 0.0f;
  const float mn = h.beta1 * m + h.omb1 * g;
  const Grid G = *nw;
  float a;
  int lo, hi;
  exact_quant_m_pair(mn, G, a, lo, hi);
  return sr_resolve(lo, hi, a, G.zm, ulo, uhi);
}

// Preconditioner: exact_mv's v' then exact_quant_w.
template <int KTAG>
__device__ __noinline__ uint64_t exact_pair_w(int qw, float g, const LUMA_GLOBAL Grid *old,
                                              const LUMA_GLOBAL Grid *nw, Hyper h, float ulo,
                                              float uhi) {
  const float v = old ? exact_decode_v(qw, old->wmin, old->dw, h.eps) : 0.0f;
  const float vn = h.beta2 * v + h.omb2 * (g * g);
  const Grid G = *nw;
  float a;
  int lo, hi;
  exact_quant_w_pair(vn, G, h.eps, a, lo, hi);
  return sr_resolve(lo, hi, a, G.zw, ulo, uhi);
}

// Per-wave queues of elements whose fast result is not certified.  Elements
// are appended without atomics (pass 1: ballot/mbcnt per element slot;
// pass 2: one wave prefix sum per iteration) and run through the exact path
// 64 at a time, one per lane, so the exact path runs at full SIMD width.
// Pass 1 appends up to 8 x 64 entries before it drains its queue.  Pass 2's
// queues are rings of 256 entries drained oldest first, 64 at a time, after
// every iteration; an iteration whose entries would not fit runs them in
// place.  Oldest first, because the exact codes are stored into lines that
// the fast path wrote some iterations earlier, and a younger line is more
// likely to still be in L2.
constexpr int kQueueCap = kVec * 64 + 64;
constexpr int kQueueCapW = 256;   // pass 2 preconditioner ring (entries)
constexpr int kQueueCapM = 64;    // pass 2 momentum ring (uncertain codes are rare)
static_assert((kQueueCapW & (kQueueCapW - 1)) == 0 && (kQueueCapM & (kQueueCapM - 1)) == 0,
              "pass 2 queues are power-of-two rings");
// Pass 2 stages the new preconditioner codes of its last kStage iterations
// in LDS (one 16-byte group per lane per iteration) and writes an
// iteration's codes to HBM only once its queued exact codes are in: the
// exact codes then land in LDS instead of in lines already written back.
// With about 9 uncertain preconditioner codes per wave iteration, the ring
// fills a 64-entry batch every 7 iterations, so 8 slots seldom force a
// partial batch.  LDS per workgroup: 4 x (64 + 256 + 8 x 64) x 16 B = 52 KB,
// so three workgroups (the VGPR limit) still fit a CU's 160 KB.
constexpr int kStage = 8;
// LDS entries (16 bytes) of one pass-2 wavefront: both queues and the ring.
constexpr int kWaveLds = kQueueCapM + kQueueCapW + kStage * 64;

// Keeps a wave-uniform value in a VGPR.  On gfx950 a VALU instruction with
// an SGPR source operand issues at about half the rate of one whose sources
// are VGPRs, inline constants or literals (measured: 0.95 vs 1.5-1.8 wave
// instructions per clock per CU), so the streaming loops read their
// per-tensor constants from VGPRs.  The empty asm makes the value opaque,
// which stops the compiler from re-reading it from the SGPR.
template <typename V>
__device__ __forceinline__ V in_vgpr(V x) {
  asm("" : "+v"(x));
  return x;
}

// Position of this lane's entry among the lanes of `mask`, offset by base.
__device__ __forceinline__ uint32_t queue_pos(uint64_t mask, uint32_t base) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, base));
}

// Decode constants of the fast path.  At t = 1 there is nothing to decode:
// all-zero constants make the fast decode return m = v = 0 exactly whatever
// the (uninitialised) codes are, so the loops carry no branch for it.
struct DecodeK {
  float dm, dw, iwmin, eps;
};

__device__ __forceinline__ DecodeK decode_consts(const LUMA_GLOBAL Grid *old, float eps) {
  DecodeK k;
  k.dm = old ? old->dm : 0.0f;
  k.dw = old ? old->dw : 0.0f;
  k.iwmin = old ? old->fast[kIwmin] : 0.0f;
  k.eps = old ? eps : 0.0f;
  return k;
}

// Candidate threshold for a running fast maximum M (float bits): elements
// whose fast value is below it are provably not the exact maximum.  A NaN
// maximum gives threshold 0 (every element becomes a candidate).
__device__ __forceinline__ uint32_t threshold_bits(uint32_t M, float lo, float sub, float hi) {
  const float t = (__uint_as_float(M) * lo - sub) * hi;
  return t > 0.0f ? __float_as_uint(t) : 0u;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, off, 64));
  return v;
}

// Fast |m'| and v' of 8 consecutive elements as float bit patterns (for
// non-negative floats the unsigned order is the float order, with every NaN
// above +Inf); invalid elements of a partial group give 0.
// Constants of the pass-1 loop, kept in VGPRs (see in_vgpr).
struct P1Const {
  float dm, ndw, nbias, iwmin, eps, b1, omb1, b2, omb2;
  float up_m, up_v, abs_v;   // pruning margins: 1 + 8u, 1 + 16u, eps^2 * 1e-10
  float inv;   // inverse gradient scale (SCALED)
  uint32_t sign;
};

// Unscales a group's gradients in place (SCALED launches only).
template <int GD, bool SCALED>
__device__ __forceinline__ void unscale_group(Group8 &G, float inv) {
  if (!SCALED) return;
#pragma unroll
  for (int j = 0; j < kVec; ++j) G.g[j] = unscale<GD>(G.g[j], inv);
}

// FULL: the group is whole and aligned, and raw already holds its codes
// and gradients; the iteration reloads raw with the group it will process
// next (en: elements en .. en+7), so that the load overlaps this group's
// arithmetic.
// PRUNE (FULL only): first bound every fast |m'| and v' of the lane's group
// by the fast formulas at its largest |q_m|, smallest q_w and largest |g|
// (each formula is non-decreasing in those, up to the few-ulp wobble of the
// hardware exp2 that the margins cover).  When that bound is below the
// thresholds Tm / Tv in every lane, no element of the iteration can be a
// candidate and its per-element decode is skipped (am = av = 0).
// Bound on the fast |m'| and v' of every element whose momentum code
// magnitude is at most qa, preconditioner code at least qw_lo (kCodeFloat |
// code) and gradient magnitude at most gb (float bits): the fast formulas
// at those extremes (each non-decreasing in them, up to the few-ulp wobble
// of the hardware exp2 that the margins cover).  Returns whether some lane's
// bound reaches the thresholds Tm / Tv (float bits, wave-uniform).
template <bool SMALL>
__device__ __forceinline__ bool p1_reach(int qa, int qw_lo, uint32_t gb, const P1Const &K,
                                         uint32_t Tm, uint32_t Tv) {
  const FastEma fb = fast_ema<SMALL ? kRegSmall : kRegGeneral, false>(qa, qw_lo, __uint_as_float(gb), K.dm, K.ndw, K.nbias,
                                            K.iwmin, K.eps, K.b1, K.omb1, K.b2, K.omb2, K.sign);
  const uint32_t um = __float_as_uint(fb.mn * K.up_m) & 0x7FFFFFFFu;
  const uint32_t uv = __float_as_uint(fmaf(fb.vn, K.up_v, K.abs_v)) & 0x7FFFFFFFu;
  return __ballot(um >= Tm || uv >= Tv) != 0;
}

typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t max_u16x2(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, a),
                                                                __builtin_bit_cast(u16x2, b)));
}

// Largest gradient magnitude of the 8 raw gradients in r, unscaled (the
// magnitude order of float32, bfloat16 and float16 bit patterns is their
// integer order, NaN above +Inf, and unscaling is monotone, so only the
// largest is unscaled).  16-bit gradients: packed 16-bit max, two per
// instruction.
template <int GD, bool SCALED>
__device__ __forceinline__ float raw_gmax(const Raw8 &r, float inv) {
  float g;
  if (GD == LUMA_GRAD_F32) {
    const uint32_t m = max(max(max(r.g0.x & 0x7FFFFFFFu, r.g0.y & 0x7FFFFFFFu),
                               max(r.g0.z & 0x7FFFFFFFu, r.g0.w & 0x7FFFFFFFu)),
                           max(max(r.g1.x & 0x7FFFFFFFu, r.g1.y & 0x7FFFFFFFu),
                               max(r.g1.z & 0x7FFFFFFFu, r.g1.w & 0x7FFFFFFFu)));
    g = __uint_as_float(m);
  } else {
    const uint32_t x = r.g0.x & 0x7FFF7FFFu, y = r.g0.y & 0x7FFF7FFFu;
    const uint32_t z = r.g0.z & 0x7FFF7FFFu, w = r.g0.w & 0x7FFF7FFFu;
    const uint32_t m2 = max_u16x2(max_u16x2(x, y), max_u16x2(z, w));
    const uint32_t m = max(m2 & 0xFFFFu, m2 >> 16);
    g = grad_lo<GD>(m);
  }
  if (SCALED) g = unscale<GD>(g, inv);
  return g;
}

// Largest gradient magnitude of a group, as float bits (NaN above +Inf).
__device__ __forceinline__ uint32_t group_gmax(const Group8 &G) {
  uint32_t gb = 0;
#pragma unroll
  for (int j = 0; j < kVec; ++j) gb = max(gb, __float_as_uint(G.g[j]) & 0x7FFFFFFFu);
  return gb;
}

// Fast |m'| and v' (float bits) of a group whose codes and gradients are in
// G; elements j >= n give 0.  PRUNE: first the group bound at the lane's own
// code extremes; when no lane reaches the thresholds, every value is 0 (no
// element of the iteration can be a candidate) and the per-element decode is
// skipped.
template <bool SMALL, bool PRUNE>
__device__ __forceinline__ void p1_compute(const Group8 &G, const P1Const &K, int n, uint32_t Tm,
                                           uint32_t Tv, uint32_t (&am)[kVec], uint32_t (&av)[kVec]) {
  if (PRUNE) {
    int qa = 0, qw_lo = G.qw[0];
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      qa = max(qa, abs(G.qm[j]));
      qw_lo = min(qw_lo, G.qw[j]);   // kCodeFloat | code: ordered as the codes
    }
    if (!p1_reach<SMALL>(qa, qw_lo, group_gmax(G), K, Tm, Tv)) {
#pragma unroll
      for (int j = 0; j < kVec; ++j) am[j] = av[j] = 0u;
      return;
    }
  }
#pragma unroll
  for (int j = 0; j < kVec; ++j) {
    const FastEma f = fast_ema<SMALL ? kRegSmall : kRegGeneral, false>(G.qm[j], G.qw[j], G.g[j], K.dm, K.ndw, K.nbias, K.iwmin,
                                             K.eps, K.b1, K.omb1, K.b2, K.omb2, K.sign);
    am[j] = __float_as_uint(f.mn) & 0x7FFFFFFFu;
    av[j] = __float_as_uint(f.vn) & 0x7FFFFFFFu;
    if (j >= n) am[j] = av[j] = 0u;
  }
}

template <int GD, bool SMALL, bool SCALED, bool FULL, bool PRUNE>
__device__ __forceinline__ void p1_iter(const Tensor &T, const P1Const &K, int64_t e0, int n,
                                        Raw8 &raw, int64_t en, uint32_t Tm, uint32_t Tv,
                                        uint32_t (&am)[kVec], uint32_t (&av)[kVec]) {
  Group8 G;
  if (FULL) {
    unpack_raw<GD>(raw, G);
    load_raw<GD>(T, en, raw);
  } else {
    load_group<GD>(T, e0, n, false, G);
  }
  unscale_group<GD, SCALED>(G, K.inv);
  p1_compute<SMALL, PRUNE>(G, K, FULL ? kVec : n, Tm, Tv, am, av);
}

// The gradient words of 8 consecutive elements (g1: float32 gradients only),
// and their unpacking into G.g.
template <int GD>
__device__ __forceinline__ void load_grads(const Tensor &T, int64_t e0, Raw8 &r) {
  if (GD == LUMA_GRAD_F32) {
    r.g0 = load_stream((const LUMA_GLOBAL vu4 *)((const LUMA_GLOBAL float *)T.grad + e0));
    r.g1 = load_stream((const LUMA_GLOBAL vu4 *)((const LUMA_GLOBAL float *)T.grad + e0 + 4));
  } else {
    r.g0 = load_stream((const LUMA_GLOBAL vu4 *)((const LUMA_GLOBAL uint16_t *)T.grad + e0));
  }
}

template <int GD>
__device__ __forceinline__ void unpack_grads(const Raw8 &r, Group8 &G) {
  if (GD == LUMA_GRAD_F32) {
    G.g[0] = __uint_as_float(r.g0.x); G.g[1] = __uint_as_float(r.g0.y);
    G.g[2] = __uint_as_float(r.g0.z); G.g[3] = __uint_as_float(r.g0.w);
    G.g[4] = __uint_as_float(r.g1.x); G.g[5] = __uint_as_float(r.g1.y);
    G.g[6] = __uint_as_float(r.g1.z); G.g[7] = __uint_as_float(r.g1.w);
  } else {
    G.g[0] = grad_lo<GD>(r.g0.x); G.g[1] = grad_hi<GD>(r.g0.x);
    G.g[2] = grad_lo<GD>(r.g0.y); G.g[3] = grad_hi<GD>(r.g0.y);
    G.g[4] = grad_lo<GD>(r.g0.z); G.g[5] = grad_hi<GD>(r.g0.z);
    G.g[6] = grad_lo<GD>(r.g0.w); G.g[7] = grad_hi<GD>(r.g0.w);
  }
}

// Pass 1 body (t >= 2, old != null): exact max |m'| and max v' of the chunk.  The wave keeps a
// running maximum of the fast values and from it a certified lower bound of
// the exact maximum (the threshold, uniform across the wave).  An element
// whose fast value is below the threshold cannot be the exact maximum; the
// others (in practice a few per chunk) go through the wave's queue to the
// exact path.
// SUMM: the tensor's code summaries of the previous step are valid (and
// old != null, the tensor 16-byte aligned).  Then each whole-group
// iteration first bounds its block from the summary and the gradients, and
// loads the block's codes only when some lane's bound reaches the
// thresholds: most blocks cost their gradients alone.
template <int GD, bool SMALL, bool SCALED, bool SUMM, int NT>
__device__ void pass1_fast_body(const Tensor &T, const Hyper &h, const LUMA_GLOBAL Grid *old,
                                float inv, int64_t ci, int64_t beg, int64_t end, float &exm,
                                float &exv, uint32_t &exi_m, uint32_t &exi_v, uint32_t *queue,
                                Share sh) {
  // Threads per chunk: kThreads, or one wavefront for a medium tensor; an
  // iteration covers nt * kVec consecutive elements.
  constexpr int nt = NT;
  constexpr int it_shift = NT == kThreads ? kItShift : kItShift - 2;  // 64 = kThreads / 4
  static_assert(NT == kThreads || NT == 64, "a workgroup or one wavefront per chunk");
  const int64_t kStride = (int64_t)1 << it_shift;
  const int n_it = (int)((end - beg + kStride - 1) >> it_shift);
  const bool vec_ok = tensor_vec_ok(T);
  // Iterations in which every lane's group is whole run in a loop of their
  // own that loads each group one iteration ahead (below).
  // (uniform: readfirstlane keeps the loop's group offsets in SGPRs)
  const int n_whole = __builtin_amdgcn_readfirstlane(vec_ok ? (int)((end - beg) >> it_shift) : 0);
  auto group_at = [&](int j) {
    return beg + ((int64_t)(j < n_whole ? j : n_whole - 1) * nt + sh.tid()) * kVec;
  };
  // The first group's loads (and with SUMM the thread's summary word) go
  // out before the per-tensor constants are derived, so that their latency
  // covers that arithmetic.
  static_assert(LUMA_SUMMARY_WORDS == kThreads, "one summary word per thread of a chunk");
  Raw8 ra, rb, rc;
  uint32_t sw = 0;
  if (n_whole > 0) {
    if (SUMM) {
      sw = T.summary[ci * LUMA_SUMMARY_WORDS + sh.tid()];
      load_grads<GD>(T, group_at(0), ra);
      load_grads<GD>(T, group_at(1), rb);
    } else {
      load_raw<GD>(T, beg + (int64_t)sh.tid() * kVec, ra);
    }
  }
  const Bounds B = make_bounds((const Grid *)old, nullptr, h.beta1, h.beta2);
  const DecodeK D = decode_consts(old, h.eps);
  P1Const K;
  // (the constants stay where the compiler puts them, in SGPRs: pass 1
  // waits on memory, not on issue, and the VGPRs hold its loads in flight)
  K.dm = (D.dm);
  K.ndw = (-D.dw);
  K.nbias = (8388608.0f * D.dw);
  K.iwmin = (D.iwmin);
  K.eps = (D.eps);
  K.b1 = (h.beta1);
  K.omb1 = (h.omb1);
  K.b2 = (h.beta2);
  K.omb2 = (h.omb2);
  K.inv = (inv);
  K.sign = (0x80000000u);
  // 8u covers the rounding of the bound's own products and the non-monotone
  // wobble of the hardware exp2 / of the expm1 branch switch (a few ulp);
  // abs_v covers decodes whose 1/w - eps rounds slightly below zero
  // (|rr| <= 4u eps, so rr^2 <= 1e-13 eps^2)
  K.up_m = (1.0f + 8.0f * kU);
  K.up_v = (1.0f + 16.0f * kU);
  K.abs_v = (D.eps * D.eps * 1e-10f);
  const float lo_m = 1.0f - B.dlt_m, hi_m = 1.0f / (1.0f + B.dlt_m);
  const float lo_v = 1.0f - B.dlt_v, hi_v = 1.0f / (1.0f + B.dlt_v);
  const float sub_m = 2.0f * B.abs_m, sub_v = 2.0f * B.abs_v;
  const uint32_t lane = lane_id();
  uint32_t Mm = 0, Mv = 0, Tm = 0, Tv = 0;  // wave maxima / thresholds (bits)
  uint32_t T0m = 0, T0v = 0;                 // thresholds from the seeds (below)
  uint32_t qlen = 0;
  // exact m', v' of element i (any element of the tensor)
  auto exact_at = [&](int64_t i) -> float2 {
    float g = load_grad(T.grad, i, GD);
    if (SCALED) g = unscale<GD>(g, inv);
    return exact_mv(T.q_m[i], (int)(uint16_t)T.q_w[i], g, old, h);
  };
  auto run = [&](uint32_t off) {
    const float2 e = exact_at(beg + off);
    if (beats(fabsf(e.x), exm)) {
      exm = fabsf(e.x);
      exi_m = off;
    }
    if (beats(e.y, exv)) {
      exv = e.y;
      exi_v = off;
    }
  };
  // The fast values of one iteration: fold them into the wave maximum and
  // queue the candidates.
  auto take = [&](int64_t e0, int n, const uint32_t (&am)[kVec], const uint32_t (&av)[kVec]) {
    const uint32_t im = max(max(max(am[0], am[1]), max(am[2], am[3])),
                            max(max(am[4], am[5]), max(am[6], am[7])));
    const uint32_t iv = max(max(max(av[0], av[1]), max(av[2], av[3])),
                            max(max(av[4], av[5]), max(av[6], av[7])));
    if (!__ballot(im >= Tm || iv >= Tv)) return;
    // some lane reached the threshold: raise the wave maximum, then queue
    // the elements that still reach the new threshold
    Mm = max(Mm, wave_max_u32(im));
    Mv = max(Mv, wave_max_u32(iv));
    Tm = max(T0m, threshold_bits(Mm, lo_m, sub_m, hi_m));
    Tv = max(T0v, threshold_bits(Mv, lo_v, sub_v, hi_v));
    const uint32_t off0 = (uint32_t)(e0 - beg);
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      const bool f = (am[j] >= Tm || av[j] >= Tv) && j < n;
      const uint64_t bm = __ballot(f);
      if (f) queue[queue_pos(bm, qlen)] = off0 + j;
      qlen += (uint32_t)__popcll(bm);
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    while (qlen >= 64) {
      qlen -= 64;
      run(queue[qlen + lane]);
    }
  };
  // Seeds: the elements that held the tensor's maxima at the previous step
  // (recorded by its finalize), wherever they lie in the tensor.  The fast
  // value at such an element gives a threshold as a running maximum does
  // (an element whose fast value is below it has an exact value below the
  // seed's, so it is not the tensor's maximum, and the seed's own fast value
  // is above it), so the thresholds start high: blocks below them are
  // skipped from the first iteration.  Every lane loads the momentum seed
  // (even lanes) or the preconditioner seed (odd lanes); the loads are
  // issued before the first group's, which they do not wait for.
  const LUMA_GLOBAL Slot &S = *T.slot;
  const int64_t si = (lane & 1u) ? S.seed_v : S.seed_m;
  const bool s_ok = si >= 0 && si < T.numel;
  const int64_t sj = s_ok ? si : 0;
  const int s_qm = (int)T.q_m[sj];
  const int s_qw = (int)((uint32_t)(uint16_t)T.q_w[sj] | kCodeFloat);
  const float s_g = load_grad(T.grad, sj, GD);
  auto seed_thresholds = [&]() {
    float g = s_g;
    if (SCALED) g = unscale<GD>(g, inv);
    const FastEma f = fast_ema<SMALL ? kRegSmall : kRegGeneral, false>(
        s_qm, s_qw, g, K.dm, K.ndw, K.nbias, K.iwmin, K.eps, K.b1, K.omb1, K.b2, K.omb2, K.sign);
    const uint32_t xb = s_ok ? (__float_as_uint((lane & 1u) ? f.vn : f.mn) & 0x7FFFFFFFu) : 0u;
    T0m = threshold_bits((uint32_t)__shfl((int)xb, 0, 64), lo_m, sub_m, hi_m);
    T0v = threshold_bits((uint32_t)__shfl((int)xb, 1, 64), lo_v, sub_v, hi_v);
    Tm = T0m;
    Tv = T0v;
  };
  // Every lane of a wave runs the same iterations (lanes past the end carry
  // n = 0), so the ballots and the queue length stay uniform across the wave;
  // a wave stops once all its groups lie past the end.
  int it = 0;
  if (SUMM && n_whole > 0) {
    // This thread's summary word sw (written by the previous pass 2 for the
    // same thread of the same chunk) and, once, the decode of its code
    // bound; each iteration then bounds with the lane's largest |g| alone.
    const FastEma d = fast_ema<SMALL ? kRegSmall : kRegGeneral, false>((int)(sw & 0xFFFFu), (int)(kCodeFloat | (sw >> 16)),
                                             0.0f, K.dm, K.ndw, K.nbias, K.iwmin, K.eps, K.b1,
                                             K.omb1, K.b2, K.omb2, K.sign);
    // One iteration on the gradients `cur` of group j: the bound at the
    // thread's code extremes and its largest |g| (the operations of
    // p1_reach); only when it reaches a threshold in some lane are the
    // wave's codes read and decoded.
    auto visit = [&](const Raw8 &cur, int j) {
      const int64_t e0 = beg + ((int64_t)j * nt + sh.tid()) * kVec;
      {
        const float g = raw_gmax<GD, SCALED>(cur, K.inv);
        const float mn = fmaf(K.b1, d.am, K.omb1 * g);
        const float vn = fmaf(K.b2, d.v, K.omb2 * (g * g));
        const uint32_t um = __float_as_uint(mn * K.up_m) & 0x7FFFFFFFu;
        const uint32_t uv = __float_as_uint(fmaf(vn, K.up_v, K.abs_v)) & 0x7FFFFFFFu;
        if (!__ballot(um >= Tm || uv >= Tv)) return;   // no candidate: codes not read
      }
      Group8 G;
      unpack_grads<GD>(cur, G);
      unscale_group<GD, SCALED>(G, K.inv);
      const vu4 a = *(const LUMA_GLOBAL vu4 *)(T.q_m + e0);
      const vu4 b = *(const LUMA_GLOBAL vu4 *)(T.q_w + e0);
      unpack_i16(a.x, G.qm[0], G.qm[1]);
      unpack_i16(a.y, G.qm[2], G.qm[3]);
      unpack_i16(a.z, G.qm[4], G.qm[5]);
      unpack_i16(a.w, G.qm[6], G.qm[7]);
      unpack_u16(b.x, G.qw[0], G.qw[1]);
      unpack_u16(b.y, G.qw[2], G.qw[3]);
      unpack_u16(b.z, G.qw[4], G.qw[5]);
      unpack_u16(b.w, G.qw[6], G.qw[7]);
      uint32_t am[kVec], av[kVec];
      p1_compute<SMALL, true>(G, K, kVec, Tm, Tv, am, av);
      take(e0, kVec, am, av);
    };
    // Three gradient buffers, each loaded two iterations before its use, in
    // a loop unrolled by three: the loop waits on memory, so each wave keeps
    // two groups' loads in flight; no buffer whose load is in flight is
    // copied (the copy would wait for it).  (ra, rb: groups 0 and 1, loaded
    // above.)  The loop runs whole triples only and the last one or two
    // groups follow it: an exit from the middle of the body would reach the
    // loop's latch with the buffers' loads in another order, and the wait
    // for the first buffer, placed for every path into the header, would
    // then also wait for the second.
    seed_thresholds();
    const int n3 = n_whole - n_whole % 3;
    for (; it < n3; it += 3) {
      load_grads<GD>(T, group_at(it + 2), rc);
      visit(ra, it);
      load_grads<GD>(T, group_at(it + 3), ra);
      visit(rb, it + 1);
      load_grads<GD>(T, group_at(it + 4), rb);
      visit(rc, it + 2);
    }
    // ra, rb: groups n3 and n3 + 1 (the last group where that lies past it)
    if (it < n_whole) visit(ra, it);
    if (it + 1 < n_whole) visit(rb, it + 1);
    it = n_whole;
  } else if (n_whole > 0) {
    // raw holds the codes and gradients of the lane's next group (the
    // current one again after the last whole group, so that every iteration
    // issues the same loads); group 0 was loaded above
    Raw8 &raw = ra;
    seed_thresholds();
    for (; it < n_whole; ++it) {
      const int64_t e0 = beg + ((int64_t)it * nt + sh.tid()) * kVec;
      const int64_t en = end - e0 - kStride >= kVec ? e0 + kStride : e0;
      uint32_t am[kVec], av[kVec];
      p1_iter<GD, SMALL, SCALED, true, true>(T, K, e0, kVec, raw, en, Tm, Tv, am, av);
      take(e0, kVec, am, av);
    }
  }
  if (n_whole == 0) seed_thresholds();
  for (; it < n_it; ++it) {
    // a wave whose groups all lie past the end is done (small tensors)
    if (beg + ((int64_t)it * nt + (sh.tid() & ~63u)) * kVec >= end) break;
    const int64_t e0 = beg + ((int64_t)it * nt + sh.tid()) * kVec;
    const int64_t rem = end - e0;
    const int n = rem <= 0 ? 0 : (rem < kVec ? (int)rem : kVec);
    uint32_t am[kVec], av[kVec];
    Raw8 unused;
    p1_iter<GD, SMALL, SCALED, false, false>(T, K, e0, n, unused, e0, Tm, Tv, am, av);
    take(e0, n, am, av);
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  if (lane < qlen) run(queue[lane]);
}

// Pass 1 of the init step (t = 1: no codes to decode).  m' = (1 - beta1) g
// and v' = (1 - beta2) g^2 are each a product (of a product) rounded to
// float32, so both are non-decreasing in |g|: the chunk's maxima are those
// of its largest |g|, and that element is recorded as both maxima's
// position, the seeds of the next step.  Only the gradients are read.
struct InitMax {
  uint32_t gb, gi;   // the lane's largest |g| (float bits, NaN above +Inf) and its offset
};

// The lane's largest |g| of the chunk [beg, end).  Out of line, and given
// the gradient pointer rather than the tensor record, so that the kernel's
// copy of the record stays in registers.
template <int GD>
__device__ __noinline__ InitMax pass1_init_scan(const LUMA_GLOBAL void *grad, int64_t beg,
                                                int64_t end, bool vec_ok, Share sh) {
  const int64_t kStride = (int64_t)sh.nt * kVec;
  Tensor T{};
  T.grad = grad;
  InitMax r{0u, kNoArg};
  auto fold = [&](float g, int64_t i) {
    const uint32_t b = __float_as_uint(g) & 0x7FFFFFFFu;
    if (b > r.gb) {
      r.gb = b;
      r.gi = (uint32_t)(i - beg);
    }
  };
  for (int64_t e0 = beg + (int64_t)sh.tid() * kVec; e0 < end; e0 += kStride) {
    if (vec_ok && end - e0 >= kVec) {
      Raw8 rw;
      load_grads<GD>(T, e0, rw);
      Group8 G;
      unpack_grads<GD>(rw, G);
#pragma unroll
      for (int j = 0; j < kVec; ++j) fold(G.g[j], e0 + j);
    } else {
      for (int j = 0; j < kVec && e0 + j < end; ++j) fold(load_grad(T.grad, e0 + j, GD), e0 + j);
    }
  }
  return r;
}

template <int GD, bool SUMM, int NT>
__device__ __forceinline__ void pass1_dispatch_s(const Tensor &T, const Hyper &h,
                                                 const LUMA_GLOBAL Grid *old, float inv,
                                                 int64_t ci, int64_t beg, int64_t end, bool small,
                                                 bool scaled, float &exm, float &exv,
                                                 uint32_t &im, uint32_t &iv, uint32_t *q, Share sh) {
  if (scaled) {
    if (small)
      pass1_fast_body<GD, true, true, SUMM, NT>(T, h, old, inv, ci, beg, end, exm, exv, im, iv, q, sh);
    else
      pass1_fast_body<GD, false, true, SUMM, NT>(T, h, old, inv, ci, beg, end, exm, exv, im, iv, q, sh);
  } else {
    if (small)
      pass1_fast_body<GD, true, false, SUMM, NT>(T, h, old, inv, ci, beg, end, exm, exv, im, iv, q, sh);
    else
      pass1_fast_body<GD, false, false, SUMM, NT>(T, h, old, inv, ci, beg, end, exm, exv, im, iv, q, sh);
  }
}

// Summaries are kept for workgroup chunks only, so the wavefront form has
// no summary variant.
template <int GD>
__device__ __forceinline__ void pass1_dispatch(const Tensor &T, const Hyper &h,
                                               const LUMA_GLOBAL Grid *old, float inv, int64_t ci,
                                               int64_t beg, int64_t end, bool small, bool scaled,
                                               bool summ, float &exm, float &exv, uint32_t &im,
                                               uint32_t &iv, uint32_t *q, Share sh) {
  if (sh.nt != kThreads)
    pass1_dispatch_s<GD, false, 64>(T, h, old, inv, ci, beg, end, small, scaled, exm, exv, im, iv, q, sh);
  else if (summ)
    pass1_dispatch_s<GD, true, kThreads>(T, h, old, inv, ci, beg, end, small, scaled, exm, exv, im, iv, q, sh);
  else
    pass1_dispatch_s<GD, false, kThreads>(T, h, old, inv, ci, beg, end, small, scaled, exm, exv, im, iv, q, sh);
}

// Whether pass 1 may use chunk ci's code summaries: the previous step's
// pass 2 wrote them with this chunk length (the slot records both), they
// fit in the array, its grid is finite, and the tensor's streams are 16-byte
// aligned (the whole-group loop).
__device__ __forceinline__ bool summaries_valid(const Tensor &T, const LUMA_GLOBAL Grid *old,
                                                int64_t prev, int64_t ci, int32_t shift,
                                                const Share &sh) {
  return sh.nt == kThreads && T.summary != nullptr &&
         (ci + 1) * LUMA_SUMMARY_WORDS <= T.summary_words &&
         old != nullptr && T.slot->summ_step == prev && T.slot->summ_shift == shift &&
         __builtin_isfinite(old->dm) && __builtin_isfinite(old->dw) &&
         __builtin_isfinite(old->fast[kIwmin]) && tensor_vec_ok(T);
}

__global__ __launch_bounds__(kThreads, 4) void pass1_fast_kernel(StepSrc src,
                                                              float *__restrict__ partials) {
  if (skip_step(src)) return;
  {
    // workgroups past the workgroup and medium records: small tensors
    const int32_t own = pass_blocks(src.medium_from, src.small_from);
    if (src.tensors && (int32_t)blockIdx.x >= own) {
      pass1_small_body(src, partials, small_wave((int64_t)blockIdx.x - own));
      return;
    }
  }
  Tensor T;
  LumaGroup grp;
  int64_t ci, rec;
  Share sh;
  if (!chunk_job(src, T, grp, ci, rec, sh)) return;   // (wave mode: no barriers below)
  const Hyper h = group_hyper(grp);
  // this step is t = step + 1; its decode reads the grid of step t - 1
  const int64_t prev = T.slot->step;
  const LUMA_GLOBAL Grid *old = prev >= 1 ? &T.slot->grid[prev & 1] : nullptr;
  int64_t beg, end;
  chunk_range(src, T, ci, beg, end);
  const bool small = old == nullptr || old->fast[kXTopM] <= kSmall;
  const bool scaled = src.scaling.grad_scale != nullptr;
  const float inv = inv_scale(src);
  __shared__ uint32_t qbuf[kThreads / 64][kQueueCap];
  uint32_t *q = qbuf[threadIdx.x >> 6];
  const bool summ = summaries_valid(T, old, prev, ci, src.chunk_shift, sh);
  float exm = 0.0f, exv = 0.0f;
  uint32_t exi_m = kNoArg, exi_v = kNoArg;
  if (old == nullptr) {
    const bool vec_ok = tensor_vec_ok(T);
    const InitMax r =
        T.grad_dtype == LUMA_GRAD_BF16  ? pass1_init_scan<LUMA_GRAD_BF16>(T.grad, beg, end, vec_ok, sh)
        : T.grad_dtype == LUMA_GRAD_F16 ? pass1_init_scan<LUMA_GRAD_F16>(T.grad, beg, end, vec_ok, sh)
                                        : pass1_init_scan<LUMA_GRAD_F32>(T.grad, beg, end, vec_ok, sh);
    // unscaling is monotone in |g|: only the largest is unscaled
    float g = __uint_as_float(r.gb);
    if (scaled) g = unscale_rt(g, inv, T.grad_dtype);
    float mn, vn;
    exact_ema(0.0f, 0.0f, g, h, mn, vn);
    exm = fabsf(mn);
    exv = vn;
    exi_m = exi_v = r.gi;
  } else if (T.grad_dtype == LUMA_GRAD_BF16)
    pass1_dispatch<LUMA_GRAD_BF16>(T, h, old, inv, ci, beg, end, small, scaled, summ, exm, exv,
                                   exi_m, exi_v, q, sh);
  else if (T.grad_dtype == LUMA_GRAD_F16)
    pass1_dispatch<LUMA_GRAD_F16>(T, h, old, inv, ci, beg, end, small, scaled, summ, exm, exv,
                                  exi_m, exi_v, q, sh);
  else
    pass1_dispatch<LUMA_GRAD_F32>(T, h, old, inv, ci, beg, end, small, scaled, summ, exm, exv,
                                  exi_m, exi_v, q, sh);
  put_chunk(partials, rec, sh, exm, exv, exi_m, exi_v);
}

// Inclusive prefix sum over the 64 lanes of a wave (all lanes active): three
// row shifts of the original value, shifts by 4 and 8 within rows, then
// broadcasts of lanes 15 and 31 into the rows above (the GCN DPP scan).
__device__ __forceinline__ uint32_t wave_scan_incl(uint32_t x) {
  const int x0 = (int)x;
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, x0, 0x111, 0xf, 0xf, true);       // row_shr:1
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, x0, 0x112, 0xf, 0xf, true);       // row_shr:2
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, x0, 0x113, 0xf, 0xf, true);       // row_shr:3
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xf, 0xe, true);   // row_shr:4, lanes 4-15
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xf, 0xc, true);   // row_shr:8, lanes 8-15
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xa, 0xf, false);  // row_bcast:15, rows 1, 3
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xc, 0xf, false);  // row_bcast:31, rows 2, 3
  return x;
}

// Per-lane selects by the bits of an index.  v_cndmask_b32 issues at about
// a fifth of the rate of plain VALU on gfx950 (0.21 vs 0.96-1.3 wave
// instructions per clock per CU), so a select is a v_bfi_b32 with an
// all-ones / all-zeros mask: bit b of k sign-extended by v_bfe_i32.  The
// empty asm keeps the compiler from turning the mask back into a compare
// and v_cndmask.
__device__ __forceinline__ uint32_t bit_mask(uint32_t k, int b) {
  uint32_t m = (uint32_t)__builtin_amdgcn_sbfe((int)k, b, 1);
  asm("" : "+v"(m));
  return m;
}

__device__ __forceinline__ uint32_t bfi(uint32_t m, uint32_t a, uint32_t b) {
  return (a & m) | (b & ~m);   // m ? a : b, bitwise
}

// a[k] for a per-lane index k in 0..7 (no indexed register access).
__device__ __forceinline__ uint32_t sel8(const uint32_t (&a)[kVec], uint32_t k) {
  const uint32_t m0 = bit_mask(k, 0), m1 = bit_mask(k, 1), m2 = bit_mask(k, 2);
  const uint32_t x01 = bfi(m0, a[1], a[0]), x23 = bfi(m0, a[3], a[2]);
  const uint32_t x45 = bfi(m0, a[5], a[4]), x67 = bfi(m0, a[7], a[6]);
  return bfi(m2, bfi(m1, x67, x45), bfi(m1, x23, x01));
}

// The packed 32-bit words of a group of 8 elements, two 16-bit values per
// word: word k >> 1 holds element k in its low (k even) or high half.
struct Words4 {
  uint32_t qm[4];   // old momentum codes
  uint32_t qw[4];   // old preconditioner codes
  uint32_t g[4];    // 16-bit gradients after unscaling (bfloat16 only)
};

// a[k >> 1] for a per-lane k in 0..7; m1, m2: bit_mask(k, 1), bit_mask(k, 2).
__device__ __forceinline__ uint32_t word_of(const uint32_t (&a)[4], uint32_t m1, uint32_t m2) {
  return bfi(m2, bfi(m1, a[3], a[2]), bfi(m1, a[1], a[0]));
}

__device__ __forceinline__ uint32_t pack_lo16(uint32_t hi, uint32_t lo) {
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// Certified LogSR decision (see luma_fast.h): with z = y + 1 - c, c the
// middle of the uniform's interval, the code is floor(z); it is certain
// when [z - e, z + e] holds no integer, e bounding |z - z_exact| plus the
// interval's half width.  Given fz = fract(z) and h = 0.5 - e, returns 1
// when not certain: the sign bit of max(h - |fz - 0.5|, -1), so that NaN
// counts as uncertain (fmax drops it) -- computed without compares, whose
// lane-mask results cost more than plain VALU on gfx950.
__device__ __forceinline__ uint32_t unsure(float fz, float h) {
  const float d = fmaxf(h - fabsf(fz - 0.5f), -1.0f);
  return __float_as_uint(d) >> 31;
}

// Adding 1.5 * 2^23 to an integer-valued float k with |k| < 2^22 gives a
// float whose low 16 bits are k's two's complement 16-bit code: one
// dual-issued add instead of a single-issued v_cvt_i32_f32.
constexpr float kCodeBias = 12582912.0f;

// Per-tensor constants of pass 2.
struct P2Const {
  DecodeK D;
  uint32_t pk0, pk1, pm0, pm1;  // Philox key and multipliers
  uint64_t pblk;                // Philox block base of the tensor (element offset >> 3)
  uint32_t prot;                // and its counter word 3 (element offset & 7)
  float ndw;                    // -dw of the old grid (decode)
  float nbias;                  // 2^23 dw: fma(2^23 + q, -dw, nbias) = q * -dw exactly
  float nk1, nk2, hk3, nk7, hk8;   // -k1, -k2, 0.5 - k3, -k7, 0.5 - k8
  float b1, omb1, b2, omb2, decay, neg_eta, eps;
  float isbc2, eps_u;       // 1 / (sqrt(bc2) (-eta)), eps / (-eta)
  float idm;                // momentum: 1/dm
  float cf, ch, cl;         // preconditioner: C = -ln2/dw as float, 16-bit head, tail
  float wmin_n, we, xmin;   // new w_min, w_min * eps, w_min / w_max
  float zoff;               // 1 - half width of a Philox bucket (1 when injected)
  float k1, k2, k3, k7, k8;
  float kmax_m, kmax_w;     // 32767, 65535
  float inv;                // inverse gradient scale (SCALED)
  uint32_t sign;            // 0x80000000
};

// Moves the constants of the loop's dual-issued instructions into VGPRs (see
// in_vgpr).  Those read only by single-issued or half-rate instructions
// (v_med3, v_and_or, v_mad_u64_u32: the clamp bounds, the sign mask, the
// Philox multipliers) and the Philox key, whose ten round keys would hold ten
// VGPR pairs, stay in SGPRs: the VGPRs go to the next iteration's loads.
__device__ __forceinline__ void launder(P2Const &C) {
  C.D.dm = in_vgpr(C.D.dm);
  C.D.dw = in_vgpr(C.D.dw);
  C.D.iwmin = in_vgpr(C.D.iwmin);
  C.D.eps = in_vgpr(C.D.eps);
  C.b1 = in_vgpr(C.b1);
  C.omb1 = in_vgpr(C.omb1);
  C.b2 = in_vgpr(C.b2);
  C.omb2 = in_vgpr(C.omb2);
  C.decay = in_vgpr(C.decay);
  C.neg_eta = in_vgpr(C.neg_eta);
  C.eps = in_vgpr(C.eps);
  C.isbc2 = in_vgpr(C.isbc2);
  C.eps_u = in_vgpr(C.eps_u);
  C.idm = in_vgpr(C.idm);
  C.cf = in_vgpr(C.cf);
  C.ch = in_vgpr(C.ch);
  C.cl = in_vgpr(C.cl);
  C.wmin_n = in_vgpr(C.wmin_n);
  C.we = in_vgpr(C.we);
  C.zoff = in_vgpr(C.zoff);
  C.k1 = in_vgpr(C.k1);
  C.k2 = in_vgpr(C.k2);
  C.k3 = in_vgpr(C.k3);
  C.k7 = in_vgpr(C.k7);
  C.k8 = in_vgpr(C.k8);
  C.ndw = in_vgpr(C.ndw);
  C.nbias = in_vgpr(C.nbias);
  C.nk1 = in_vgpr(C.nk1);
  C.nk2 = in_vgpr(C.nk2);
  C.hk3 = in_vgpr(C.hk3);
  C.nk7 = in_vgpr(C.nk7);
  C.hk8 = in_vgpr(C.hk8);
  C.inv = in_vgpr(C.inv);
}

// One iteration of 8 consecutive elements.  FULL: all 8 valid and 16-byte
// aligned (vector loads/stores, no masking).  Returns which codes need the
// exact path (bit j: momentum code of element j, bit 8 + j: preconditioner
// code); Q, W and top_w (block T_w) are kept for the queues.
// STAGE (FULL only): the preconditioner codes go to *stage (LDS) instead
// of HBM.

// Running extremes of the codes one thread stores in its share of a chunk:
// packed 16-bit signed max and min of the momentum codes and unsigned min of
// the preconditioner codes, two codes per word and per instruction, from the
// 16-byte store vectors.
struct CodeAcc {
  uint32_t mx, mn, wn;
};

__device__ __forceinline__ uint32_t max_i16x2(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(s16x2, a),
                                                                __builtin_bit_cast(s16x2, b)));
}

__device__ __forceinline__ uint32_t min_i16x2(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(s16x2, a),
                                                                __builtin_bit_cast(s16x2, b)));
}

__device__ __forceinline__ uint32_t min_u16x2(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(u16x2, a),
                                                                __builtin_bit_cast(u16x2, b)));
}

// (The words are copied into scalars first: this compiler's
// __builtin_bit_cast of a vector element such as a.y reads the vector's
// first word instead.)
__device__ __forceinline__ void acc_codes(CodeAcc &acc, vu4 a, vu4 b) {
  const uint32_t ax = a.x, ay = a.y, az = a.z, aw = a.w;
  const uint32_t bx = b.x, by = b.y, bz = b.z, bw = b.w;
  acc.mx = max_i16x2(acc.mx, max_i16x2(max_i16x2(ax, ay), max_i16x2(az, aw)));
  acc.mn = min_i16x2(acc.mn, min_i16x2(min_i16x2(ax, ay), min_i16x2(az, aw)));
  acc.wn = min_u16x2(acc.wn, min_u16x2(min_u16x2(bx, by), min_u16x2(bz, bw)));
}

// acc: folds in the codes the fast path stores for the lane's valid
// elements (the code summaries widen them by the decision margin).
// The 16-byte vectors one whole group reads: old codes, gradients (g1:
// float32 only) and parameters.
struct P2Raw {
  Raw8 r;
  vf4 p0, p1;
};

// float32 gradients (two vectors) are loaded by the iteration itself, not a
// whole iteration ahead: two buffers of them would take the kernel past the
// 168 VGPRs that keep three waves per SIMD.
template <int GD>
__device__ __forceinline__ void load_p2_grads(const Tensor &T, int64_t e0, Raw8 &r) {
  if (GD == LUMA_GRAD_F32) {
    r.g0 = load_stream((const LUMA_GLOBAL vu4 *)((const LUMA_GLOBAL float *)T.grad + e0));
    r.g1 = load_stream((const LUMA_GLOBAL vu4 *)((const LUMA_GLOBAL float *)T.grad + e0 + 4));
  } else {
    r.g0 = load_stream((const LUMA_GLOBAL vu4 *)((const LUMA_GLOBAL uint16_t *)T.grad + e0));
  }
}

template <int GD>
__device__ __forceinline__ void load_p2raw(const Tensor &T, int64_t e0, P2Raw &R) {
  R.r.qm = *(const LUMA_GLOBAL vu4 *)(T.q_m + e0);
  R.r.qw = load_stream((const LUMA_GLOBAL vu4 *)(T.q_w + e0));
  if (GD != LUMA_GRAD_F32) load_p2_grads<GD>(T, e0, R.r);
  R.p0 = load_stream((const LUMA_GLOBAL vf4 *)(T.param + e0));
  R.p1 = load_stream((const LUMA_GLOBAL vf4 *)(T.param + e0 + 4));
}

// W: the words of the old codes and (bfloat16) gradients, for the queues.
// FULL: the group's vectors are in RW (load_p2raw); otherwise it loads its
// n valid elements itself.
template <int GD, bool INJ, int REG, bool SCALED, bool FULL, bool STAGE>
__device__ __forceinline__ uint32_t p2_iter(const Tensor &T, const P2Const &C, int64_t e0, int n,
                                            const P2Raw &RW, uint32_t k0, uint32_t k1, Group8 &Q,
                                            Words4 &W, U4 &top_w, uint4 *stage, CodeAcc &acc) {
  if (FULL) {
    Raw8 R = RW.r;
    if (GD == LUMA_GRAD_F32) load_p2_grads<GD>(T, e0, R);
    unpack_raw<GD>(R, Q);
    W.qm[0] = R.qm.x; W.qm[1] = R.qm.y; W.qm[2] = R.qm.z; W.qm[3] = R.qm.w;
    W.qw[0] = R.qw.x; W.qw[1] = R.qw.y; W.qw[2] = R.qw.z; W.qw[3] = R.qw.w;
    W.g[0] = R.g0.x; W.g[1] = R.g0.y; W.g[2] = R.g0.z; W.g[3] = R.g0.w;
  } else {
    load_group<GD, true>(T, e0, n, false, Q);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      W.qm[i] = pack_lo16((uint32_t)Q.qm[2 * i + 1], (uint32_t)Q.qm[2 * i]);
      W.qw[i] = pack_lo16((uint32_t)Q.qw[2 * i + 1], (uint32_t)Q.qw[2 * i]);
    }
  }
  unscale_group<GD, SCALED>(Q, C.inv);
  // bfloat16 words of the unscaled gradients: the loaded words unless scaled
  // (an unscaled bfloat16 gradient is a float32 with its low half zero)
  if (GD == LUMA_GRAD_BF16 && (SCALED || !FULL)) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      W.g[i] = __builtin_amdgcn_perm(__float_as_uint(Q.g[2 * i + 1]), __float_as_uint(Q.g[2 * i]),
                                     0x07060302u);
  }
  float p[kVec];
  if (FULL) {
    p[0] = RW.p0.x; p[1] = RW.p0.y; p[2] = RW.p0.z; p[3] = RW.p0.w;
    p[4] = RW.p1.x; p[5] = RW.p1.y; p[6] = RW.p1.z; p[7] = RW.p1.w;
  } else {
#pragma unroll
    for (int j = 0; j < kVec; ++j) p[j] = j < n ? T.param[e0 + j] : 0.0f;
  }
  // offsets zoff - (lower end of the uniform's interval): z = y + offset
  float zmu_m[kVec], zmu_w[kVec];
  if (INJ) {
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      zmu_m[j] = C.zoff - ((FULL || j < n) ? T.u_m[e0 + j] : 0.5f);
      zmu_w[j] = C.zoff - ((FULL || j < n) ? T.u_w[e0 + j] : 0.5f);
    }
  } else {
    // the top 16 bits of both uniforms of elements e0 .. e0+7, one block at a
    // time; T_w is kept for the queue entries (T_m is recomputed by the rare
    // iteration that queues a momentum code)
    const uint64_t b = C.pblk + ((uint64_t)e0 >> 3);
    const U4 tm = philox4x32_10_v((uint32_t)b, (uint32_t)(b >> 32), kBlockTopM, C.prot, C.pk0,
                                  C.pk1, C.pm0, C.pm1);
#pragma unroll
    for (int j = 0; j < kVec; ++j) zmu_m[j] = fmaf((float)u4_half(tm, j), -1.0f / 65536.0f, C.zoff);
    __builtin_amdgcn_sched_barrier(0);
    top_w = philox4x32_10_v((uint32_t)b, (uint32_t)(b >> 32), kBlockTopW, C.prot, C.pk0, C.pk1,
                            C.pm0, C.pm1);
#pragma unroll
    for (int j = 0; j < kVec; ++j) zmu_w[j] = fmaf((float)u4_half(top_w, j), -1.0f / 65536.0f, C.zoff);
  }
  uint32_t om[kVec], ow[kVec];   // codes in the low 16 bits (kCodeBias)
  uint32_t flags = 0;
#pragma unroll
  for (int j = 0; j < kVec; ++j) {
    const FastEma f = fast_ema<REG, true>(Q.qm[j], Q.qw[j], Q.g[j], C.D.dm, C.ndw, C.nbias, C.D.iwmin,
                                            C.D.eps, C.b1, C.omb1, C.b2, C.omb2, C.sign);
    const float s = __builtin_amdgcn_sqrtf(f.vn);
    // AdamW update (functional.py:278-279), within 1e-6 of the exact path:
    // p*decay + m' / ((sqrt(v')/sqrt(bc2) + eps) / (-eta))
    const float den = fmaf(s, C.isbc2, C.eps_u);
    p[j] = fmaf(p[j], C.decay, f.mn * __builtin_amdgcn_rcpf(den));
    // momentum code: z = log1p(|m'|)/dm + offset.  |m'| <= S_m' exactly, so
    // the exact path's clamp is inactive; the code's sign is m''s.
    const float am = in_vgpr(fabsf(f.mn));   // one v_and, not an |.| modifier per fma
    const float L = fast_log1p<REG>(am);
    const float zm = fmaf(L, C.idm, zmu_m[j]);
    const float hm = fmaf(f.am, C.nk1, fmaf(zm, C.nk2, C.hk3));    // 0.5 - e
    // floor(z) as z - fract(z) (exact for |z| < 2^23; v_fract is needed for
    // the certification anyway, and the subtraction dual-issues where
    // v_floor does not)
    const float fzm = __builtin_amdgcn_fractf(zm);
    const float cm = __uint_as_float(
        __float_as_uint(__builtin_amdgcn_fmed3f(zm - fzm, 0.0f, C.kmax_m)) |
        (__float_as_uint(f.mn) & C.sign));
    om[j] = __float_as_uint(cm + kCodeBias);   // low 16 bits: the signed code
    // preconditioner code: x = w_min t, clamped to the exact path's w range;
    // y = -log2(x) ln2/dw = (e + log2 mant) C, with e C exact (16-bit C_hi)
    // so that only O(|C|) terms round.  delta_w = 0 gives C = 0: code 0.
    const float x = __builtin_amdgcn_fmed3f(fmaf(s, C.wmin_n, C.we), C.xmin, 1.0f);
    const float ef = (float)__builtin_amdgcn_frexp_expf(x);
    const float l2 = __builtin_amdgcn_logf(__builtin_amdgcn_frexp_mantf(x));
    const float A = ef * C.ch;
    const float fA = __builtin_amdgcn_fractf(A);
    const float zw = fmaf(l2, C.cf, fmaf(ef, C.cl, fA + zmu_w[j]));
    const float hw = fmaf(A, C.nk7, C.hk8);                        // 0.5 - e
    const float fzw = __builtin_amdgcn_fractf(zw);
    ow[j] = __float_as_uint(
        __builtin_amdgcn_fmed3f((A - fA) + (zw - fzw), 0.0f, C.kmax_w) + kCodeBias);
    // uncertain when 0.5 - e - |fract(z) - 0.5| < 0 or NaN: its sign bit
    const uint32_t um = unsure(fzm, hm), uw = unsure(fzw, hw);
    if (FULL || j < n) flags |= (um << j) | (uw << (8 + j));
  }
  if (FULL) {
    vf4 p0, p1;
    p0.x = p[0]; p0.y = p[1]; p0.z = p[2]; p0.w = p[3];
    p1.x = p[4]; p1.y = p[5]; p1.z = p[6]; p1.w = p[7];
    store_stream(p0, (LUMA_GLOBAL vf4 *)(T.param + e0));
    store_stream(p1, (LUMA_GLOBAL vf4 *)(T.param + e0 + 4));
    // two codes per word: the low halves of om[2i] and om[2i + 1] (v_perm)
    vu4 a, b;
    a.x = __builtin_amdgcn_perm(om[1], om[0], 0x05040100u);
    a.y = __builtin_amdgcn_perm(om[3], om[2], 0x05040100u);
    a.z = __builtin_amdgcn_perm(om[5], om[4], 0x05040100u);
    a.w = __builtin_amdgcn_perm(om[7], om[6], 0x05040100u);
    b.x = __builtin_amdgcn_perm(ow[1], ow[0], 0x05040100u);
    b.y = __builtin_amdgcn_perm(ow[3], ow[2], 0x05040100u);
    b.z = __builtin_amdgcn_perm(ow[5], ow[4], 0x05040100u);
    b.w = __builtin_amdgcn_perm(ow[7], ow[6], 0x05040100u);
    *(LUMA_GLOBAL vu4 *)(T.q_m + e0) = a;
    if (STAGE)
      *stage = make_uint4(b.x, b.y, b.z, b.w);
    else
      *(LUMA_GLOBAL vu4 *)(T.q_w + e0) = b;
    acc_codes(acc, a, b);
  } else {
    int qa = 0;
    uint32_t qw = 65535u;
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      if (j < n) {
        T.param[e0 + j] = p[j];
        T.q_m[e0 + j] = (int16_t)(uint16_t)om[j];
        T.q_w[e0 + j] = (int16_t)(uint16_t)ow[j];
        qa = max(qa, abs((int)(int16_t)(uint16_t)om[j]));
        qw = min(qw, ow[j] & 0xFFFFu);
      }
    }
    acc.mx = max_i16x2(acc.mx, (uint32_t)qa * 0x10001u);
    acc.wn = min_u16x2(acc.wn, qw * 0x10001u);
  }
  return flags;
}

template <int GD, bool INJ, int REG, bool SCALED, int KTAG>
__device__ void pass2_fast_body(const Tensor &T, const Hyper &h, const LUMA_GLOBAL Grid *old,
                                const LUMA_GLOBAL Grid *nw, float inv, int64_t ci, int64_t beg,
                                int64_t end, uint32_t k0, uint32_t k1, uint4 *queue,
                                Share sh) {
  // Threads per chunk: kThreads, or one wavefront for a medium tensor; an
  // iteration covers nt * kVec = 1 << it_shift consecutive elements.
  const int nt = sh.nt;
  const int it_shift = __builtin_ctz((unsigned)nt) + 3;
  const bool vec_ok = tensor_vec_ok(T);
  // Iterations in which every lane's group is whole stage their
  // preconditioner codes; before a slot is reused, the iteration it holds has
  // its queued entries run and is written back.
  const int n_whole = vec_ok ? (int)((end - beg) >> it_shift) : 0;
  // Each iteration's vectors are loaded one iteration ahead, into two
  // buffers in a loop unrolled by two (copying a buffer whose loads are in
  // flight would make the copy wait for them); past the last whole group the
  // loads repeat the last group, and are not used.
  auto group_at = [&](int j) {
    return beg + ((int64_t)(j < n_whole ? j : n_whole - 1) * nt + sh.tid()) * kVec;
  };
  // The first group's loads go out before the per-tensor constants below
  // are derived, so that their latency covers that arithmetic.
  P2Raw ra, rb;
  if (n_whole > 0) load_p2raw<GD>(T, group_at(0), ra);
  const Bounds B = make_bounds((const Grid *)old, (const Grid *)nw, h.beta1, h.beta2);
  P2Const C;
  C.D = decode_consts(old, h.eps);
  C.b1 = h.beta1; C.omb1 = h.omb1; C.b2 = h.beta2; C.omb2 = h.omb2;
  C.decay = h.decay; C.neg_eta = h.neg_eta; C.eps = h.eps;
  // the update's denominator divided by -eta (lr = 0: an infinite
  // denominator, so the update term is exactly 0)
  {
    const double ne = (double)h.neg_eta;
    const double isb = 1.0 / ::sqrt((double)h.bc2);
    C.isbc2 = ne != 0.0 ? (float)(isb / ne) : 0.0f;
    C.eps_u = ne != 0.0 ? (float)((double)h.eps / ne) : INFINITY;
  }
  // z = y + zoff - u_low has floor(z) = the LogSR code when u is known to
  // lie in [u_low, u_low + 2 hb): zoff = 1 - hb (Philox: buckets of 2^-16,
  // the uniform's top 16 bits).
  const float hb = INJ ? 0.0f : 0x1p-17f;
  C.zoff = 1.0f - hb;
  C.idm = nw->fast[kIdm];
  C.cf = nw->fast[kNl2dw];
  C.ch = nw->fast[kCwHi];
  C.cl = nw->fast[kCwLo];
  C.wmin_n = nw->wmin;
  C.we = nw->fast[kWe];
  C.xmin = nw->fast[kXMin];
  C.k1 = B.k1;
  C.k2 = B.k2;
  C.k3 = B.k3 + hb;
  C.k7 = B.k7;
  C.k8 = B.k8 + hb;
  C.kmax_m = 32767.0f;
  C.kmax_w = 65535.0f;
  C.inv = inv;
  C.sign = 0x80000000u;
  C.pk0 = k0;
  C.pk1 = k1;
  C.pm0 = kPhiloxM0;
  C.pm1 = kPhiloxM1;
  const PhiloxBase pb = philox_base(T.elem_offset);
  C.pblk = pb.blk;
  C.prot = pb.rot;
  C.ndw = -C.D.dw;
  C.nbias = 8388608.0f * C.D.dw;
  C.nk1 = -C.k1;
  C.nk2 = -C.k2;
  C.hk3 = 0.5f - C.k3;
  C.nk7 = -C.k7;
  C.hk8 = 0.5f - C.k8;
  // Code summaries: a fast code differs from the exact one by at most
  // ceil(e), e the decision bound (momentum: |m| k1 + z k2 + k3 with
  // |m| <= 1.01 S_m(old), z <= 32769; preconditioner: |A| k7 + k8 with
  // |A| <= 150 |C_hi|), and by at most 1 when e < 1.  A non-finite bound
  // gives the widest margin (the summary then bounds nothing).
  const float em = (old ? old->sm * 1.01f : 0.0f) * B.k1 + 32769.0f * B.k2 + C.k3;
  const float ew = 150.0f * fabsf(C.ch) * B.k7 + C.k8;
  const uint32_t marg_m = em < 32767.0f ? (uint32_t)fmaxf(1.0f, ceilf(em)) : 32767u;
  const uint32_t marg_w = ew < 65535.0f ? (uint32_t)fmaxf(1.0f, ceilf(ew)) : 65535u;
  launder(C);
  const uint32_t lane = lane_id();
  // the wave's LDS block: momentum ring, preconditioner ring, staging slots
  uint4 *queue_m = queue, *queue_w = queue + kQueueCapM;
  uint4 *stage = queue_w + kQueueCapW;
  uint32_t qlen_m = 0, qlen_w = 0;   // pending entries
  uint32_t head_m = 0, head_w = 0;   // ring position of the oldest
  // Queue entry of element k of a group: x = chunk offset (k = x & 7),
  // y = the word of T_m (momentum) or T_w (preconditioner) holding the top
  // 16 bits of the element's uniform (its low 8 bits come from block L),
  // z = the gradient (bfloat16: the
  // word of two unscaled gradients holding it; otherwise its float32 bits;
  // no second read of HBM), w = the word of two old codes holding its code.
  // The entry keeps whole words so that building it costs two selects per
  // field; the drain, 64 entries at a time, takes the element's half.  The
  // fast codes were already stored (or staged); the exact ones overwrite
  // them (same wavefront, so the stores stay in program order).
  // The code of a queued element from its pair: lo = hi when the uniform's
  // interval decided it; else (Philox) block L gives u's low 8 bits.
  const float zm_new = nw->zm, zw_new = nw->zw;
  auto draw = [&](const CodePair &c, float z, int64_t i, uint32_t top, int which) -> int {
    if (c.lo == c.hi) return c.lo;
    const U4 low = philox_block((uint64_t)i, pb, kBlockLow, k0, k1);
    const float u = (float)((top << 8) | u4_byte(low, 2 * (int)(i & 7) + which)) * 0x1p-24f;
    return sr_below<KTAG>(c.a, z, u) ? c.hi : c.lo;
  };
  // The interval of an entry's uniform: the injected u itself, or (Philox)
  // the interval of its top 16 bits.
  auto u_lo = [&](uint32_t top, const LUMA_GLOBAL float *u, int64_t i) -> float {
    return INJ ? u[i] : (float)(top << 8) * 0x1p-24f;
  };
  auto u_hi = [&](uint32_t top, const LUMA_GLOBAL float *u, int64_t i) -> float {
    return INJ ? u[i] : (float)((top << 8) | 0xFFu) * 0x1p-24f;
  };
  // Staging: whole-group iterations [staged_lo, staged_hi) keep their
  // preconditioner codes in stage[(it % kStage) * 64 + lane] until written
  // back.  Chunk offset o belongs to iteration o >> it_shift and to lane
  // (o >> 3) & 63 of this wave.
  int staged_lo = 0, staged_hi = 0;
  // an entry's element: its half of the words (sh = 16 for odd k)
  auto ent_grad = [&](const uint4 &ent, uint32_t sh) -> float {
    return GD == LUMA_GRAD_BF16 ? __uint_as_float((ent.z >> sh) << 16) : __uint_as_float(ent.z);
  };
  auto run_m = [&](uint4 ent) {
    const int64_t i = beg + ent.x;
    const uint32_t sh = (ent.x & 1u) << 4;
    const uint32_t top = INJ ? 0u : (ent.y >> sh) & 0xFFFFu;
    const CodePair c = unpack_pair(exact_pair_m<KTAG>((int)(int16_t)(ent.w >> sh), ent_grad(ent, sh),
                                                old, nw, h, u_lo(top, T.u_m, i),
                                                u_hi(top, T.u_m, i)));
    T.q_m[i] = (int16_t)draw(c, zm_new, i, top, 0);
  };
  auto run_w = [&](uint4 ent) {
    const uint32_t o = ent.x;
    const int64_t i = beg + o;
    const uint32_t sh = (o & 1u) << 4;
    const uint32_t top = INJ ? 0u : (ent.y >> sh) & 0xFFFFu;
    const CodePair c = unpack_pair(exact_pair_w<KTAG>((int)((ent.w >> sh) & 0xFFFFu), ent_grad(ent, sh),
                                                old, nw, h, u_lo(top, T.u_w, i),
                                                u_hi(top, T.u_w, i)));
    const uint16_t code = (uint16_t)draw(c, zw_new, i, top, 1);
    const int it_e = (int)(o >> it_shift);
    if (it_e >= staged_lo && it_e < staged_hi) {
      uint16_t *slot = (uint16_t *)&stage[(it_e % kStage) * 64 + ((o >> 3) & 63u)];
      slot[o & 7u] = code;
    } else {
      T.q_w[i] = (int16_t)code;
    }
  };
  // Queue the codes of one iteration that the fast path could not certify,
  // and run full batches of 64, oldest first.
  auto take = [&](int64_t e0, uint32_t flags, const Group8 &Q, const Words4 &W,
                  const U4 &top_w) {
    if (!__ballot(flags != 0)) return;
    const uint32_t off0 = (uint32_t)(e0 - beg);
    // queue positions: a wave prefix sum of (momentum count | preconditioner
    // count << 16) gives each lane its first slot in both queues
    const uint32_t fm = flags & 0xFFu, fw = flags >> 8;
    const uint32_t cnt = (uint32_t)__builtin_popcount(fm) | ((uint32_t)__builtin_popcount(fw) << 16);
    const uint32_t incl = wave_scan_incl(cnt);
    const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
    const uint32_t excl = incl - cnt;
    const uint32_t tot_m = tot & 0xFFFFu, tot_w = tot >> 16;
    // queue entry of element off0 + k: the top 16 bits of its uniform are
    // half k of T_m (momentum) or T_w (preconditioner), in word k/2
    const uint32_t cw[4] = {top_w.x, top_w.y, top_w.z, top_w.w};
    uint32_t cm[4] = {0u, 0u, 0u, 0u};
    if (!INJ && __ballot(fm != 0u)) {
      const uint64_t b = C.pblk + ((uint64_t)e0 >> 3);
      const U4 tm = philox4x32_10_v((uint32_t)b, (uint32_t)(b >> 32), kBlockTopM, C.prot, C.pk0,
                                    C.pk1, C.pm0, C.pm1);
      cm[0] = tm.x; cm[1] = tm.y; cm[2] = tm.z; cm[3] = tm.w;
    }
    auto entry = [&](uint32_t k, const uint32_t (&codes)[4], const uint32_t (&tops)[4]) {
      const uint32_t m1 = bit_mask(k, 1), m2 = bit_mask(k, 2);
      uint32_t g;
      if (GD == LUMA_GRAD_BF16) {
        g = word_of(W.g, m1, m2);
      } else {
        uint32_t gb[kVec];
#pragma unroll
        for (int j = 0; j < kVec; ++j) gb[j] = __float_as_uint(Q.g[j]);
        g = sel8(gb, k);
      }
      return make_uint4(off0 + k, INJ ? 0u : word_of(tops, m1, m2), g, word_of(codes, m1, m2));
    };
    if (qlen_m + tot_m <= (uint32_t)kQueueCapM) {
      uint32_t pos = head_m + qlen_m + (excl & 0xFFFFu);
      for (uint32_t f = fm; f != 0u; f &= f - 1u) {
        const uint32_t k = (uint32_t)__builtin_ctz(f);
        queue_m[pos++ & (kQueueCapM - 1)] = entry(k, W.qm, cm);
      }
      qlen_m += tot_m;
    } else {
      // more than the queue holds (only when most codes are uncertain): in place
      for (uint32_t f = fm; f != 0u; f &= f - 1u) {
        const uint32_t k = (uint32_t)__builtin_ctz(f);
        run_m(entry(k, W.qm, cm));
      }
    }
    if (qlen_w + tot_w <= (uint32_t)kQueueCapW) {
      uint32_t pos = head_w + qlen_w + (excl >> 16);
      for (uint32_t f = fw; f != 0u; f &= f - 1u) {
        const uint32_t k = (uint32_t)__builtin_ctz(f);
        queue_w[pos++ & (kQueueCapW - 1)] = entry(k, W.qw, cw);
      }
      qlen_w += tot_w;
    } else {
      for (uint32_t f = fw; f != 0u; f &= f - 1u) {
        const uint32_t k = (uint32_t)__builtin_ctz(f);
        run_w(entry(k, W.qw, cw));
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    while (qlen_m >= 64) {
      run_m(queue_m[(head_m + lane) & (kQueueCapM - 1)]);
      head_m += 64;
      qlen_m -= 64;
    }
    while (qlen_w >= 64) {
      run_w(queue_w[(head_w + lane) & (kQueueCapW - 1)]);
      head_w += 64;
      qlen_w -= 64;
    }
  };
  // Run the oldest min(qlen_w, 64) preconditioner entries (a partial batch).
  auto batch_w = [&]() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const uint32_t nb = qlen_w < 64u ? qlen_w : 64u;
    if (lane < nb) run_w(queue_w[(head_w + lane) & (kQueueCapW - 1)]);
    head_w += nb;
    qlen_w -= nb;
  };
  // Oldest pending preconditioner entry's iteration (the ring is FIFO).
  auto oldest_w = [&]() -> int {
    const uint32_t x = queue_w[head_w & (kQueueCapW - 1)].x;
    return (int)((uint32_t)__builtin_amdgcn_readfirstlane((int)x) >> it_shift);
  };
  // Write iteration j's staged preconditioner codes to HBM.
  auto write_back = [&](int j) {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const uint4 v = stage[(j % kStage) * 64 + lane];
    const int64_t e = beg + ((int64_t)j * nt + sh.tid()) * kVec;
    vu4 w;
    w.x = v.x; w.y = v.y; w.z = v.z; w.w = v.w;
    store_stream(w, (LUMA_GLOBAL vu4 *)(T.q_w + e));
  };
  // Every lane of a wave runs the same iterations (lanes past the end carry
  // n = 0), so the ballots and the queue lengths stay uniform across the wave;
  // a wave stops once all its groups lie past the end.
  const int64_t kStride = (int64_t)1 << it_shift;
  const int n_it = (int)((end - beg + kStride - 1) >> it_shift);
  CodeAcc acc{0u, 0u, 0xFFFFFFFFu};
  auto whole_iter = [&](const P2Raw &R, int j) {
    const int64_t e0 = group_at(j);
    Group8 Q;
    Words4 W;
    U4 top_w{};
    const uint32_t flags = p2_iter<GD, INJ, REG, SCALED, true, true>(
        T, C, e0, kVec, R, k0, k1, Q, W, top_w, &stage[(j % kStage) * 64 + lane], acc);
    staged_hi = j + 1;
    take(e0, flags, Q, W, top_w);
    const int wb = j + 1 - kStage;   // the slot iteration j + 1 will use
    if (wb >= 0) {
      while (qlen_w > 0 && oldest_w() <= wb) batch_w();
      write_back(wb);
      staged_lo = wb + 1;
    }
  };
  int it = 0;
  if (n_whole > 0) {
    // Whole pairs only: an exit from the middle of the body would reach the
    // loop's latch too, and the waits placed for every path into the header
    // would then wait for more than the current buffer.  An odd last whole
    // group is stepped by the loop below (its own loads, no staging).
    // (the scheduling barriers keep each half's loads ahead of its first use
    // of the buffer loaded one half earlier: moved above them, that use
    // waits first and the loads go out late)
    const int n2 = n_whole & ~1;
    for (; it < n2; it += 2) {
      load_p2raw<GD>(T, group_at(it + 1), rb);
      __builtin_amdgcn_sched_barrier(0);
      whole_iter(ra, it);
      load_p2raw<GD>(T, group_at(it + 2), ra);
      __builtin_amdgcn_sched_barrier(0);
      whole_iter(rb, it + 1);
    }
  }
  // drain the staged iterations
  while (qlen_w > 0) batch_w();
  for (int j = staged_lo; j < staged_hi; ++j) write_back(j);
  staged_lo = staged_hi = 0;
  for (; it < n_it; ++it) {
    // a wave whose groups all lie past the end is done (small tensors)
    if (beg + ((int64_t)it * nt + (sh.tid() & ~63u)) * kVec >= end) break;
    const int64_t e0 = beg + ((int64_t)it * nt + sh.tid()) * kVec;
    const int64_t rem = end - e0;
    const int n = rem <= 0 ? 0 : (rem < kVec ? (int)rem : kVec);
    Group8 Q;
    Words4 W;
    U4 top_w{};
    P2Raw R;
    const bool whole = vec_ok && n == kVec;
    if (whole) load_p2raw<GD>(T, e0, R);
    const uint32_t flags =
        whole ? p2_iter<GD, INJ, REG, SCALED, true, false>(T, C, e0, n, R, k0, k1, Q, W, top_w,
                                                             nullptr, acc)
              : p2_iter<GD, INJ, REG, SCALED, false, false>(T, C, e0, n, R, k0, k1, Q, W,
                                                              top_w, nullptr, acc);
    take(e0, flags, Q, W, top_w);
  }
  // The thread's summary word: its largest |Q_m| + margin, its smallest
  // Q_w - margin (clamped to the code ranges).
  // (one word per thread of a kThreads workgroup: the wavefront route writes none)
  if (nt == kThreads && T.summary != nullptr && (ci + 1) * LUMA_SUMMARY_WORDS <= T.summary_words) {
    const int mx = max((int)(int16_t)(acc.mx & 0xFFFFu), (int)(int16_t)(acc.mx >> 16));
    const int mn = min((int)(int16_t)(acc.mn & 0xFFFFu), (int)(int16_t)(acc.mn >> 16));
    const uint32_t qa = (uint32_t)max(mx, -mn), qw = min(acc.wn & 0xFFFFu, acc.wn >> 16);
    const uint32_t a = min(qa + marg_m, 32767u), w = qw > marg_w ? qw - marg_w : 0u;
    T.summary[ci * LUMA_SUMMARY_WORDS + sh.tid()] = a | (w << 16);
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  if (lane < qlen_m) run_m(queue_m[(head_m + lane) & (kQueueCapM - 1)]);
  if (lane < qlen_w) run_w(queue_w[(head_w + lane) & (kQueueCapW - 1)]);
}

template <int GD, bool SCALED, bool INJ_OK, bool INJ>
__device__ __forceinline__ void pass2_dispatch_r(const Tensor &T, const Hyper &h,
                                                 const LUMA_GLOBAL Grid *old,
                                                 const LUMA_GLOBAL Grid *nw, float inv, int64_t ci,
                                                 int64_t beg, int64_t end, uint32_t k0,
                                                 uint32_t k1, int reg, uint4 *q, Share sh) {
  if (reg == kRegSmall)
    pass2_fast_body<GD, INJ, kRegSmall, SCALED, INJ_OK>(T, h, old, nw, inv, ci, beg, end, k0, k1, q, sh);
  else if (reg == kRegMedium)
    pass2_fast_body<GD, INJ, kRegMedium, SCALED, INJ_OK>(T, h, old, nw, inv, ci, beg, end, k0, k1, q, sh);
  else
    pass2_fast_body<GD, INJ, kRegGeneral, SCALED, INJ_OK>(T, h, old, nw, inv, ci, beg, end, k0, k1,
                                                          q, sh);
}

template <int GD, bool SCALED, bool INJ_OK>
__device__ __forceinline__ void pass2_dispatch_s(const Tensor &T, const Hyper &h,
                                                 const LUMA_GLOBAL Grid *old,
                                                 const LUMA_GLOBAL Grid *nw, float inv, int64_t ci,
                                                 int64_t beg, int64_t end, uint32_t k0,
                                                 uint32_t k1, bool inj, int reg, uint4 *q,
                                                 Share sh) {
  if (INJ_OK && inj)
    pass2_dispatch_r<GD, SCALED, INJ_OK, true>(T, h, old, nw, inv, ci, beg, end, k0, k1, reg, q, sh);
  else
    pass2_dispatch_r<GD, SCALED, INJ_OK, false>(T, h, old, nw, inv, ci, beg, end, k0, k1, reg, q, sh);
}

template <int GD, bool INJ_OK>
__device__ __forceinline__ void pass2_dispatch(const Tensor &T, const Hyper &h,
                                               const LUMA_GLOBAL Grid *old,
                                               const LUMA_GLOBAL Grid *nw, float inv, bool scaled,
                                               int64_t ci, int64_t beg, int64_t end, uint32_t k0,
                                               uint32_t k1, bool inj, int reg, uint4 *q, Share sh) {
  if (scaled)
    pass2_dispatch_s<GD, true, INJ_OK>(T, h, old, nw, inv, ci, beg, end, k0, k1, inj, reg, q, sh);
  else
    pass2_dispatch_s<GD, false, INJ_OK>(T, h, old, nw, inv, ci, beg, end, k0, k1, inj, reg, q, sh);
}

// INJ_OK: a launch with injected uniforms.  Philox launches use the kernel
// without the injected-uniform paths: compiled together with them, the
// kernel's register allocation (the largest over every path it holds) goes
// from 167 VGPRs to 248 and spills, which would halve the occupancy of the
// Philox paths.
template <bool INJ_OK>
__global__ __launch_bounds__(kThreads) void pass2_fast_kernel(StepSrc src, uint64_t base_seed,
                                                              int noise_mode) {
  if (skip_step(src)) return;
  Tensor T;
  LumaGroup grp;
  int64_t ci, rec;
  Share sh;
  // (the small tensors too: one wavefront each, after the medium ones)
  if (!chunk_job(src, T, grp, ci, rec, sh, true)) return;   // (no barriers below)
  const LUMA_GLOBAL Slot *S = T.slot;
  const int64_t t = S->step;   // advanced by finalize
  const Hyper h = S->hyp;
  const LUMA_GLOBAL Grid *old = t >= 2 ? &S->grid[(t - 1) & 1] : nullptr;
  const LUMA_GLOBAL Grid *nw = &S->grid[t & 1];
  int64_t beg, end;
  chunk_range(src, T, ci, beg, end);
  uint32_t k0, k1;
  step_key(base_seed, t, T.param_id, k0, k1);
  const bool inj = injected(T, noise_mode);
  // momentum regime (see luma_fast.h): old grid's decode range, new scale
  const float x_top = old == nullptr ? 0.0f : old->fast[kXTopM];
  const int reg = momentum_regime(x_top, nw->sm);
  const bool scaled = src.scaling.grad_scale != nullptr;
  const float inv = inv_scale(src);
  // each wavefront's queues and staging ring
  __shared__ uint4 qbuf[kThreads / 64][kWaveLds];
  uint4 *q = qbuf[threadIdx.x >> 6];
  if (T.grad_dtype == LUMA_GRAD_BF16)
    pass2_dispatch<LUMA_GRAD_BF16, INJ_OK>(T, h, old, nw, inv, scaled, ci, beg, end, k0, k1, inj,
                                           reg, q, sh);
  else if (T.grad_dtype == LUMA_GRAD_F16)
    pass2_dispatch<LUMA_GRAD_F16, INJ_OK>(T, h, old, nw, inv, scaled, ci, beg, end, k0, k1, inj,
                                          reg, q, sh);
  else
    pass2_dispatch<LUMA_GRAD_F32, INJ_OK>(T, h, old, nw, inv, scaled, ci, beg, end, k0, k1, inj,
                                          reg, q, sh);
}

// ---------------------------------------------------------------------------
//  Scale slots, decode (export) and quantise (import)
// ---------------------------------------------------------------------------

// Writes the state of one slot: step count t, the scales of step t and its grid.
__device__ void write_slot(Slot &s, int64_t t, double s_m, double s_v, double eps) {
  const int par = (int)(t & 1);
  s.s_m[par] = s_m;
  s.s_v[par] = s_v;
  make_grid(s_m, s_v, eps, s.grid[par]);
  make_fast(s.grid[par], (float)eps);
  s.step = t;
  s.summ_step = 0;   // codes written by other means: no summaries for them
  s.summ_shift = 0;
  s.seed_m = s.seed_v = -1;
}

__global__ void set_scales_kernel(const LumaScaleInit *__restrict__ items, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const LumaScaleInit it = items[i];
  write_slot(*static_cast<Slot *>(it.slot), it.step, it.s_m, it.s_v, it.eps);
}

__global__ void get_scales_kernel(void *const *__restrict__ slots, int n,
                                  double *__restrict__ scales, int64_t *__restrict__ steps) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const Slot &s = *static_cast<const Slot *>(slots[i]);
  const int par = (int)(s.step & 1);
  scales[2 * i] = s.s_m[par];
  scales[2 * i + 1] = s.s_v[par];
  steps[i] = s.step;
}

__global__ __launch_bounds__(kThreads) void decode_kernel(const int16_t *__restrict__ q_m,
                                                          const int16_t *__restrict__ q_w,
                                                          int64_t n, const Slot *__restrict__ slot,
                                                          double eps, float *__restrict__ m_out,
                                                          float *__restrict__ v_out) {
  __shared__ Grid g;
  if (threadIdx.x == 0) {
    const int par = (int)(slot->step & 1);
    make_grid(slot->s_m[par], slot->s_v[par], eps, g);
  }
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
                                                            int nch, Slot *__restrict__ slot,
                                                            int64_t step, double eps) {
  float am = 0.0f, av = 0.0f;
  for (int i = threadIdx.x; i < nch; i += 64) {
    am = nan_max(am, partials[2 * i]);
    av = nan_max(av, partials[2 * i + 1]);
  }
  am = wave_max(am);
  av = wave_max(av);
  if (threadIdx.x == 0) write_slot(*slot, step, py_max((double)am, 1e-9), py_max((double)av, 0.0), eps);
}

__global__ __launch_bounds__(kThreads) void quant_kernel(const float *__restrict__ m,
                                                         const float *__restrict__ v, int64_t n,
                                                         int16_t *__restrict__ q_m,
                                                         int16_t *__restrict__ q_w,
                                                         const Slot *__restrict__ slot, int par,
                                                         double eps, uint64_t seed,
                                                         int noise_mode, const float *__restrict__ u_m,
                                                         const float *__restrict__ u_w) {
  const Grid G = slot->grid[par];
  const float epsf = (float)eps;
  const uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
  const int64_t beg = (int64_t)blockIdx.x * kChunk;
  const int64_t end = beg + kChunk < n ? beg + kChunk : n;
  for (int64_t e0 = beg + (int64_t)threadIdx.x * kVec; e0 < end; e0 += (int64_t)kThreads * kVec) {
    U4 top_m{}, top_w{}, low{};
    if (noise_mode == LUMA_NOISE_PHILOX) {
      top_m = philox_block((uint64_t)e0, PhiloxBase{0, 0}, kBlockTopM, k0, k1);
      top_w = philox_block((uint64_t)e0, PhiloxBase{0, 0}, kBlockTopW, k0, k1);
      low = philox_block((uint64_t)e0, PhiloxBase{0, 0}, kBlockLow, k0, k1);
    }
    for (int j = 0; j < kVec; ++j) {
      const int64_t i = e0 + j;
      if (i >= end) break;
      float um, uw;
      if (noise_mode == LUMA_NOISE_PHILOX) {
        uint32_t bm, bw;
        philox_uniform_bits(top_m, top_w, low, (uint64_t)i, bm, bw);
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

// Step scalars of steps t0 .. t0+n-1 (luma_hyper_rows).
__global__ void hyper_rows_kernel(LumaGroup g, int64_t t0, int n, float *__restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const Hyper h = step_hyper(g, t0 + i);
  float *o = out + 8 * (int64_t)i;
  o[0] = h.beta1;
  o[1] = h.omb1;
  o[2] = h.beta2;
  o[3] = h.omb2;
  o[4] = h.decay;
  o[5] = h.neg_eta;
  o[6] = h.bc2;
  o[7] = h.eps;
}

}  // namespace luma

// ---------------------------------------------------------------------------
//  C ABI
// ---------------------------------------------------------------------------

using namespace luma;

// Workspace of luma_step_noalloc: pass 1's record of each chunk (its two
// maxima and their positions), for at most LUMA_NOALLOC_MAX_CHUNKS chunks
// (4 MiB).  Each GPU the library runs on holds
// its own copy until the process ends.  In host code `scratch` only names the
// symbol; its device address (one per device) comes from hipGetSymbolAddress.
static __device__ __align__(256) float scratch[kPartialWords * (size_t)LUMA_NOALLOC_MAX_CHUNKS];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static float *g_scratch_ptr[kMaxDevices] = {};

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

int64_t luma_summary_words(int64_t numel, int32_t chunk_elems) {
  if (numel <= 0) return 0;
  if (chunk_elems <= 0) chunk_elems = LUMA_CHUNK_ELEMS;
  return ((numel - 1) / chunk_elems + 1) * LUMA_SUMMARY_WORDS;
}

size_t luma_workspace_bytes(int32_t n_chunks) {
  return (size_t)(n_chunks > 0 ? n_chunks : 0) * kPartialWords * sizeof(float);
}

void luma_layout(int32_t out[8]) {
  out[0] = (int32_t)sizeof(LumaTensor);
  out[1] = (int32_t)sizeof(LumaChunk);
  out[2] = (int32_t)sizeof(LumaGroup);
  out[3] = (int32_t)sizeof(LumaScaleInit);
  out[4] = (int32_t)sizeof(LumaStepArgs);
  out[5] = (int32_t)sizeof(Slot);
  out[6] = (int32_t)LUMA_CHUNK_ELEMS;
  out[7] = 0;
}

// The launches of one step over `n_chunks` chunks of `n_tensors` tensors,
// with optional event records between them: pass 1, finalize, pass 2 (in the
// exact-only mode a set with small tensors adds the wavefront-per-tensor
// kernel of each pass).
static int launch_step(StepSrc src, int32_t n_tensors, int32_t n_chunks, float *partials,
                       uint64_t base_seed, int32_t noise_mode, int32_t flags, hipStream_t s,
                       void *const *events) {
  if (noise_mode != LUMA_NOISE_PHILOX && noise_mode != LUMA_NOISE_INJECTED)
    return fail("luma_step: unknown noise_mode");
  // only the fast pass 2 writes code summaries
  src.summaries = (flags & LUMA_FLAG_EXACT_ONLY) == 0;
  auto mark = [&](int i) -> int {
    if (!events || !events[i]) return 0;
    const hipError_t e = hipEventRecord(static_cast<hipEvent_t>(events[i]), s);
    return e == hipSuccess ? 0 : fail("luma_step: event record", e);
  };
  if (int r = mark(0)) return r;
  const bool exact = (flags & LUMA_FLAG_EXACT_ONLY) != 0;
  // chunks [0, medium_from): a workgroup each; [medium_from, small_from): a
  // wavefront each, four per workgroup, in the same launches;
  // [small_from, n_chunks): small tensors, a wavefront each
  // (the fast pass 1 runs the small tensors' exact pass 1 in workgroups past
  // its own, and the fast pass 2 steps them as it steps the medium ones; the
  // exact-only mode leaves them to the small kernels)
  const int32_t blocks = pass_blocks(src.medium_from, src.small_from);
  const int32_t small_blocks = (n_chunks - src.small_from + kThreads / 64 - 1) / (kThreads / 64);
  const int32_t fast_blocks = blocks + (src.tensors ? small_blocks : 0);
  if (exact ? blocks > 0 : fast_blocks > 0) {
    if (exact)
      hipLaunchKernelGGL(pass1_exact_kernel, dim3(blocks), dim3(kThreads), 0, s, src, partials);
    else
      hipLaunchKernelGGL(pass1_fast_kernel, dim3(fast_blocks), dim3(kThreads), 0, s, src, partials);
    if (int r = check_launch("luma_step: pass 1 launch")) return r;
  }
  if (exact && small_blocks > 0) {
    hipLaunchKernelGGL(pass1_small_kernel, dim3(small_blocks), dim3(kThreads), 0, s, src, partials);
    if (int r = check_launch("luma_step: pass 1 (small tensors) launch")) return r;
  }
  if (int r = mark(1)) return r;
  const int32_t fin_waves = finalize_waves(src, n_tensors);
  hipLaunchKernelGGL(finalize_kernel, dim3((fin_waves + kThreads / 64 - 1) / (kThreads / 64)),
                     dim3(kThreads), 0, s, src, (const float *)partials, n_tensors);
  if (int r = check_launch("luma_step: finalize launch")) return r;
  if (int r = mark(2)) return r;
  // the fast pass 2 steps the small tensors as it does the medium ones, one
  // wavefront each in workgroups after theirs
  const int32_t p2_blocks = pass_blocks(src.medium_from, src.tensors ? n_chunks : src.small_from);
  if (exact ? blocks > 0 : p2_blocks > 0) {
    if (exact)
      hipLaunchKernelGGL(pass2_exact_kernel, dim3(blocks), dim3(kThreads), 0, s, src, base_seed,
                         (int)noise_mode);
    else if (noise_mode == LUMA_NOISE_INJECTED)
      hipLaunchKernelGGL(pass2_fast_kernel<true>, dim3(p2_blocks), dim3(kThreads), 0, s, src,
                         base_seed, (int)noise_mode);
    else
      hipLaunchKernelGGL(pass2_fast_kernel<false>, dim3(p2_blocks), dim3(kThreads), 0, s, src,
                         base_seed, (int)noise_mode);
    if (int r = check_launch("luma_step: pass 2 launch")) return r;
  }
  if (exact && small_blocks > 0) {
    hipLaunchKernelGGL(pass2_small_kernel, dim3(small_blocks), dim3(kThreads), 0, s, src,
                       base_seed, (int)noise_mode);
    if (int r = check_launch("luma_step: pass 2 (small tensors) launch")) return r;
  }
  return mark(3);
}

static int step_impl(const LumaStepArgs *a, void *stream, void *const *events) {
  if (!a) return fail("luma_step: null args");
  if (a->n_tensors <= 0 || a->n_chunks <= 0) return 0;
  if (!a->tensors || !a->chunks || !a->groups || !a->partials)
    return fail("luma_step: null table pointer");
  if ((uintptr_t)a->partials & 15u) return fail("luma_step: partials must be 16-byte aligned");
  const int32_t c = a->chunk_elems ? a->chunk_elems : (int32_t)LUMA_CHUNK_ELEMS;
  if (c < LUMA_CHUNK_ELEMS_MIN || c > LUMA_CHUNK_ELEMS || (c & (c - 1)) != 0)
    return fail("luma_step: chunk_elems must be a power of two in [LUMA_CHUNK_ELEMS_MIN, LUMA_CHUNK_ELEMS]");
  StepSrc src{};
  src.tensors = reinterpret_cast<const Tensor *>(a->tensors);
  src.chunks = a->chunks;
  src.groups = a->groups;
  src.scaling = a->scaling;
  src.chunk_shift = __builtin_ctz((unsigned)c);
  if (a->small_chunks < 0 || a->small_chunks > a->n_chunks)
    return fail("luma_step: small_chunks must be in [0, n_chunks]");
  if (a->medium_chunks < 0 || a->medium_chunks > a->n_chunks - a->small_chunks)
    return fail("luma_step: medium_chunks must be in [0, n_chunks - small_chunks]");
  src.small_from = a->n_chunks - a->small_chunks;
  src.medium_from = src.small_from - a->medium_chunks;
  src.n_chunks = a->n_chunks;
  return launch_step(src, a->n_tensors, a->n_chunks, a->partials, a->base_seed, a->noise_mode,
                     a->flags, static_cast<hipStream_t>(stream), events);
}

int luma_step(const LumaStepArgs *a, void *stream) { return step_impl(a, stream, nullptr); }

int luma_step_profiled(const LumaStepArgs *a, void *stream, void *const events[4]) {
  return step_impl(a, stream, events);
}

// Device address of this device's `scratch`, looked up on the first call
// made with the device current and kept for later calls.
static int scratch_for(hipStream_t stream, float **out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail("luma_step_noalloc: hipGetDevice", e);
  if (stream) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess) return fail("luma_step_noalloc: hipStreamGetDevice", e);
    if ((int)sdev != dev) return fail("luma_step_noalloc: the stream's device must be the current device");
  }
  if (dev < 0 || dev >= kMaxDevices) return fail("luma_step_noalloc: device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) return fail("luma_step_noalloc: hipGetSymbolAddress(scratch)", e);
    g_scratch_ptr[dev] = static_cast<float *>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

int luma_step_noalloc(const LumaStepArgs *a, void *stream) {
  if (!a) return fail("luma_step_noalloc: null args");
  if (a->n_tensors <= 0 || a->n_chunks <= 0) return 0;
  if (a->n_chunks > LUMA_NOALLOC_MAX_CHUNKS)
    return fail("luma_step_noalloc: more chunks than LUMA_NOALLOC_MAX_CHUNKS (use luma_step with a "
                "caller-allocated workspace, or a longer chunk_elems)");
  float *ws = nullptr;
  if (int r = scratch_for(static_cast<hipStream_t>(stream), &ws)) return r;
  LumaStepArgs b = *a;
  b.partials = ws;   // every chunk writes its record before finalize reads it
  return step_impl(&b, stream, nullptr);
}

int luma_step_tensor(const LumaTensor *tensor, const LumaGroup *group, float *partials,
                     uint64_t base_seed, int32_t noise_mode, int32_t flags,
                     const LumaScaling *scaling, void *stream) {
  if (!tensor || !group) return fail("luma_step_tensor: null tensor or group");
  if (tensor->numel <= 0) return 0;
  if (!tensor->param || !tensor->grad || !tensor->q_m || !tensor->q_w || !tensor->slot ||
      !partials)
    return fail("luma_step_tensor: null pointer");
  if ((uintptr_t)partials & 15u) return fail("luma_step_tensor: partials must be 16-byte aligned");
  if (noise_mode == LUMA_NOISE_INJECTED && (!tensor->u_m || !tensor->u_w))
    return fail("luma_step_tensor: injected noise needs u_m and u_w");
  // 4096 chunks fill the chip (16 workgroups per CU); a smaller tensor takes
  // shorter chunks, down to LUMA_STEP_TENSOR_CHUNK_MIN
  int shift = __builtin_ctz((unsigned)LUMA_CHUNK_ELEMS);
  while (shift > __builtin_ctz((unsigned)LUMA_STEP_TENSOR_CHUNK_MIN) &&
         ((tensor->numel - 1) >> shift) + 1 < 4096)
    --shift;
  const int64_t nch = ((tensor->numel - 1) >> shift) + 1;
  if (nch > 0x7fffffff) return fail("luma_step_tensor: tensor too large");
  StepSrc src{};
  memcpy(&src.one, tensor, sizeof(Tensor));
  src.one.first_chunk = 0;
  src.group = *group;
  src.chunk_shift = shift;
  src.small_from = (int32_t)nch;   // one tensor: every chunk takes a workgroup
  src.medium_from = (int32_t)nch;
  src.n_chunks = (int32_t)nch;
  if (scaling) src.scaling = *scaling;
  return launch_step(src, 1, (int32_t)nch, partials, base_seed, noise_mode, flags,
                     static_cast<hipStream_t>(stream), nullptr);
}

int luma_set_scales(const LumaScaleInit *items, int32_t n, void *stream) {
  if (n <= 0) return 0;
  if (!items) return fail("luma_set_scales: null pointer");
  hipLaunchKernelGGL(set_scales_kernel, dim3((n + 63) / 64), dim3(64), 0,
                     static_cast<hipStream_t>(stream), items, n);
  return check_launch("luma_set_scales: launch");
}

int luma_get_scales(void *const *slots, int32_t n, double *scales, int64_t *steps, void *stream) {
  if (n <= 0) return 0;
  if (!slots || !scales || !steps) return fail("luma_get_scales: null pointer");
  hipLaunchKernelGGL(get_scales_kernel, dim3((n + 63) / 64), dim3(64), 0,
                     static_cast<hipStream_t>(stream), slots, n, scales, steps);
  return check_launch("luma_get_scales: launch");
}

int luma_decode(const int16_t *q_m, const int16_t *q_w, int64_t numel, const void *slot,
                double eps, float *m_out, float *v_out, void *stream) {
  if (numel <= 0) return 0;
  if (!q_m || !q_w || !slot || !m_out || !v_out) return fail("luma_decode: null pointer");
  int64_t blocks = (numel + kThreads * 8 - 1) / (kThreads * 8);
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(decode_kernel, dim3((unsigned)blocks), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), q_m, q_w, numel,
                     static_cast<const Slot *>(slot), eps, m_out, v_out);
  return check_launch("luma_decode: launch");
}

int luma_quantize(const float *m, const float *v, int64_t numel, int16_t *q_m, int16_t *q_w,
                  void *slot, int64_t step, double eps, uint64_t seed, int32_t noise_mode,
                  const float *u_m, const float *u_w, float *partials, void *stream) {
  if (numel <= 0) return 0;
  if (!m || !v || !q_m || !q_w || !slot || !partials) return fail("luma_quantize: null pointer");
  if (noise_mode == LUMA_NOISE_INJECTED && (!u_m || !u_w))
    return fail("luma_quantize: injected noise needs u_m and u_w");
  if (noise_mode != LUMA_NOISE_PHILOX && noise_mode != LUMA_NOISE_INJECTED)
    return fail("luma_quantize: unknown noise_mode");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t nch = (numel + kChunk - 1) / kChunk;
  if (nch > 0x7fffffff) return fail("luma_quantize: tensor too large");
  Slot *S = static_cast<Slot *>(slot);
  const int par = (int)(step & 1);
  hipLaunchKernelGGL(quant_max_kernel, dim3((unsigned)nch), dim3(kThreads), 0, s, m, v, numel,
                     partials);
  if (int r = check_launch("luma_quantize: max launch")) return r;
  hipLaunchKernelGGL(quant_finalize_kernel, dim3(1), dim3(64), 0, s, partials, (int)nch, S, step,
                     eps);
  if (int r = check_launch("luma_quantize: finalize launch")) return r;
  hipLaunchKernelGGL(quant_kernel, dim3((unsigned)nch), dim3(kThreads), 0, s, m, v, numel, q_m, q_w,
                     (const Slot *)S, par, eps, seed, noise_mode, u_m, u_w);
  return check_launch("luma_quantize: launch");
}

int luma_hyper_rows(const LumaGroup *group, int64_t t0, int32_t n, float *out, void *stream) {
  if (n <= 0) return 0;
  if (!group || !out) return fail("luma_hyper_rows: null pointer");
  if (t0 < 1) return fail("luma_hyper_rows: steps start at 1");
  hipLaunchKernelGGL(hyper_rows_kernel, dim3((n + 255) / 256), dim3(256), 0,
                     static_cast<hipStream_t>(stream), *group, t0, n, out);
  return check_launch("luma_hyper_rows: launch");
}

void luma_philox4x32(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
  const U4 o = philox4x32_10(ctr[0], ctr[1], ctr[2], ctr[3], key[0], key[1]);
  out[0] = o.x;
  out[1] = o.y;
  out[2] = o.z;
  out[3] = o.w;
}

}  // extern "C"
