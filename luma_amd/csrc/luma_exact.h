// Exact per-element arithmetic of the LUMA step, float32 with the reference's
// rounding sequence (src/luma_optimizer/functional.py:113-176, 201-219,
// 259-284; optimizer.py:231-235).
//
// Rules that make the results bit-reproducible against the reference:
//  * every multiply, add and divide is one IEEE float32 operation rounded to
//    nearest -- the file must be compiled with -ffp-contract=off and the
//    default correctly rounded float32 divide;
//  * expm1 / exp / log1p / log / sqrt are correctly rounded: evaluated in
//    float64 (ocml, < 1 ulp of float64) and rounded once to float32, which
//    gives the correctly rounded float32 result except for inputs within
//    about 2^-28 relative of a rounding boundary (sqrt: always, since
//    53 >= 2*24+2 makes the double rounding innocuous);
//  * scalars enter as the float32 casts of the reference's Python doubles.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "luma_hyper.h"

namespace luma {

constexpr float kKM = 32767.0f;
constexpr float kKW = 65535.0f;

// Grid of one tensor for one step: float32 casts of _precompute
// (functional.py:74-92) plus the clamp bounds of _quantize_* .
struct Grid {
  float dm;      // f32(delta_m)
  float zm;      // f32(z_m) = f32(expm1(delta_m))
  float wmin;    // f32(w_min)
  float dw;      // f32(delta_w)
  float zw;      // f32(z_w)
  float wmax;    // f32(1 / eps)
  float sm;      // f32(S_m), momentum clamp bound (functional.py:142)
  int32_t dwpos; // delta_w > 0 evaluated in double (functional.py:166)
  float fast[20];
};
static_assert(sizeof(Grid) == 112, "grid layout");

// Persistent per-tensor state (one LUMA_SLOT_BYTES buffer per tensor): the
// step count, scales and grids double-buffered by step parity, and the
// scalars of the latest step.  Step t writes s_m/s_v/grid[t & 1]; its
// decode reads grid[(t - 1) & 1].
struct Slot {
  int64_t step;    // completed steps (0: no state yet, the next step is t = 1)
  int64_t summ_step;   // the step whose pass 2 wrote the tensor's code summaries (0: none)
  double s_m[2];
  double s_v[2];
  Hyper hyp;       // scalars of step `step` (written by the step's finalize)
  Grid grid[2];
  // Elements of the tensor that held the largest |m'| and v' at step `step`
  // (-1: none).  Their exact values at the next step are lower bounds of
  // that step's maxima, whichever elements they are.
  int64_t seed_m, seed_v;
  int32_t summ_shift;   // log2 of the chunk length the code summaries were written with
  int32_t reserved2;
  uint8_t reserved3[16];
  uint8_t pad[LUMA_SLOT_BYTES - 88 - 2 * sizeof(Grid) - 24 - 16];
};
static_assert(sizeof(Hyper) == 40, "hyper layout");
static_assert(offsetof(Slot, grid) == 88, "slot layout");
static_assert(sizeof(Slot) == LUMA_SLOT_BYTES, "slot layout");

__device__ __forceinline__ float cr_expm1(float x) { return (float)::expm1((double)x); }
__device__ __forceinline__ float cr_exp(float x) { return (float)::exp((double)x); }
__device__ __forceinline__ float cr_log1p(float x) { return (float)::log1p((double)x); }
__device__ __forceinline__ float cr_log(float x) { return (float)::log((double)x); }
__device__ __forceinline__ float cr_sqrt(float x) { return (float)__builtin_sqrt((double)x); }

// torch semantics of max/min with a NaN operand: the NaN wins.
__device__ __forceinline__ float nan_max(float a, float b) { return (a != a || a > b) ? a : b; }
__device__ __forceinline__ float clamp_t(float x, float lo, float hi) {
  if (x != x) return x;
  x = x < lo ? lo : x;
  return x > hi ? hi : x;
}

// _precompute (functional.py:74-92) in double; K_M = 32767, K_W = 65535.
__device__ inline void make_grid(double S_m, double S_v, double eps, Grid &g) {
  const double w_min = 1.0 / (::sqrt(S_v) + eps);
  const double delta_m = ::log1p(S_m) / 32767.0;
  const double z_m = ::expm1(delta_m);
  const double ratio = 1.0 / (eps * w_min);
  const double delta_w = ratio > 1.0 ? ::log(ratio) / 65535.0 : 0.0;
  const double z_w = delta_w > 0.0 ? ::expm1(delta_w) : 1.0;
  g.dm = (float)delta_m;
  g.zm = (float)z_m;
  g.wmin = (float)w_min;
  g.dw = (float)delta_w;
  g.zw = (float)z_w;
  g.wmax = (float)(1.0 / eps);
  g.sm = (float)S_m;
  g.dwpos = delta_w > 0.0 ? 1 : 0;
  for (int i = 0; i < 20; ++i) g.fast[i] = 0.0f;
}

// Decode (functional.py:113-116): m = sgn(q) * expm1(|q| * dm).
__device__ __forceinline__ float exact_decode_m(int q, float dm) {
  const float e = cr_expm1((float)(q < 0 ? -q : q) * dm);
  return q > 0 ? e : (q < 0 ? -e : 0.0f);
}

// Decode (functional.py:119-126, 270): v = (1/(w_min*exp(u16(q)*dw)) - eps)_+^2.
__device__ __forceinline__ float exact_decode_v(int q, float wmin, float dw, float eps) {
  const float w = wmin * cr_exp((float)(q & 0xFFFF) * dw);
  float r = 1.0f / w - eps;
  r = (r != r || r > 0.0f) ? r : 0.0f;
  return r * r;
}

// EMA (functional.py:274-275): three / four roundings, no fused multiply-add.
__device__ __forceinline__ void exact_ema(float m, float v, float g, const Hyper &h, float &mn,
                                          float &vn) {
  mn = h.beta1 * m + h.omb1 * g;
  vn = h.beta2 * v + h.omb2 * (g * g);
}

// AdamW update (functional.py:278-279): p*decay + (neg_eta*m')/(sqrt(v'/bc2)+eps).
__device__ __forceinline__ float exact_param_update(float p, float mn, float vn, const Hyper &h) {
  const float p1 = p * h.decay;
  const float den = cr_sqrt(vn / h.bc2) + h.eps;
  return p1 + (h.neg_eta * mn) / den;
}

// LogSR (functional.py:38-67) for one element, delta > 0; u in [0,1).
__device__ __forceinline__ float exact_log_sr(float y, float delta, float z, float u, float kmax) {
  const float k = floorf(y);
  const float fr = y - k;
  const float p = cr_expm1(fr * delta) / z;
  const float q = k + (u < p ? 1.0f : 0.0f);
  return clamp_t(q, 0.0f, kmax);
}

// LogSR up to its decision: the code is qhi when u < p, else qlo, where
// p = exact_sr_prob(a, z) (the same float32 operations as exact_log_sr,
// for callers that know u only to an interval or bracket p first).
__device__ __forceinline__ void exact_log_sr_pair(float y, float delta, float kmax, float &a,
                                                  float &qlo, float &qhi) {
  const float k = floorf(y);
  const float fr = y - k;
  a = fr * delta;
  qlo = clamp_t(k + 0.0f, 0.0f, kmax);
  qhi = clamp_t(k + 1.0f, 0.0f, kmax);
}

// LogSR's probability p* = expm1(a) / z as exact_log_sr rounds it.
__device__ __forceinline__ float exact_sr_prob(float a, float z) { return cr_expm1(a) / z; }

// Bounds pl <= p <= ph of p = exact_sr_prob(a, z) without the double
// expm1, for 0 <= a < 2^-8 and z > 2^-100 (else false).  expm1 by its cubic
// Taylor polynomial (truncation below a^3/24 < 0.05u relative, u = 2^-24),
// its three roundings (2.01u), v_rcp_f32 (1 ulp, 2u) and the product (u):
// |P - p/z| <= 5.01u; the exact path's correctly rounded expm1 and division
// add u each, so |P - p| <= 7.1u p.  The bracket is 16u P wide on each side,
// plus 2^-126 for subnormal p.
__device__ __forceinline__ bool sr_prob_bracket(float a, float z, float &pl, float &ph) {
  if (!(a >= 0.0f && a < 0x1p-8f && z > 0x1p-100f)) return false;
  const float t = fmaf(a, fmaf(a, 1.0f / 6.0f, 0.5f), 1.0f);
  const float P = (a * t) * __builtin_amdgcn_rcpf(z);
  const float d = fmaf(P, 0x1p-20f, 0x1p-126f);
  pl = P - d;
  ph = P + d;
  return true;
}

// The momentum code's sign and int16 conversion (functional.py:146-150).
__device__ __forceinline__ int signed_code_m(float mc, float q) {
  const float s = mc > 0.0f ? q : (mc < 0.0f ? -q : (mc != mc ? mc : 0.0f));
  return (int)s;
}

// Quantise m (functional.py:133-150).
__device__ __forceinline__ int exact_quant_m(float mn, const Grid &g, float u) {
  const float mc = clamp_t(mn, -g.sm, g.sm);
  const float y = cr_log1p(fabsf(mc)) / g.dm;
  const float q = exact_log_sr(y, g.dm, g.zm, u, kKM);
  return signed_code_m(mc, q);
}

// exact_quant_m before the draw: codes for u >= p (lo) and u < p (hi), with
// p = exact_sr_prob(a, g.zm).
__device__ __forceinline__ void exact_quant_m_pair(float mn, const Grid &g, float &a, int &lo,
                                                   int &hi) {
  const float mc = clamp_t(mn, -g.sm, g.sm);
  const float y = cr_log1p(fabsf(mc)) / g.dm;
  float qlo, qhi;
  exact_log_sr_pair(y, g.dm, kKM, a, qlo, qhi);
  lo = signed_code_m(mc, qlo);
  hi = signed_code_m(mc, qhi);
}

// Quantise v (functional.py:153-176); returns the uint16 code in [0, 65535].
__device__ __forceinline__ int exact_quant_w(float vn, const Grid &g, float eps, float u) {
  if (!g.dwpos) return 0;
  const float vc = (vn != vn || vn > 0.0f) ? vn : 0.0f;
  const float w = 1.0f / (cr_sqrt(vc) + eps);
  const float wc = clamp_t(w, g.wmin, g.wmax);
  const float y = cr_log(wc / g.wmin) / g.dw;
  const float q = exact_log_sr(y, g.dw, g.zw, u, kKW);
  return (int)q;
}

// exact_quant_w before the draw: codes for u >= p (lo) and u < p (hi), with
// p = exact_sr_prob(a, g.zw).
__device__ __forceinline__ void exact_quant_w_pair(float vn, const Grid &g, float eps, float &a,
                                                   int &lo, int &hi) {
  if (!g.dwpos) {
    a = 0.0f;
    lo = hi = 0;
    return;
  }
  const float vc = (vn != vn || vn > 0.0f) ? vn : 0.0f;
  const float w = 1.0f / (cr_sqrt(vc) + eps);
  const float wc = clamp_t(w, g.wmin, g.wmax);
  const float y = cr_log(wc / g.wmin) / g.dw;
  float qlo, qhi;
  exact_log_sr_pair(y, g.dw, kKW, a, qlo, qhi);
  lo = (int)qlo;
  hi = (int)qhi;
}

}  // namespace luma
