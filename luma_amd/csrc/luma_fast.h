// Fast per-element arithmetic of the LUMA step with certified error bounds.
//
// The fast path computes m', v' and the quantiser's continuous bin index y
// with hardware transcendentals and fused multiply-adds, together with a
// bound E on |y_fast - y_exact|, where y_exact is what the exact path
// (luma_exact.h, the reference's float32 rounding sequence with correctly
// rounded elementary functions) would compute.  A rounding decision is taken
// from the fast values only when E proves it equals the exact decision;
// otherwise the element is flagged and recomputed on the exact path.  The
// results are therefore bit-identical to the exact path; the bounds only
// decide how often the exact path runs.
//
// Decision rule.  LogSR (functional.py:38-67) returns k + [u < p*(y - k)]
// with p* non-decreasing in the fraction, so for a fixed uniform u it equals
// floor(y - t(u)) + 1 where t = p*^{-1}.  With p*(f) = expm1(f*d)/expm1(d)
// one has |t(u) - u| <= d/8 (d <= 3e-3 for any float32 scale), so with u in
// an interval [c - h0, c + h0] the decision is certain when
// [y - c - h, y - c + h], h = h0 + E + d/8 + slack, holds no integer.
//
// Worst-case errors of the gfx950 instructions used, measured over every
// normal float32 input against float64 (u = 2^-24): v_exp_f32 1.42u,
// v_log_f32 2.0u * max(|log2 x|, 1), v_sqrt_f32 1.56u, v_rcp_f32 1.54u.
// The bounds below use 2u for each and a safety factor of 2 on the total.
#pragma once

#include <hip/hip_runtime.h>

#include "luma_exact.h"

namespace luma {

constexpr float kU = 5.9604644775390625e-08f;  // 2^-24
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kLn2Hi = 0.693145751953125f;       // ln2 with its low 8 bits cleared
constexpr float kLn2Lo = 1.42860682030941723e-6f;  // ln2 - kLn2Hi
constexpr float kSmall = 0.125f;  // polynomial regime bound of expm1 / log1p
constexpr float kSafety = 2.0f;

// Indices into Grid::fast, filled by make_fast (finalize) for the new grid.
enum FastSlot {
  kIdm = 0,     // f32(1 / dm)
  kYTopM,       // exact y of |m| = S_m (largest momentum bin index)
  kIwmin,       // f32(1 / w_min)
  kNl2dw,       // f32(-ln2 / dw), 0 when delta_w == 0
  kYTopW,       // exact y of w = w_max, 0 when delta_w == 0
  kXTopM,       // f32(32767 * dm): largest momentum decode argument
  kXTopW,       // f32(65535 * dw): largest preconditioner decode argument
  kW2,          // (1 / w_min)^2: bound on (1/w)^2 of any decoded code
  kFastCount
};

// expm1 on [0, x_top]: Taylor polynomial x * (1 + x/2 + ... + x^5/720) when
// x_top <= 1/8 (truncation 0.013u, float32 evaluation < 2.3u), else degree-8
// Taylor below 0.5 and exp2 - 1 above.
__device__ __forceinline__ float fast_expm1_small(float x) {
  float c = fmaf(x, 1.0f / 720.0f, 1.0f / 120.0f);
  c = fmaf(x, c, 1.0f / 24.0f);
  c = fmaf(x, c, 1.0f / 6.0f);
  c = fmaf(x, c, 0.5f);
  c = fmaf(x, c, 1.0f);
  return x * c;
}

__device__ __forceinline__ float fast_expm1_general(float x) {
  float p = fmaf(x, 1.0f / 40320.0f, 1.0f / 5040.0f);
  p = fmaf(x, p, 1.0f / 720.0f);
  p = fmaf(x, p, 1.0f / 120.0f);
  p = fmaf(x, p, 1.0f / 24.0f);
  p = fmaf(x, p, 1.0f / 6.0f);
  p = fmaf(x, p, 0.5f);
  p = fmaf(x, p, 1.0f);
  const float a = x * p;
  const float b = __builtin_amdgcn_exp2f(x * kLog2e) - 1.0f;
  return x < 0.5f ? a : b;
}

// Relative error of the fast expm1 on [0, x_top] vs the correctly rounded value.
__device__ __forceinline__ float fast_expm1_relerr(float x_top) {
  if (x_top <= kSmall) return 4.0f * kU;
  // exp2 branch: (argument rounding x*u + 2u + 1u for the subtraction) * e^x/(e^x-1) <= 2.55
  return 2.55f * (x_top * kU + 4.0f * kU);
}

// log1p on [0, a_top]: Taylor polynomial a * (1 - a/2 + ... - a^7/8) when
// a_top <= 1/8 (truncation 0.11u, float32 evaluation < 2u); else
// 2*atanh(a/(2+a)) (odd series to s^11, s <= 1/5) for a <= 0.5 and
// ln2*log2(b) + (a - (b - 1))/b, b = RN(1 + a), above (log1p >= 0.4 there,
// so v_log_f32's absolute error stays a few u relative).
__device__ __forceinline__ float fast_log1p_small(float a) {
  float c = fmaf(a, -1.0f / 8.0f, 1.0f / 7.0f);
  c = fmaf(a, c, -1.0f / 6.0f);
  c = fmaf(a, c, 1.0f / 5.0f);
  c = fmaf(a, c, -0.25f);
  c = fmaf(a, c, 1.0f / 3.0f);
  c = fmaf(a, c, -0.5f);
  c = fmaf(a, c, 1.0f);
  return a * c;
}

__device__ __forceinline__ float fast_log1p_general(float a) {
  const float s = a * __builtin_amdgcn_rcpf(2.0f + a);
  const float s2 = s * s;
  float c = fmaf(s2, 2.0f / 11.0f, 2.0f / 9.0f);
  c = fmaf(s2, c, 2.0f / 7.0f);
  c = fmaf(s2, c, 2.0f / 5.0f);
  c = fmaf(s2, c, 2.0f / 3.0f);
  c = fmaf(s2, c, 2.0f);
  const float lo = s * c;
  const float b = 1.0f + a;
  const float corr = (a - (b - 1.0f)) * __builtin_amdgcn_rcpf(b);
  const float hi = fmaf(__builtin_amdgcn_logf(b), kLn2, corr);
  return a <= 0.5f ? lo : hi;
}

// Relative error bound of the fast log1p on [0, a_top].
__device__ __forceinline__ float fast_log1p_relerr(float a_top) {
  return a_top <= kSmall ? 4.0f * kU : 10.0f * kU;
}

// Largest a / log1p(a) on [0, a_top]: converts |m'| / dm into bins.
__device__ __forceinline__ float a_over_log1p(float a_top) {
  return a_top > 0.0f ? (float)((double)a_top / ::log1p((double)a_top)) * 1.01f : 1.01f;
}

// Fast decode + EMA of one element (functional.py:113-126, 269-275).
// m-decode argument x = |q| * dm is formed exactly as on the exact path.
struct FastEma {
  float mn;   // m'
  float vn;   // v'
  float am;   // |m| decoded (for the error bound)
  float xw;   // preconditioner decode argument
};

// PRECISE_V: form e^-x with the two-word argument reduction (pass 2, whose
// parameter update and code bounds use v'); pass 1 only needs the cheaper
// single exp2, whose error its max-tracking bound covers (x * u term).
template <bool SMALL_M, bool PRECISE_V>
__device__ __forceinline__ FastEma fast_ema(int qm, int qw, float g, float dm, float dw,
                                            float iwmin, float eps, float b1, float omb1,
                                            float b2, float omb2) {
  FastEma r;
  const float qf = (float)qm;
  const float x = fabsf(qf) * dm;
  const float e = SMALL_M ? fast_expm1_small(x) : fast_expm1_general(x);
  const float m = copysignf(e, qf);
  r.am = e;
  r.xw = (float)(qw & 0xFFFF) * dw;
  // w_min / w = e^-x: 2^a with a = RN(-x*log2e), times e^d, where
  // d = -x - a*ln2 is formed with a two-word ln2, so the rounding of the
  // exponent argument does not scale with x.
  const float a = r.xw * -kLog2e;
  float ex = __builtin_amdgcn_exp2f(a);
  if (PRECISE_V) {
    float d = fmaf(a, -kLn2Hi, -r.xw);
    d = fmaf(a, -kLn2Lo, d);
    ex = fmaf(ex, d, ex);
  }
  const float rr = fmaf(iwmin, ex, -eps);  // 1/w - eps
  const float v = rr * rr;
  const float c1g = omb1 * g;
  const float g2 = g * g;
  const float c2g2 = omb2 * g2;
  r.mn = fmaf(b1, m, c1g);
  r.vn = fmaf(b2, v, c2g2);
  return r;
}

}  // namespace luma

namespace luma {

// Derived constants of a freshly computed grid (finalize, set_scales, import).
__device__ inline void make_fast(Grid &g) {
  for (int i = 0; i < 20; ++i) g.fast[i] = 0.0f;
  g.fast[kIdm] = (float)(1.0 / (double)g.dm);
  g.fast[kYTopM] = cr_log1p(g.sm) / g.dm;
  g.fast[kIwmin] = (float)(1.0 / (double)g.wmin);
  g.fast[kNl2dw] = g.dwpos ? (float)(-0.6931471805599453 / (double)g.dw) : 0.0f;
  g.fast[kYTopW] = g.dwpos ? cr_log(g.wmax / g.wmin) / g.dw : 0.0f;
  g.fast[kXTopM] = 32767.0f * g.dm;
  g.fast[kXTopW] = 65535.0f * g.dw;
  const double iw = 1.0 / (double)g.wmin;
  g.fast[kW2] = (float)(iw * iw * (1.0 + 1e-6));
}

// Error bounds of one tensor's fast path for one step (built per workgroup).
struct Bounds {
  // pass 1: |m'_exact| in |m'_fast| * (1 +- dlt_m) +- abs_m, same for v'.
  float dlt_m, abs_m, dlt_v, abs_v;
  // pass 2: |y_fast - y_exact| <= |m| * k1 + y * k2 + k3 (momentum)
  //                             <= x_w * k6 + y * k7 + k8 (preconditioner)
  float k1, k2, k3, k6, k7, k8;
};

// old: grid the codes were written with (null at t = 1); nw: grid of the
// new scales (null in pass 1).
__device__ inline Bounds make_bounds(const Grid *old, const Grid *nw, float b1, float b2) {
  Bounds B;
  const float rho_x = 2.0f * kU;  // v_exp_f32
  float rho_e1 = 0.0f, rho_p = 0.0f, s_old = 0.0f, w2 = 0.0f;
  if (old) {
    rho_e1 = fast_expm1_relerr(old->fast[kXTopM]) + 0.5f * kU;
    rho_p = rho_x + 6.0f * kU + (nw ? 0.0f : old->fast[kXTopW] * kU);
    s_old = old->sm * 1.01f;
    w2 = old->fast[kW2];
  }
  B.dlt_m = kSafety * 1.0f * kU;
  B.abs_m = kSafety * b1 * s_old * (rho_e1 + 0.5f * kU) + 1e-37f;
  B.dlt_v = kSafety * 2.5f * kU;
  B.abs_v = kSafety * 2.0f * b2 * w2 * rho_p + 1e-37f;
  B.k1 = B.k2 = B.k3 = B.k6 = B.k7 = B.k8 = 0.0f;
  if (nw) {
    const float rho_l = fast_log1p_relerr(nw->sm);
    const float aol = a_over_log1p(nw->sm);
    B.k1 = old ? kSafety * b1 * (rho_e1 + 0.5f * kU) * nw->fast[kIdm] : 0.0f;
    B.k2 = kSafety * (kU * aol + rho_l + 3.0f * kU);
    B.k3 = nw->dm * 0.125f + 8.0f * kU + 1e-6f;
    if (nw->dwpos) {
      const float idw = 1.0f / nw->dw;
      B.k6 = 0.0f;
      B.k7 = kSafety * 4.4f * kU;
      B.k8 = kSafety * ((old ? rho_x + 13.0f * kU : 8.0f * kU) * idw) + nw->dw * 0.125f +
             8.0f * kU + 1e-6f;
    }
  }
  return B;
}

}  // namespace luma
