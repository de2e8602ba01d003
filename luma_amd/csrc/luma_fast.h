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
// normal float32 input against float64 (u = 2^-24, the unit roundoff):
// v_exp_f32 1.42u, v_log_f32 2.0u * max(|log2 x|, 1) (absolute, log2
// units), v_sqrt_f32 1.56u, v_rcp_f32 1.54u.  The pass-2 bounds below are
// first-order sums of every rounding of both paths (derivations at
// make_bounds) times kSafety2 = 1.05.  The sums bound the first-order error
// for these instruction errors; the higher-order terms (products of
// roundings) are at most the first-order sum times its own relative size,
// about 30u, so below 2e-6 of the bound, which the 5% covers.  (Compared
// with the exact path over 1.6e10 elements of five parameter sets, the
// first codes that differ appear at a factor 0.25; at 0.5 none do.)  Pass 1
// keeps a factor of 2.
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
constexpr float kSafety = 2.0f;     // pass 1
constexpr float kSafety2 = 1.05f;   // pass 2

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
  kCwHi,        // C = -ln2/dw (double) rounded to 16 significant bits, 0 when delta_w == 0
  kCwLo,        // f32(C - kCwHi)
  kWe,          // f32(w_min * eps)
  kXMin,        // f32(w_min / w_max): smallest w_min * t of an unclamped w
  kFastCount
};

// Near-minimax polynomials for expm1(x)/x and log1p(a)/a on (0, 1/8]
// (relative-error weighted least squares, leading coefficient fixed at 1,
// coefficients rounded to float32).  Truncation error 0.003u and 0.007u;
// float32 Horner evaluation of x * c(x) measured at most 1.98u and 1.51u
// over 3.2M points (tests/test_fast_poly.py).
constexpr float kExpm1Poly[5] = {1.0f, 4.999999702e-01f, 1.666688621e-01f, 4.161759466e-02f,
                                 8.779187687e-03f};
constexpr float kLog1pPoly[6] = {1.0f, -4.999998808e-01f, 3.333228827e-01f, -2.496366203e-01f,
                                 1.942020208e-01f, -1.225474551e-01f};
// expm1(x)/x on (0, 1/2] for the medium regime (same fit, degree 5): float32
// Horner evaluation of x * c(x) measured at most 2.0u (tests/test_fast_poly.py),
// against 1.97u for the degree-7 Taylor polynomial of the general form.
constexpr float kExpm1PolyMed[6] = {1.0f, 5.000001788e-01f, 1.666617095e-01f, 4.171263799e-02f,
                                    8.149511181e-03f, 1.715260907e-03f};

// expm1 on [0, x_top]: kExpm1Poly when x_top <= 1/8, else degree-8 Taylor
// below 0.5 and exp2 - 1 above.
__device__ __forceinline__ float fast_expm1_small(float x) {
  float c = fmaf(x, kExpm1Poly[4], kExpm1Poly[3]);
  c = fmaf(x, c, kExpm1Poly[2]);
  c = fmaf(x, c, kExpm1Poly[1]);
  c = fmaf(x, c, kExpm1Poly[0]);
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
  if (x_top <= kSmall) return 3.0f * kU;
  // exp2 branch: (argument rounding x*u + 2u + 1u for the subtraction) * e^x/(e^x-1) <= 2.55
  return 2.55f * (x_top * kU + 4.0f * kU);
}

// log1p on [0, a_top]: kLog1pPoly when a_top <= 1/8; else
// 2*atanh(a/(2+a)) (odd series to s^11, s <= 1/5) for a <= 0.5 and
// ln2*log2(b) + (a - (b - 1))/b, b = RN(1 + a), above (log1p >= 0.4 there,
// so v_log_f32's absolute error stays a few u relative).
__device__ __forceinline__ float fast_log1p_small(float a) {
  float c = fmaf(a, kLog1pPoly[5], kLog1pPoly[4]);
  c = fmaf(a, c, kLog1pPoly[3]);
  c = fmaf(a, c, kLog1pPoly[2]);
  c = fmaf(a, c, kLog1pPoly[1]);
  c = fmaf(a, c, kLog1pPoly[0]);
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
  return a_top <= kSmall ? 3.0f * kU : 10.0f * kU;
}

// Momentum regimes of a tensor's fast path, from its largest decode argument
// x_top = 32767 dm (old grid) and its largest |m'|, S_m (new scale):
//   kRegSmall    x_top <= 1/8 and S_m <= 1/8: the minimax polynomials;
//   kRegMedium   x_top < 1/2 and S_m <= 1/2: a degree-5 minimax expm1 on
//                (0, 1/2] and the atanh-series log1p to s^9, no second
//                branch and no per-element select;
//   kRegGeneral  both branches of each and a select per element.
// Bounds charged (make_bounds): expm1, fast_expm1_relerr(x_top) in every
// regime (3u up to 1/8, above that at least 10.5u; the medium and general
// polynomials stay within 2u); log1p, 3u in the small regime and 10u
// otherwise, whatever S_m is (the atanh forms: the rounding of 2 + a, of
// v_rcp_f32 and of the product give s within 3.6u, the series to s^9 adds
// 2.9u at most, to s^11 2.9u as well: below 7u).  The series stays within
// that for a fast |m'| a few ulp above S_m.
constexpr int kRegSmall = 0, kRegMedium = 1, kRegGeneral = 2;
constexpr float kMedium = 0.5f;

__device__ __forceinline__ int momentum_regime(float x_top, float sm) {
  if (x_top <= kSmall && sm <= kSmall) return kRegSmall;
  if (x_top < kMedium && sm <= kMedium) return kRegMedium;
  return kRegGeneral;
}

template <int REG>
__device__ __forceinline__ float fast_expm1(float x) {
  if (REG == kRegSmall) return fast_expm1_small(x);
  if (REG == kRegGeneral) return fast_expm1_general(x);
  float c = fmaf(x, kExpm1PolyMed[5], kExpm1PolyMed[4]);
  c = fmaf(x, c, kExpm1PolyMed[3]);
  c = fmaf(x, c, kExpm1PolyMed[2]);
  c = fmaf(x, c, kExpm1PolyMed[1]);
  c = fmaf(x, c, kExpm1PolyMed[0]);
  return x * c;
}

template <int REG>
__device__ __forceinline__ float fast_log1p(float a) {
  if (REG == kRegSmall) return fast_log1p_small(a);
  if (REG == kRegGeneral) return fast_log1p_general(a);
  const float s = a * __builtin_amdgcn_rcpf(2.0f + a);
  const float s2 = s * s;
  float c = fmaf(s2, 2.0f / 9.0f, 2.0f / 7.0f);
  c = fmaf(s2, c, 2.0f / 5.0f);
  c = fmaf(s2, c, 2.0f / 3.0f);
  c = fmaf(s2, c, 2.0f);
  return s * c;
}

// Fast decode + EMA of one element (functional.py:113-126, 269-275).
// m-decode argument x = |q| * dm is formed exactly as on the exact path.
struct FastEma {
  float mn;   // m'
  float vn;   // v'
  float am;   // |m| decoded (for the error bound)
  float v;    // v decoded
};

// ndw = -dw, nbias = 2^23 dw; sign = 0x80000000 (passed in so that callers
// can keep them in VGPRs).  qw holds the bits of the float 2^23 + q (code q
// in the low 16 bits), so the preconditioner argument
// fma(2^23 + q, -dw, 2^23 dw) = RN(q * -dw) is exactly -(the exact path's
// float32 q * dw), formed without a v_cvt.
//
// PRECISE_V: form e^-x with the two-word argument reduction (pass 2, whose
// parameter update and code bounds use v'); pass 1 only needs the cheaper
// single exp2, whose error its max-tracking bound covers (x * u term).
template <int REG_M, bool PRECISE_V>
__device__ __forceinline__ FastEma fast_ema(int qm, int qw, float g, float dm, float ndw,
                                            float nbias, float iwmin, float eps, float b1, float omb1,
                                            float b2, float omb2, uint32_t sign) {
  FastEma r;
  const float qf = (float)qm;
  const float x = fabsf(qf) * dm;
  const float e = fast_expm1<REG_M>(x);
  const float m = __uint_as_float(__float_as_uint(e) | (__float_as_uint(qf) & sign));
  r.am = e;
  const float nx = fmaf(__int_as_float(qw), ndw, nbias);
  // w_min / w = e^-x: 2^a with a = RN(-x*log2e), times e^d, where
  // d = -x - a*ln2 is formed with a two-word ln2, so the rounding of the
  // exponent argument does not scale with x.
  const float a = nx * kLog2e;
  float ex = __builtin_amdgcn_exp2f(a);
  if (PRECISE_V) {
    float d = fmaf(a, -kLn2Hi, nx);
    d = fmaf(a, -kLn2Lo, d);
    ex = fmaf(ex, d, ex);
  }
  const float rr = fmaf(iwmin, ex, -eps);  // 1/w - eps
  const float v = rr * rr;
  r.v = v;
  const float c1g = omb1 * g;
  const float g2 = g * g;
  const float c2g2 = omb2 * g2;
  r.mn = fmaf(b1, m, c1g);
  r.vn = fmaf(b2, v, c2g2);
  return r;
}

}  // namespace luma

namespace luma {

// Derived constants of a freshly computed grid (finalize, set_scales, import);
// eps is the group's float32 eps.
__device__ inline void make_fast(Grid &g, float eps) {
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
  if (g.dwpos) {
    const double c = -0.6931471805599453 / (double)g.dw;
    int e;
    const double m = ::frexp(c, &e);
    const double hi = ::ldexp(::nearbyint(::ldexp(m, 16)), e - 16);
    g.fast[kCwHi] = (float)hi;
    g.fast[kCwLo] = (float)(c - hi);
  }
  g.fast[kWe] = (float)((double)g.wmin * (double)eps);
  g.fast[kXMin] = (float)((double)g.wmin / (double)g.wmax);
}

// Error bounds of one tensor's fast path for one step (built per workgroup).
struct Bounds {
  // pass 1: |m'_exact| in |m'_fast| * (1 +- dlt_m) +- abs_m, same for v'.
  float dlt_m, abs_m, dlt_v, abs_v;
  // pass 2, in bins: |z_fast - z_exact| <= |m| * k1 + z * k2 + k3 (momentum)
  //                                      <= A * k7 + k8 (preconditioner)
  // where z is the bin index plus an offset in (0, 1] and A = e * C_hi.
  float k1, k2, k3, k7, k8;
};

// old: grid the codes were written with (null at t = 1); nw: grid of the
// new scales (null in pass 1).
//
// Momentum (first order; a = |m'|, y = log1p(a)/dm).  Decode: the fast
// expm1 (rho_e) and the exact one (u) differ by (rho_e + u)|m|; the exact
// path's b1*m rounds once more (u b1 |m|); both EMAs round the sum (u a
// each; omb1*g is the same float32 product in both).  A change da moves y
// by da/((1+a) dm), and a/((1+a) log1p a) <= 1, so the EMA terms cost
// 2u y.  Then the fast log1p (rho_l y), 1/dm's rounding (u y), the exact
// log1p and division (2u y) and the fused z = L/dm + offset (u (y + 1)):
//   k1 = b1 (rho_e + 2u) / dm,  k2 = rho_l + 6u,  k3 = u  (times kSafety2).
//
// Preconditioner (relative error of x = w_min t against the exact path's
// 1 / (w / w_min); P = 1/w_old, R = P - eps).  Exact decode rounds exp,
// w_min*E and 1/W (3u); the fast one has 1/w_min's rounding, exp2 with
// the two-word reduction and its fma (u + 2.42u): |P_f - P_E| <= 6.42u P.
// Both round P - eps and r^2.  The EMA, sqrt and t = s + eps propagate
// the decode error with weight (s/t)(b2 v/v')(P/R) <= 1 (because
// v' >= b2 v), giving 6.42u + 3.5u (EMA, squaring) + 3.56u (sqrt: 1.56u +
// u) + u (t) + 2u (1/t, w/w_min) + 2u (fast fma and w_min*eps) = 18.5u
// at t >= 2 (7.6u at t = 1, where v = 0).  In bins that is rel / dw.  Then
// y = (e + log2 mant) C with C = -ln2/dw: v_log_f32 on the mantissa (2u
// log2 units), C's rounding and the product (2u|C|), the fma with C_lo and
// the sum with the offset (2u|C|), x_min's rounding (u/dw), and the exact
// path's log and division (2u y <= 2u (A + |C|)):
//   k7 = 2u,  k8 = (rel + 1 + 4.16 + 1.39) u / dw + 4u  (times kSafety2).
// LogSR's t(u) is within delta/8 of u, added unscaled; 1e-6 covers the
// exact path's rounding of p* (a few u) and of 1 - u.
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
  B.k1 = B.k2 = B.k3 = B.k7 = B.k8 = 0.0f;
  if (nw) {
    const float rho_e = old ? fast_expm1_relerr(old->fast[kXTopM]) : 0.0f;
    // the log1p form is the regime's, which also depends on the old grid
    const int reg = momentum_regime(old ? old->fast[kXTopM] : 0.0f, nw->sm);
    const float rho_l = reg == kRegSmall ? fast_log1p_relerr(nw->sm) : 10.0f * kU;
    B.k1 = old ? kSafety2 * b1 * (rho_e + 2.0f * kU) * nw->fast[kIdm] : 0.0f;
    B.k2 = kSafety2 * (rho_l + 6.0f * kU);
    B.k3 = kSafety2 * kU + nw->dm * 0.125f + 1e-6f;
    if (nw->dwpos) {
      const float idw = 1.0f / nw->dw;
      const float rel = old ? 18.5f * kU : 7.6f * kU;
      B.k7 = kSafety2 * 2.0f * kU;
      B.k8 = kSafety2 * ((rel + 6.55f * kU) * idw + 4.0f * kU) + nw->dw * 0.125f + 1e-6f;
    } else {
      B.k8 = 1e-6f;
    }
  }
  return B;
}

}  // namespace luma
