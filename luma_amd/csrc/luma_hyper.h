// Step scalars of the LUMA update, derived from a param group's
// hyper-parameters (the Python doubles of optimizer.py:80-92) and the step
// count t with the reference's double arithmetic:
//   bc1 = 1 - beta1**t, bc2 = 1 - beta2**t, eta = lr / bc1
//   (functional.py:209-211 at t = 1, 262-264 after),
//   decay = 1 - weight_decay*lr (functional.py:213, 278),
// each rounded once to float32 where the float32 tensor op consumes it.
//
// beta**t is the correctly rounded power, from double-double binary
// powering (relative error below 2^-95 before the final rounding).  Python's
// ** calls the C library's pow, which is within 0.52 ulp and so can differ
// from the correctly rounded power by one double ulp; after the float32
// rounding the two agree (no difference over t = 1 .. 2e6 for fifteen betas
// between 0 and 0.99999).
//
// Plain C++ (host and device): the same code is compiled into the HIP
// library and into a host check.  Needs -ffp-contract=off.
#pragma once

#include <math.h>
#include <stdint.h>

#include "../../include/luma.h"

#ifndef LUMA_HYPER_FN
#if defined(__HIPCC__)
#define LUMA_HYPER_FN __host__ __device__
#else
#define LUMA_HYPER_FN
#endif
#endif

namespace luma {

// Float32 scalars of one (group, step).
struct Hyper {
  float beta1, omb1, beta2, omb2;
  float decay, neg_eta, bc2, eps;
  double eps_d;  // eps itself, for the float64 grid (functional.py:74-92)
};

struct DD {
  double hi, lo;
};

// Product of two double-doubles, normalised (|lo| <= ulp(hi)/2).
LUMA_HYPER_FN inline DD dd_mul(DD a, DD b) {
  const double p = a.hi * b.hi;
  double e = fma(a.hi, b.hi, -p);
  e += a.hi * b.lo + a.lo * b.hi;
  DD r;
  r.hi = p + e;
  r.lo = e - (r.hi - p);
  return r;
}

// Correctly rounded b^t for 0 <= b <= 1 and t >= 1.  Returns 0 once the
// power is below 2^-60, where 1 - b^t rounds to 1 in double either way.
LUMA_HYPER_FN inline double pow_rn(double b, int64_t t) {
  DD r = {1.0, 0.0}, x = {b, 0.0};
  for (;;) {
    if (t & 1) r = dd_mul(r, x);
    t >>= 1;
    if (t == 0) break;
    x = dd_mul(x, x);
    // every later factor, and so the result, is at most x (b <= 1)
    if (x.hi < 0x1p-60) return 0.0;
  }
  return r.hi < 0x1p-60 ? 0.0 : r.hi + r.lo;
}

// Step-independent fields (pass 1 reads only these).
LUMA_HYPER_FN inline Hyper group_hyper(const LumaGroup &g) {
  Hyper h;
  h.beta1 = (float)g.beta1;
  h.omb1 = (float)(1.0 - g.beta1);
  h.beta2 = (float)g.beta2;
  h.omb2 = (float)(1.0 - g.beta2);
  h.decay = (float)(1.0 - g.weight_decay * g.lr);
  h.neg_eta = 0.0f;
  h.bc2 = 1.0f;
  h.eps = (float)g.eps;
  h.eps_d = g.eps;
  return h;
}

// All fields for step t >= 1.
LUMA_HYPER_FN inline Hyper step_hyper(const LumaGroup &g, int64_t t) {
  Hyper h = group_hyper(g);
  const double bc1 = 1.0 - pow_rn(g.beta1, t);
  const double bc2 = 1.0 - pow_rn(g.beta2, t);
  const double eta = g.lr / bc1;
  h.neg_eta = (float)(-eta);
  h.bc2 = (float)bc2;
  return h;
}

}  // namespace luma
