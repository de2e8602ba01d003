// Host build of the step-scalar derivation in luma_amd/csrc/luma_hyper.h (the
// code the HIP kernels run), for checking against Python's double arithmetic.
// stdin: lines "lr beta1 beta2 eps weight_decay t0 n" (doubles as %a hex);
// stdout: per step, the 8 float32 scalars as hexadecimal bit patterns.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "luma_hyper.h"

int main() {
  char buf[1024];
  while (fgets(buf, sizeof buf, stdin)) {
    LumaGroup g;
    memset(&g, 0, sizeof g);
    long long t0, n;
    if (sscanf(buf, "%la %la %la %la %la %lld %lld", &g.lr, &g.beta1, &g.beta2, &g.eps,
               &g.weight_decay, &t0, &n) != 7)
      return 2;
    for (long long t = t0; t < t0 + n; ++t) {
      const luma::Hyper h = luma::step_hyper(g, t);
      const float v[8] = {h.beta1, h.omb1, h.beta2, h.omb2, h.decay, h.neg_eta, h.bc2, h.eps};
      for (int i = 0; i < 8; ++i) {
        unsigned u;
        memcpy(&u, &v[i], 4);
        printf(i ? " %08x" : "%08x", u);
      }
      printf("\n");
    }
  }
  return 0;
}
