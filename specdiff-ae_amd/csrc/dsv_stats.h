// dsv_stats.h — per-row statistics of the acceptance test, shared by the
// logits sweep (dsv_accept.hip) and the fused lm_head (dsv_lmhead.hip).
//
// Argmax: largest value, NaN above every number, ties to the lowest index
// (torch.argmax).  Typical acceptance: online (m, l, s) of the softmax in the
// log2 domain, m = max of y*log2e, l = sum 2^(y*log2e - m),
// s = sum y * 2^(y*log2e - m), merged by rescaling to the larger m.
#pragma once

#include "dsv_internal.h"

namespace dsv {

struct ArgMax {
  float v;
  int i;
};

// a ranks before b: larger value, NaN above all numbers, ties -> lower index.
__device__ __forceinline__ bool am_better(float av, int ai, float bv, int bi) {
  const bool an = av != av, bn = bv != bv;
  if (an || bn) return an && (!bn || ai < bi);
  if (av != bv) return av > bv;
  return ai < bi;
}

struct Soft {
  float m;  // max of y*log2e
  float l;  // sum 2^(z - m)
  float s;  // sum y * 2^(z - m)
};

__device__ __forceinline__ Soft soft_merge(Soft a, Soft b) {
  if (a.m == -__builtin_huge_valf()) return b;
  if (b.m == -__builtin_huge_valf()) return a;
  const float m = fmaxf(a.m, b.m);
  const float fa = __builtin_amdgcn_exp2f(a.m - m), fb = __builtin_amdgcn_exp2f(b.m - m);
  return Soft{m, a.l * fa + b.l * fb, a.s * fa + b.s * fb};
}

}  // namespace dsv
