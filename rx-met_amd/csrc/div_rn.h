// div_rn.h — x / s correctly rounded in fp32 from the correctly rounded reciprocal of s.
//
// Markstein's quotient: with rs = RN(1 / s), q = RN(x rs) is within one ulp of x / s, the
// residual r = x - s q is exact when computed by one fma, and RN(q + r rs) = RN(x / s).  The
// conditions are that the residual neither underflows nor overflows — here x and q both in
// [2^-100, 2^100] — and a quotient of two fp32 values is never a rounding midpoint.  Outside
// that range (zero, tiny or huge operands, NaN, inf, a zero or denormal scale) the division
// itself is taken.  Three operations instead of the dozen of an IEEE division, for kernels
// that divide every element by one scale.
#pragma once

#include <hip/hip_runtime.h>

namespace rxmet {

__device__ __forceinline__ float div_rn(float x, float s, float rs) {
  const float q = x * rs;
  const float ax = fabsf(x), aq = fabsf(q);
  if (ax >= 0x1p-100f && ax <= 0x1p100f && aq >= 0x1p-100f && aq <= 0x1p100f)
    return fmaf(fmaf(-q, s, x), rs, q);
  return x / s;
}

}  // namespace rxmet
