// Quotient used by the quantizer's fast path, shared by the device code and
// the host-side exhaustive check of the test-suite (same source, so the check
// proves the arithmetic the kernel runs).
#pragma once

#include <stdint.h>

#include "inferop/fp8.h"

namespace inferop_qmath {

// fl32(1/448) = 0x3B124925: scale = absmax * kInv448 (reference.cpp:73).
constexpr float kInv448 = 1.0f / 448.0f;

// Smallest group absmax (as fp32 bits, 2^-80) the fast path accepts for 16-bit
// inputs.  Below it the Markstein residual of an element whose quotient can
// reach the E4M3 range may fall into the fp32 subnormal range and lose bits.
constexpr uint32_t kFastMinAbsmaxBits = 0x17800000u;

// Correctly rounded x / s from r = RN(1/s) (Markstein, IBM J. Res. Dev. 1990):
// q0 = RN(x*r) is within one ulp of x/s, the residual e = x - q0*s is exact
// under a fused multiply-add, and RN(q0 + e*r) is the correctly rounded
// quotient.  The sign of x is put back at the end because q0 + e*r can turn
// a -0 quotient into +0.  Contraction must stay off: q0 has to be rounded.
INFEROP_HD inline float div_by_recip(float x, float s, float r) {
#if defined(__clang__)
#pragma clang fp contract(off)
#endif
  const float q0 = x * r;
  const float e = __builtin_fmaf(-q0, s, x);
  const float q1 = __builtin_fmaf(e, r, q0);
  return __builtin_copysignf(q1, x);
}

}  // namespace inferop_qmath
