// Correctly rounded fp32 division of many dividends by one divisor, in three
// operations each instead of the dozen of a general fp32 divide.
//
// With y = RN(1 / b) computed once (one correctly rounded division),
//   q0 = RN(x * y),  r = fma(-b, q0, x),  q = RN(q0 + r * y)   (fma)
// is the correction step of P. Markstein ("Computation of elementary functions
// on the IBM RISC System/6000 processor", IBM J. Res. Dev. 34(1), 1990): r is
// the exact remainder x - b q0, and one correction gives RN(x / b).  Here it is
// used only where that is certain by exhaustion: x is a bf16 or f16 value (its
// significand is one of the 1024 f16 significands, which include the 128 of
// bf16) and b is any fp32 value; tests/cpp/test_host.cpp "div full" checks the
// sequence against x / b for every (x significand, b significand) pair, and
// the quotient's significand depends on those two alone while no step leaves
// the normal range.  The domain below keeps every step normal:
//   b in [2^-32, 2^32], and x == 0 or |x| >= 2^-60
// (then |x| / b >= 2^-92, the remainder's bits sit no lower than about
// 2^-48 |x| >= 2^-108, far above 2^-126, and |x| <= 2^64 keeps q below 2^96).
// A zero x gets its sign back by copysign, which the fma chain loses for -0.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>

namespace oxide {

// Bitwise & and | rather than && and ||: no short-circuit branches in the
// callers' per-element loops.
__host__ __device__ inline bool exact_div_divisor_ok(float b) { return (b >= 0x1p-32f) & (b <= 0x1p32f); }

__host__ __device__ inline bool exact_div_dividend_ok(float x) {
  const float a = fabsf(x);
  return (x == 0.f) | ((a >= 0x1p-60f) & (a <= 0x1p64f));
}

// RN(x / b) for x, b in the domain above; y must be RN(1 / b) (1.0f / b).
__host__ __device__ inline float exact_div(float x, float b, float y) {
#pragma clang fp contract(off)
  const float q0 = x * y;
  const float r = fmaf(-b, q0, x);
  return copysignf(fmaf(r, y, q0), x);
}

}  // namespace oxide
