// Deterministic fp32 exp / sigmoid shared by the scoring kernel.
//
// The selection of experts must be bit-identical to the CPU restatement on the
// same logits, so exp and sigmoid are not the device library's: they are the
// published Cody-Waite argument reduction followed by a degree-7 Taylor
// polynomial, written as a fixed sequence of fp32-rounded multiplies and adds
// (no contraction into FMA), which numpy float32 reproduces operation by
// operation.
//
//   k = rint(x * log2e)
//   r = (x - k*ln2_hi) - k*ln2_lo      ln2_hi = 0x3F317200 has 15 significant
//                                      bits, so k*ln2_hi is exact for |k| <= 2^9
//   p = ((((((1/7! r + 1/6!) r + 1/5!) r + 1/4!) r + 1/3!) r + 1/2) r + 1) r + 1
//   exp(x) = ldexp(p, k)
//
// x < -86 returns 0 and x > 88 returns +inf, so every finite result is a
// normal float.  Truncation error of the series on |r| <= ln2/2 is ~5e-9
// relative; the rounding of the Horner steps adds a few ulp.
#pragma once
#include <hip/hip_runtime.h>

namespace moe {

__device__ __forceinline__ float det_exp(float x) {
#pragma clang fp contract(off)
  const float LOG2E = 0x1.715476p+0f;
  const float LN2_HI = 0x1.62e4p-1f;
  const float LN2_LO = 0x1.7f7d1cp-20f;
  if (x < -86.0f) return 0.0f;
  if (x > 88.0f) return __builtin_inff();
  const float k = rintf(x * LOG2E);
  float r = x - k * LN2_HI;
  r = r - k * LN2_LO;
  float p = 0x1.a01a02p-13f;  // 1/7!
  p = p * r + 0x1.6c16c2p-10f;
  p = p * r + 0x1.111112p-7f;
  p = p * r + 0x1.555556p-5f;
  p = p * r + 0x1.555556p-3f;
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  return ldexpf(p, (int)k);
}

__device__ __forceinline__ float det_sigmoid(float x) {
#pragma clang fp contract(off)
  const float xc = fminf(fmaxf(x, -86.0f), 86.0f);
  const float e = det_exp(-xc);
  return __fdiv_rn(1.0f, 1.0f + e);
}

}  // namespace moe
