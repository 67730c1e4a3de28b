// Router gate scores (sigmoid and softmax of ref.py:347-361 / ref.py:601-631)
// with a fully specified evaluation, so that any IEEE-754 binary64
// implementation running the same operation sequence returns the same bits.
//
// Only correctly rounded binary64 add, subtract, multiply and divide, floor,
// exact scaling by a power of two, and one final rounding to f32 are used:
// no fused multiply-add (each step is a separate __d*_rn call and the file is
// compiled with fp contraction off), no library exp.
//
// exp(t): Cody & Waite argument reduction (W. J. Cody and W. Waite, "Software
// Manual for the Elementary Functions", Prentice-Hall 1980): n = floor(t/ln2
// + 1/2), r = (t - n*ln2_hi) - n*ln2_lo, with ln2 split as in fdlibm's
// e_exp.c (ln2_hi carries 21 trailing zero bits, so n*ln2_hi is exact for
// |n| < 2^11).  Then the degree-13 Taylor polynomial of e^r on
// |r| <= ln2/2 in Horner form (truncation below 2^-56 relative), scaled by 2^n.
// Arguments above 709 give +inf and below -708 give 0 (the scaled result
// would leave the normal binary64 range).
//
// sigmoid(x) = f32(1 / (1 + exp(-x))): the binary64 value is within a few
// units of 2^-53 relative of the true sigmoid, so the f32 result is the
// correctly rounded sigmoid except when the true value lies within ~2^-50
// relative of an f32 rounding boundary.
#pragma once

#include <hip/hip_runtime.h>

namespace lmoe {

namespace gate {
constexpr double kInvLn2 = 0x1.71547652b82fep+0;
constexpr double kLn2Hi = 0x1.62e42fee00000p-1;
constexpr double kLn2Lo = 0x1.a39ef35793c76p-33;
// 1/j!, j = 0..13, each rounded to nearest binary64
constexpr double kInvFact[14] = {
    0x1.0000000000000p+0,  0x1.0000000000000p+0,  0x1.0000000000000p-1,  0x1.5555555555555p-3,
    0x1.5555555555555p-5,  0x1.1111111111111p-7,  0x1.6c16c16c16c17p-10, 0x1.a01a01a01a01ap-13,
    0x1.a01a01a01a01ap-16, 0x1.71de3a556c734p-19, 0x1.27e4fb7789f5cp-22, 0x1.ae64567f544e4p-26,
    0x1.1eed8eff8d898p-29, 0x1.6124613a86d09p-33};
}  // namespace gate

__device__ __forceinline__ double gate_exp64(double t) {
  if (t != t) return t;
  if (t > 709.0) return __builtin_huge_val();
  if (t < -708.0) return 0.0;
  const double n = floor(__dadd_rn(__dmul_rn(t, gate::kInvLn2), 0.5));
  const double r = __dsub_rn(__dsub_rn(t, __dmul_rn(n, gate::kLn2Hi)), __dmul_rn(n, gate::kLn2Lo));
  double p = gate::kInvFact[13];
#pragma unroll
  for (int j = 12; j >= 0; --j) p = __dadd_rn(__dmul_rn(p, r), gate::kInvFact[j]);
  return ldexp(p, static_cast<int>(n));
}

// The router's sigmoid gate score of one f32 logit.
__device__ __forceinline__ float gate_sigmoid(float x) {
  const double e = gate_exp64(-static_cast<double>(x));
  return __double2float_rn(__ddiv_rn(1.0, __dadd_rn(1.0, e)));
}

}  // namespace lmoe
