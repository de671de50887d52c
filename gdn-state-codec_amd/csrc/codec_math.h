// Scalar arithmetic shared by the codec kernels, written so the same code can be
// compiled for the host (tests/test_codec_math.py builds it with g++ and checks
// it exhaustively against IEEE division and std::lround).
//
// Bit-exactness contract: the codec reproduces the reference's portable C++
// quant stage (native/src/gdn_state_codec_state_capsule.cpp:190-251), which
// divides with IEEE fp32 division and rounds with std::lround.  The helpers
// below are drop-in replacements that are exact on the domains stated at each
// one; callers fall back to plain `/` outside those domains.
#pragma once

#include <math.h>
#include <stdint.h>

#if defined(__HIPCC__)
#define GDN_HD __host__ __device__ __forceinline__
#else
#define GDN_HD inline
#endif

namespace gdn {

// Quotient a / b from y = RN(1/b) with one residual correction (Markstein 1990,
// "Computation of elementary functions on the IBM RISC System/6000 processor"):
//   q0 = RN(a*y);  r = a - b*q0 (exact, one fma);  q = RN(q0 + r*y).
// It equals RN(a/b) when y = RN(1/b), 2^-100 <= |a| <= 2^120,
// 2^-90 <= |b| <= 2^90 and 2^-120 <= |a/b| <= 2^120: then b*q0 has no bits
// below 2^-149, so r is exactly representable, and no step overflows or
// underflows, which is the theorem's premise.  a == +0 yields +0; a == -0
// yields +0 where IEEE gives -0, so callers keep -0 out (or only use the
// result through fabs or an integer rounding, where the sign cannot show).
GDN_HD float div_by_reciprocal(float a, float b, float y) {
  const float q0 = a * y;
  const float r = fmaf(-q0, b, a);
  return fmaf(r, y, q0);
}

// std::lround for |x| <= 127, returned as int: truncation of x + copysign(c, x)
// with c = 0.5 - 2^-25 (the largest float below 0.5).  Using 0.5 itself would
// round x = 0.5 - 2^-25 up to 1; with c every half-integer still rounds away
// from zero because n + 0.5 + c lies within half an ulp of n + 1 for n >= 1,
// and 0.5 + c = 1 - 2^-25 ties to the even 1.0.  Verified for every float in
// [-127, 127] by tests/test_codec_math.py.
GDN_HD int round_half_away_small(float x) {
  const float c = copysignf(0.49999997f, x);
  return static_cast<int>(x + c);
}

// Largest positive quantized magnitude (kQuantizedMaximum,
// state_capsule.cpp:20) and its correctly rounded reciprocal.
constexpr float kQuantizedMaximum = 127.0f;
constexpr float kInvQuantizedMaximum = 1.0f / 127.0f;

// a / 127 from a two-part reciprocal in two operations: q = RN(a*R + RN(a*L))
// with R = RN(1/127) and L = RN(1/127 - R) (about 2^-35), one multiply and one
// fma.  a*(R + L) is within 2^-55 |a| of a/127 and RN(a*L) adds at most
// 2^-24 |a*L| < 2^-58 |a|, so the fma's argument is within 2^-54 |a| (about
// 2^-47 of the quotient) of a/127.  A quotient a/127 of a normal a is never
// exactly halfway between two floats (that would need 127 to divide a's
// significand, and then the quotient is representable), and it lies at least
// 2^-31 of itself away from every halfway point, since both are multiples of
// 2^(e-8) for a = A * 2^e; so the fma rounds to RN(a/127).  Checked for every
// float with 2^-100 <= |a| < 2^121 by tests/test_codec_math.py; a = +-0
// gives +-0 as IEEE division does.
constexpr float kInvQuantizedMaximumLow =
    static_cast<float>(1.0 / 127.0 - static_cast<double>(1.0f / 127.0f));

GDN_HD float div_by_127(float a) {
  return fmaf(a, kInvQuantizedMaximum, a * kInvQuantizedMaximumLow);
}

// The quant stage's code clamp(lround(p), -127, 127) with p = RN(RN(m / scale)
// * 127) (state_capsule.cpp:213-219), from one fma, a fraction and a floor per
// value.  Preconditions:
// |m| <= scale (scale is the maximum |m| of its column), m finite, and
// factor = RN(127 / scale), or factor = 0 when scale == 0 (then m == 0).
//
// Let a = m / scale, |a| <= 1, and Y = m * factor (exact inside an fma).  Then
// p = 127 a (1+d1)(1+d2) and Y = 127 a (1+d3) with |di| <= 2^-24, so
// |p - Y| <= 127 (3 * 2^-24 + 2^-48) < 2^-15.4.  The lift u = RN(Y + 0.5 +
// 2^-14) adds at most 2^-18 (half an ulp below 128), so p + 0.5 lies within
// 2^-15 of u - 2^-14.  If fract(u) >= 2^-13, then p + 0.5 and Y + 0.5 both lie
// strictly between floor(u) and floor(u) + 1: neither is a tie, and the
// integer nearest p, lround(p), equals the integer nearest Y, which is
// floor(p + 0.5) = floor(u).  |Y| < 127.5, so no clamp is needed.  Values with
// fract(u) < 2^-13 (about 1 in 8,192) take the exact path.
constexpr float kCodeLiftOffset = 0.5f + 0x1p-14f;
constexpr float kCodeLiftMargin = 0x1p-13f;

GDN_HD float code_lift(float m, float factor) { return fmaf(m, factor, kCodeLiftOffset); }

// The same code formed from the product q0 = RN(r * y) of the stage's input r
// and y = RN(1 / s) (the first step of the reciprocal division of r by s), for
// an encoder that keeps q0 instead of m = RN(r / s): u = RN(q0 * factor + 0.5 +
// 2^-14) with factor = RN(127 / scale).  Preconditions: m = RN(r / s)
// satisfies |m| <= scale, r * y and r / s are 0 or normal, factor as above.
// With A = r / s, p = RN(RN(m / scale) * 127) = 127 A / scale (1+d0)(1+d1)(1+d2)
// and Y = q0 * factor = 127 A / scale (1+e1)(1+e2)(1+e3), all |di|, |ei|
// <= 2^-24, and |A / scale| <= 1 + 2^-24, so |p - Y| <= 127 * 6.01 * 2^-24 <
// 2^-14.42; the lift's rounding adds at most 2^-18, so p + 0.5 lies within
// eps = 2^-14.3 of u - 2^-14.  If fract(u) >= 2^-13, p + 0.5 lies strictly
// between floor(u) and floor(u) + 1 (2^-13 - 2^-14 > eps on the low side,
// 2^-14 > eps on the high side): no tie, and lround(p) = floor(u).  Values
// with fract(u) < 2^-13 (about 1 in 8,192) take the exact path.
constexpr float kWideLiftOffset = 0.5f + 0x1p-14f;
constexpr float kWideLiftMargin = 0x1p-13f;

GDN_HD float wide_code_lift(float q0, float factor) {
  return fmaf(q0, factor, kWideLiftOffset);
}

// The exact path's m = RN(r / s) from the kept product q0 = RN(r * y): the
// remaining two steps of div_by_reciprocal(r, s, y).
GDN_HD float quotient_from_product(float q0, float r, float s, float y) {
  return fmaf(fmaf(-q0, s, r), y, q0);
}

// x - floor(x); on the device one v_fract_f32 (which returns the largest float
// below 1 where the subtraction would round to 1; both compare >= the margin).
GDN_HD float lift_fraction(float u) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_fractf(u);
#else
  return u - floorf(u);
#endif
}

// The code of m when its lift u passed the margin: floor(u).  (The encoder
// forms it with v_cvt_flr_i32_f32, which writes floor(u) as an integer.)
GDN_HD int32_t lifted_code(float u) { return static_cast<int32_t>(floorf(u)); }

// Reference smoothing floor (GdnStateCodecParameters::smoothing_floor,
// gdn_state_codec_state_capsule.h:17).
constexpr float kSmoothingFloor = 1.0e-8f;

// bf16 <-> fp32.  Widening is exact; narrowing rounds to nearest even exactly as
// the reference's FloatToBFloat16 (windowed_gdn_step.cpp:26-32).
GDN_HD float bf16_to_float(uint16_t bits) {
  union {
    uint32_t u;
    float f;
  } v;
  v.u = static_cast<uint32_t>(bits) << 16;
  return v.f;
}

GDN_HD uint16_t float_to_bf16(float value) {
  union {
    uint32_t u;
    float f;
  } v;
  v.f = value;
  const uint32_t lsb = (v.u >> 16) & 1u;
  return static_cast<uint16_t>((v.u + 0x7FFFu + lsb) >> 16);
}

// A bf16 input r recovered from q0 = RN(r * y), y = RN(1 / s): r is the bf16
// nearest RN(q0 * s).  q0 * s = r (1+e1)(1+e2)(1+e3) with |ei| <= 2^-24, within
// 2^-22.4 |r| of r, while the bf16 neighbours of r (8 significant bits) are at
// least 2^-8 |r| away, so the nearest bf16 is r itself for every r whose
// product and quotient are 0 or normal (the sign of a zero is kept).
GDN_HD float bf16_input_from_product(float q0, float s) {
  return bf16_to_float(float_to_bf16(q0 * s));
}

}  // namespace gdn
