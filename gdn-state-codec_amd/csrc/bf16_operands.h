// bf16 operands for v_mfma_f32_16x16x32_bf16 from int8 codes and fp32 values.
//
// Codes are exact in bf16 (the upper half of their exact fp32 value).  fp32
// values are split into bf16 parts: three that sum to them exactly, or two
// that leave a remainder below 2^-16 of the value.  MFMA products of a code
// (7 significant bits) and a part (8) are exact, so only the split remainder
// and the fp32 accumulation differ from the exact dot product.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gdn {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;

// Upper halves of two fp32 bit patterns packed as a bf16 pair (low element
// first): one byte permute.
__device__ __forceinline__ uint32_t upper_halves(uint32_t first, uint32_t second) {
  return __builtin_amdgcn_perm(second, first, 0x07060302u);
}

// Two-way bf16 split of a pair of fp32 values, rounding to nearest even
// (one v_cvt_pk_bf16_f32 per part): hi = RN(c), c = w clamped to the largest
// finite bf16 (0x1.fep127), and lo = RN(w - hi), where w - hi is exact in
// fp32 (below the clamp hi is within 2^-8 |w| of w; above it w and hi are in
// [2^127, 2^128) and Sterbenz's lemma applies).  |w - hi| <= 2^-8 |w| and
// |w - hi - lo| <= 2^-8 |w - hi| <= 2^-16 |w| for every finite w with
// |w| >= 2^-110 (bf16 has 8 significant bits and fp32's exponent range, so
// neither rounding underflows there).  Without the clamp a finite
// |w| > 0x1.fep127 would round hi to inf and leave lo = -inf.  A NaN w gives
// a NaN lo.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
constexpr float kLargestBf16 = 0x1.fep127f;

__device__ __forceinline__ void split2_pair(float w0, float w1, uint32_t& hi, uint32_t& lo) {
  const float c0 = fminf(fmaxf(w0, -kLargestBf16), kLargestBf16);
  const float c1 = fminf(fmaxf(w1, -kLargestBf16), kLargestBf16);
  hi = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){c0, c1}, bf16x2_t));
  const float r0 = w0 - __uint_as_float(hi << 16);
  const float r1 = w1 - __uint_as_float(hi & 0xFFFF0000u);
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){r0, r1}, bf16x2_t));
}

// bf16 pair of the signed bytes 2*kPair, 2*kPair+1 of `word` (low element
// first).  bf16 of an int8 code is the upper half of its exact fp32 value: two
// SDWA conversions select and sign-extend the bytes in the operand read, and
// one byte permute packs the two upper halves.  One asm block keeps a single
// temporary live per pair.
template <int kPair>
__device__ __forceinline__ uint32_t bf16_pair_of_codes(uint32_t word) {
  uint32_t packed, low;
  if constexpr (kPair == 0) {
    asm("v_cvt_f32_i32_sdwa %1, sext(%2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_cvt_f32_i32_sdwa %0, sext(%2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1\n\t"
        "v_perm_b32 %0, %0, %1, %3"
        : "=&v"(packed), "=&v"(low) : "v"(word), "s"(0x07060302u));
  } else {
    asm("v_cvt_f32_i32_sdwa %1, sext(%2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
        "v_cvt_f32_i32_sdwa %0, sext(%2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3\n\t"
        "v_perm_b32 %0, %0, %1, %3"
        : "=&v"(packed), "=&v"(low) : "v"(word), "s"(0x07060302u));
  }
  return packed;
}

__device__ __forceinline__ bf16x8 codes_to_bf16x8(uint32_t w0, uint32_t w1) {
  uint4 packed;
  packed.x = bf16_pair_of_codes<0>(w0);
  packed.y = bf16_pair_of_codes<1>(w0);
  packed.z = bf16_pair_of_codes<0>(w1);
  packed.w = bf16_pair_of_codes<1>(w1);
  return __builtin_bit_cast(bf16x8, packed);
}

}  // namespace gdn
