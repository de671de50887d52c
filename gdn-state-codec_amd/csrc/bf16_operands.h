// bf16 operands for v_mfma_f32_16x16x32_bf16 from int8 codes and fp32 values.
//
// Codes are exact in bf16 (the upper half of their exact fp32 value); fp32
// values are split into three bf16 parts that sum to them exactly, so MFMA
// products of codes and parts are exact and only the fp32 accumulation rounds.
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

// Three-way bf16 split of a pair of fp32 values, w = hi + mid + lo exactly,
// by truncation: hi keeps the sign, exponent and top 7 fraction bits of w;
// the remainder r = w - hi is exact in fp32 and has at most 16 significant
// bits; mid keeps the top 8 of those and lo = r - mid, exact, has at most 8,
// so every part is a bf16 value (the upper half of its fp32 pattern).
__device__ __forceinline__ void split3_pair(float w0, float w1, uint32_t& hi,
                                            uint32_t& mid, uint32_t& lo) {
  constexpr uint32_t kUpper = 0xFFFF0000u;
  const uint32_t h0 = __float_as_uint(w0) & kUpper;
  const uint32_t h1 = __float_as_uint(w1) & kUpper;
  const float r0 = w0 - __uint_as_float(h0);
  const float r1 = w1 - __uint_as_float(h1);
  const uint32_t m0 = __float_as_uint(r0) & kUpper;
  const uint32_t m1 = __float_as_uint(r1) & kUpper;
  const float t0 = r0 - __uint_as_float(m0);
  const float t1 = r1 - __uint_as_float(m1);
  hi = upper_halves(h0, h1);
  mid = upper_halves(m0, m1);
  lo = upper_halves(__float_as_uint(t0), __float_as_uint(t1));
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
