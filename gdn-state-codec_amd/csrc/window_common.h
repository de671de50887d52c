// Constants and wave-level helpers shared by the windowed decode kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gdn {

// Window geometry fixed by the reference (state_capsule.cpp:29-32;
// windowed_gdn_step.cpp:6-10): p = 16 records, rank-4 compensators, and one
// position word per 8-word slot so independently written positions do not
// share a 32-byte sector.
constexpr int kWindow = 16;
constexpr int kRank = 4;
constexpr int kPositionStride = 8;
// Largest `states` the windowed entry points admit (windowed_gdn_step.cpp:678).
constexpr uint32_t kMaxWindowStates = 16384;
// Qwen3.5 query scale 128^-1/2 as the bf16 kernels hard-code it
// (windowed_gdn_step.cpp:328, encoded_projection.cpp:374).
constexpr float kQueryScale = 0.08838834764831845f;

// The gate g = exp(log_decay) rounded once to fp32: exp is evaluated in double
// and rounded, so the value does not depend on a single-precision exp's
// last-bit behaviour (the CPU oracle evaluates the same expression).
__device__ __forceinline__ float decay_gate(float log_decay) {
  return static_cast<float>(exp(static_cast<double>(log_decay)));
}

__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
}

// -0.0f as a value the compiler cannot see through (one SGPR); see
// half_product.
__device__ __forceinline__ float opaque_negative_zero() {
  uint32_t bits = 0x80000000u;
  asm("" : "+s"(bits));
  return __uint_as_float(bits);
}

// The product of two fp16 values (the low 16 bits of a_bits and b_bits) in
// fp32. Their 11-bit significands multiply to at most 22 bits and the
// exponents stay in the fp32 normal range, so the product is exact and equals
// widening both operands and multiplying with one rounding. fma(a, b, -0)
// computes it as one v_fma_mix_f32, which widens the halves (op_sel picks the
// high half of a pair) inside the instruction; adding -0 leaves every product,
// a signed zero included, unchanged. neg_zero must come from
// opaque_negative_zero(): with a literal -0 the compiler turns the fma into a
// multiply of two separately widened operands.
__device__ __forceinline__ float half_product(uint32_t a_bits, uint32_t b_bits, float neg_zero) {
  return __builtin_fmaf(half_bits_to_float(a_bits), half_bits_to_float(b_bits), neg_zero);
}

// value - a*b for fp16 a and b: the product is exact (half_product), so one
// fma rounds exactly what the subtraction of the rounded product rounds.
__device__ __forceinline__ float minus_half_product(float value, uint32_t a_bits, uint32_t b_bits) {
  return __builtin_fmaf(-half_bits_to_float(a_bits), half_bits_to_float(b_bits), value);
}

// Round an fp32 value to nearest even fp16 (v_cvt_f16_f32), with fp16
// subnormals. The empty asm pins `value` as a rounded fp32 register:
// without it the compiler folds a producing multiply into v_fma_mixlo_f16,
// which rounds the exact product once to fp16 and differs from rounding the
// fp32 product at fp16 ties.
__device__ __forceinline__ uint32_t float_to_half_bits(float value) {
  asm volatile("" : "+v"(value));
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(value));
}

// Butterfly sum over the 64 lanes; every lane receives the same value.
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int mask = 32; mask >= 1; mask >>= 1) x += __shfl_xor(x, mask);
  return x;
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int mask = 32; mask >= 1; mask >>= 1) x = fmaxf(x, __shfl_xor(x, mask));
  return x;
}

// Orders this wavefront's LDS writes before its later LDS reads of other
// lanes' data (the kernels here synchronize within a wavefront only).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace gdn
