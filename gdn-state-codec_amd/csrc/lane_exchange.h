// Cross-lane exchanges of a 64-lane wavefront on the VALU: DPP for partners
// lane ^ 1, 2, 4, 8 and the gfx950 permlane swaps for lane ^ 16, 32.  They
// replace ds_bpermute (__shfl_xor), which goes through the LDS unit and needs
// a wait before its result is used.
//
// Every helper forms the same sums and maxima as the butterfly it replaces:
// each lane adds the same two operands (at most commuted, which IEEE addition
// and fmaxf leave bit-identical), so results do not change.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gdn {

// dpp<ctrl, row_mask>(x): x of the DPP source lane; a lane whose source lies
// outside its row, or whose row is masked off, keeps its own x.
template <int kCtrl, int kRowMask = 0xF>
__device__ __forceinline__ int dpp(int x) {
  return __builtin_amdgcn_update_dpp(x, x, kCtrl, kRowMask, 0xF, false);
}
template <int kCtrl, int kRowMask = 0xF>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(dpp<kCtrl, kRowMask>(__float_as_int(x)));
}

constexpr int kDppQuadSwap1 = 0xB1;    // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kDppQuadSwap2 = 0x4E;    // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kDppQuadReverse = 0x1B;  // quad_perm [3,2,1,0]: lane ^ 3
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror: 7 - lane within 8
constexpr int kDppRowRotate8 = 0x128;  // row_ror 8: lane ^ 8 within 16

// x of lane ^ kMask, kMask in {1, 2, 4, 8}.
template <int kMask, typename T>
__device__ __forceinline__ T from_lane_xor(T x) {
  static_assert(kMask == 1 || kMask == 2 || kMask == 4 || kMask == 8, "DPP partner");
  if constexpr (kMask == 1) return dpp<kDppQuadSwap1>(x);
  if constexpr (kMask == 2) return dpp<kDppQuadSwap2>(x);
  // lane ^ 4 = 7 - (lane ^ 3) within each group of 8.
  if constexpr (kMask == 4) return dpp<kDppHalfMirror>(dpp<kDppQuadReverse>(x));
  if constexpr (kMask == 8) return dpp<kDppRowRotate8>(x);
}

// The sum of the two results of a permlane swap.  The elements are copied to
// uint32_t before the bit casts: with this compiler, __builtin_bit_cast
// applied directly to element 1 of the swap's result reads element 0.
template <typename T, typename Pair>
__device__ __forceinline__ T swap_sum(const Pair& r) {
  const uint32_t first = r[0];
  const uint32_t second = r[1];
  return __builtin_bit_cast(T, first) + __builtin_bit_cast(T, second);
}

// One step of a transposing pairwise reduction over lane bit kMask: a lane
// with the bit clear ends with lo + (partner's lo), a lane with the bit set
// with hi + (partner's hi).
template <int kMask, typename T>
__device__ __forceinline__ T fold(T lo, T hi, int lane) {
  if constexpr (kMask == 16 || kMask == 32) {
    // permlane{16,32}_swap(a, b) returns {a with the upper half's a replaced
    // by the lower half's b, b with the lower half's b replaced by the upper
    // half's a}, halves being 16-lane rows (pairs of rows) or 32-lane halves:
    // the two results are a lane's own operand and its partner's.
    const auto r = kMask == 32
        ? __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, lo),
                                           __builtin_bit_cast(uint32_t, hi), false, false)
        : __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, lo),
                                           __builtin_bit_cast(uint32_t, hi), false, false);
    return swap_sum<T>(r);
  } else {
    const bool up = (lane & kMask) != 0;
    const T send = up ? lo : hi;
    const T keep = up ? hi : lo;
    return keep + from_lane_xor<kMask>(send);
  }
}

// fold with fmaxf in place of the sum: a lane with the bit clear ends with
// max(lo, partner's lo), a lane with the bit set with max(hi, partner's hi).
template <int kMask>
__device__ __forceinline__ float fold_max(float lo, float hi, int lane) {
  if constexpr (kMask == 16 || kMask == 32) {
    const auto r = kMask == 32
        ? __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, lo),
                                           __builtin_bit_cast(uint32_t, hi), false, false)
        : __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, lo),
                                           __builtin_bit_cast(uint32_t, hi), false, false);
    const uint32_t first = r[0];
    const uint32_t second = r[1];
    return fmaxf(__builtin_bit_cast(float, first), __builtin_bit_cast(float, second));
  } else {
    const bool up = (lane & kMask) != 0;
    const float send = up ? lo : hi;
    const float keep = up ? hi : lo;
    return fmaxf(keep, from_lane_xor<kMask>(send));
  }
}

// max(x, x of lane ^ kMask), the same value in both lanes of a pair.
template <int kMask>
__device__ __forceinline__ float max_partner(float x) {
  if constexpr (kMask == 16 || kMask == 32) {
    const uint32_t bits = __builtin_bit_cast(uint32_t, x);
    const auto r = kMask == 32 ? __builtin_amdgcn_permlane32_swap(bits, bits, false, false)
                               : __builtin_amdgcn_permlane16_swap(bits, bits, false, false);
    const uint32_t first = r[0];
    const uint32_t second = r[1];
    return fmaxf(__builtin_bit_cast(float, first), __builtin_bit_cast(float, second));
  } else {
    return fmaxf(x, from_lane_xor<kMask>(x));
  }
}

// x + (x of lane ^ kMask), the same value in both lanes of a pair.
template <int kMask>
__device__ __forceinline__ float add_partner(float x) {
  if constexpr (kMask == 16 || kMask == 32) {
    const uint32_t bits = __builtin_bit_cast(uint32_t, x);
    const auto r = kMask == 32 ? __builtin_amdgcn_permlane32_swap(bits, bits, false, false)
                               : __builtin_amdgcn_permlane16_swap(bits, bits, false, false);
    return swap_sum<float>(r);
  } else {
    return x + from_lane_xor<kMask>(x);
  }
}

// 32- or 64-bit x of lane ^ kMask (kMask in 1, 2, 4, 8) by DPP; a 64-bit value
// moves as two dwords.
template <int kMask, typename T>
__device__ __forceinline__ T dpp_xor(T x) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit values");
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, from_lane_xor<kMask>(__builtin_bit_cast(int, x)));
  } else {
    const uint64_t bits = __builtin_bit_cast(uint64_t, x);
    const uint32_t low = from_lane_xor<kMask>(static_cast<int>(static_cast<uint32_t>(bits)));
    const uint32_t high = from_lane_xor<kMask>(static_cast<int>(static_cast<uint32_t>(bits >> 32)));
    return __builtin_bit_cast(T, (static_cast<uint64_t>(high) << 32) | low);
  }
}

// The two results of permlane{16,32}_swap(a, b) (kMask 16 or 32) for 32- or
// 64-bit values, a 64-bit value as two dwords: a lane whose kMask bit is clear
// gets its own a and its partner's a, a lane whose bit is set its partner's b
// and its own b (in some order).
template <int kMask, typename T>
__device__ __forceinline__ void swap_with_partner(T a, T b, T& first, T& second) {
  static_assert(kMask == 16 || kMask == 32, "permlane partner");
  const auto swap = [](uint32_t x, uint32_t y, uint32_t& r0, uint32_t& r1) {
    const auto r = kMask == 32 ? __builtin_amdgcn_permlane32_swap(x, y, false, false)
                               : __builtin_amdgcn_permlane16_swap(x, y, false, false);
    r0 = r[0];
    r1 = r[1];
  };
  if constexpr (sizeof(T) == 4) {
    uint32_t r0, r1;
    swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b), r0, r1);
    first = __builtin_bit_cast(T, r0);
    second = __builtin_bit_cast(T, r1);
  } else {
    static_assert(sizeof(T) == 8, "32- or 64-bit values");
    const uint64_t x = __builtin_bit_cast(uint64_t, a);
    const uint64_t y = __builtin_bit_cast(uint64_t, b);
    uint32_t l0, l1, h0, h1;
    swap(static_cast<uint32_t>(x), static_cast<uint32_t>(y), l0, l1);
    swap(static_cast<uint32_t>(x >> 32), static_cast<uint32_t>(y >> 32), h0, h1);
    first = __builtin_bit_cast(T, (static_cast<uint64_t>(h0) << 32) | l0);
    second = __builtin_bit_cast(T, (static_cast<uint64_t>(h1) << 32) | l1);
  }
}

// op(x, x of lane ^ kMask) for a commutative op, in both lanes of the pair.
template <int kMask, typename T, typename Op>
__device__ __forceinline__ T combine_with_partner(T x, Op op) {
  if constexpr (kMask == 16 || kMask == 32) {
    T first, second;
    swap_with_partner<kMask>(x, x, first, second);
    return op(first, second);
  } else {
    return op(x, dpp_xor<kMask>(x));
  }
}

// fold for any commutative op and 32- or 64-bit values: a lane with the kMask
// bit clear ends with op(lo, partner's lo), a lane with the bit set with
// op(hi, partner's hi).
template <int kMask, typename T, typename Op>
__device__ __forceinline__ T fold_with(T lo, T hi, int lane, Op op) {
  if constexpr (kMask == 16 || kMask == 32) {
    T first, second;
    swap_with_partner<kMask>(lo, hi, first, second);
    return op(first, second);
  } else {
    const bool up = (lane & kMask) != 0;
    const T send = up ? lo : hi;
    const T keep = up ? hi : lo;
    return op(keep, dpp_xor<kMask>(send));
  }
}

// Sum over the 64 lanes, every lane receiving the same value (butterfly over
// lane bits 32, 16, ..., 1).
__device__ __forceinline__ float wave_sum_valu(float x) {
  x = add_partner<32>(x);
  x = add_partner<16>(x);
  x = add_partner<8>(x);
  x = add_partner<4>(x);
  x = add_partner<2>(x);
  return add_partner<1>(x);
}

// Maximum over the wavefront, in every lane (fmaxf, so the order of the
// comparisons cannot change the result): row prefixes by row_shr 1, 2, 4, 8,
// rows merged by row_bcast 15 and 31, then lane 63 read back.
__device__ __forceinline__ float wave_max_valu(float x) {
  x = fmaxf(x, dpp<0x111>(x));
  x = fmaxf(x, dpp<0x112>(x));
  x = fmaxf(x, dpp<0x114>(x));
  x = fmaxf(x, dpp<0x118>(x));
  x = fmaxf(x, dpp<0x142, 0xA>(x));
  x = fmaxf(x, dpp<0x143, 0xC>(x));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}

}  // namespace gdn
