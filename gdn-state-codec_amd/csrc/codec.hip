// Quant-only int8 codec of GDN recurrent-state head tiles on gfx950.
//
// Numerics follow the reference's portable C++ quant stage bit for bit
// (native/src/gdn_state_codec_state_capsule.cpp:190-226 encode, :229-251
// decode):
//   s[k]     = sqrtf(max((float)(sum_v |r[k][v]| in double, in v order) / 128, 1e-8))
//   m[k][v]  = r[k][v] / s[k]
//   scale[v] = max_k |m[k][v]|
//   code     = scale == 0 ? 0 : lround(m / scale * 127)      (clamped to +-127)
//   dense    = ((s[k] * code) / 127) * scale[v] (+ sum_r ck[k][r] * cv[v][r])
//
// Encode: one workgroup of 256 threads (4 wavefronts) owns one 128x128 tile.
// Thread t holds rows 8j + t/32 (j = 0..15) and the four consecutive columns
// 4*(t%32)..+3 of each, so every load instruction of a wavefront reads 1 KiB of
// contiguous HBM and every code store writes 256 contiguous bytes.  Decode:
// one workgroup of 16 (fp32 output) or 8 (bf16 output) wavefronts owns a tile,
// with the same column quads and fewer rows per thread (DecodeShape).  "Row"
// and "column" are the tile's memory-major and minor axes; which of them is the
// key axis depends on the layout.
//
// The smoothing sum is order-dependent only when some partial sum needs more
// than 53 bits.  All terms are non-negative multiples of 2^(e_min-23) (e_min:
// exponent of the smallest non-zero |r| of the tile, at least -126), so when
// the largest key sum T satisfies T < 2^(e_min+29) every partial sum, in any
// order, is exact and equals the reference's sequential double sum.  The
// kernel sums with a lane tree, checks that bound per tile, and otherwise
// recomputes the 128 key sums serially in the reference's order.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "codec_math.h"
#include "lane_exchange.h"
#include "launch.h"
#include "stream_memory.h"

namespace gdn {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerThread = 16;

// Encode modes.
constexpr int kModeEncode = 0;         // smoothing + scales + codes
constexpr int kModeSmoothingOnly = 1;  // smoothing only
constexpr int kModeGivenSmoothing = 2; // scales + codes from caller's smoothing

// Work-item -> tile mapping.  Without slot ids item i is tile i on both sides.
// With slot ids, item i = (layer * batch + entry) * heads + head indexes the
// compact encoded side and the pool side is tile
// (layer * slots + slot_ids[entry]) * heads + head; entries whose slot id is
// negative (padding) or not below `slots` are skipped.
//
// Workgroups take items in the XCD-contiguous order (work_order.h) except the
// fp32 pool gather-encode, which keeps the dispatch order.  Measured A/B on one
// box (ms, identity -> XCD-contiguous): config-2 quantize 3.19 -> 3.11 and
// dequantize 3.69 -> 3.66; config-5 decode-scatter fp32 7.28 -> 6.26 and bf16
// 4.40 -> 3.90; bf16 gather-encode 4.50 -> 4.42; fp32 gather-encode 6.16 -> 6.43.
struct TileMap {
  const int32_t* slot_ids;
  uint32_t batch;
  uint32_t heads;
  uint32_t slots;
  bool dispatch_order;  // true: item = workgroup index
};

__device__ __forceinline__ uint64_t work_item(const TileMap& map) {
  return map.dispatch_order ? static_cast<uint64_t>(blockIdx.x)
                            : xcd_contiguous_item(blockIdx.x, gridDim.x);
}

__device__ __forceinline__ bool pool_entry(const TileMap& map, uint64_t item,
                                           uint64_t* entry) {
  if (map.slot_ids == nullptr) {
    *entry = item;
    return true;
  }
  const uint64_t head = item % map.heads;
  const uint64_t rest = item / map.heads;
  const uint64_t batch_entry = rest % map.batch;
  const uint64_t layer = rest / map.batch;
  const int32_t slot = map.slot_ids[batch_entry];
  if (slot < 0 || static_cast<uint32_t>(slot) >= map.slots) return false;
  *entry = (layer * map.slots + static_cast<uint64_t>(slot)) * map.heads + head;
  return true;
}

template <typename T>
__device__ __forceinline__ void load4(const T* p, float (&v)[4]);

template <>
__device__ __forceinline__ void load4<float>(const float* p, float (&v)[4]) {
  const float4 q = stream_load(reinterpret_cast<const float4*>(p));
  v[0] = q.x;
  v[1] = q.y;
  v[2] = q.z;
  v[3] = q.w;
}

__device__ __forceinline__ float load1(const float* p) { return *p; }
__device__ __forceinline__ float load1(const uint16_t* p) {
  return bf16_to_float(*p);
}

__device__ __forceinline__ void store4(float* p, const float (&v)[4]) {
  stream_store(reinterpret_cast<float4*>(p), make_float4(v[0], v[1], v[2], v[3]));
}

__device__ __forceinline__ void store4(uint16_t* p, const float (&v)[4]) {
  uint2 q;
  q.x = static_cast<uint32_t>(float_to_bf16(v[0])) |
        (static_cast<uint32_t>(float_to_bf16(v[1])) << 16);
  q.y = static_cast<uint32_t>(float_to_bf16(v[2])) |
        (static_cast<uint32_t>(float_to_bf16(v[3])) << 16);
  stream_store(reinterpret_cast<uint2*>(p), q);
}

// The thread's 16 rows x 4 columns of a tile (row j at offset + j * 8 * 128
// elements; the offset is unsigned so the loads can use a scalar base), widened
// to fp32, and the smallest non-zero magnitude among them (INFINITY if all are
// zero).
//
// fp32: on the bits, (b << 1) drops the sign and keeps the order of the
// magnitudes, and subtracting 1 turns a zero into the largest unsigned value,
// so one unsigned minimum (v_lshl_add + half a v_min3 per value) skips zeros.
__device__ __forceinline__ float load_rows(const float* tile, uint32_t offset,
                                           float (&x)[kRowsPerThread][4]) {
#pragma unroll
  for (int j = 0; j < kRowsPerThread; ++j) load4(tile + offset + j * 8 * kDim, x[j]);
  uint32_t min_key = 0xFFFFFFFFu;
#pragma unroll
  for (int j = 0; j < kRowsPerThread; ++j) {
#pragma unroll
    for (int i = 0; i < 4; i += 2) {
      const uint32_t a = (__float_as_uint(x[j][i]) << 1) - 1u;
      const uint32_t b = (__float_as_uint(x[j][i + 1]) << 1) - 1u;
      min_key = min(min_key, min(a, b));
    }
  }
  return min_key == 0xFFFFFFFFu ? INFINITY : __uint_as_float((min_key + 1u) >> 1);
}

// bf16: on each packed pair, h * 0xFFFE mod 2^16 is 2^16 - 2|h| for a
// non-zero h (the sign bit is shifted out) and 0 for +-0, so the largest key
// belongs to the smallest non-zero magnitude: one v_pk_mul_lo_u16 and one
// v_pk_max_u16 per two values.  The multiplier passes through an empty asm
// statement so that the compiler keeps the single multiply instead of
// rewriting it as a shift and a subtraction.
typedef uint16_t u16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float load_rows(const uint16_t* tile, uint32_t offset,
                                           float (&x)[kRowsPerThread][4]) {
  // 32-bit byte offsets from the workgroup's tile base: the loads use the
  // scalar-base addressing form instead of a 64-bit address per row.
  const char* base = reinterpret_cast<const char*>(tile);
  uint2 raw[kRowsPerThread];
#pragma unroll
  for (int j = 0; j < kRowsPerThread; ++j) {
    const uint32_t bytes = 2u * (offset + static_cast<uint32_t>(j * 8 * kDim));
    raw[j] = stream_load(reinterpret_cast<const uint2*>(base + bytes));
  }
  u16x2_t multiplier = {0xFFFEu, 0xFFFEu};
  asm("" : "+v"(multiplier));
  u16x2_t best = {0u, 0u};
#pragma unroll
  for (int j = 0; j < kRowsPerThread; ++j) {
    best = __builtin_elementwise_max(best, __builtin_bit_cast(u16x2_t, raw[j].x) * multiplier);
    best = __builtin_elementwise_max(best, __builtin_bit_cast(u16x2_t, raw[j].y) * multiplier);
    x[j][0] = __uint_as_float(raw[j].x << 16);
    x[j][1] = __uint_as_float(raw[j].x & 0xFFFF0000u);
    x[j][2] = __uint_as_float(raw[j].y << 16);
    x[j][3] = __uint_as_float(raw[j].y & 0xFFFF0000u);
  }
  const uint32_t key = max(static_cast<uint32_t>(best.x), static_cast<uint32_t>(best.y));
  return key == 0u ? INFINITY : __uint_as_float(((0x10000u - key) >> 1) << 16);
}

// Cross-lane exchanges.  Encodes of bf16 tiles (the slot pool's) exchange on
// the VALU (DPP and permlane swaps, lane_exchange.h); fp32 tiles go through
// ds_bpermute (__shfl_xor).  Measured on one box against the all-bpermute
// kernel (ms): bf16 pool gather-encode 4.54 -> 4.39 with VALU exchanges; with
// them, config-2 quantize went 3.14 -> 3.26 (its 64-bit key sums) and the fp32
// pool gather-encode 6.24 -> 6.30.  Both forms combine the same operands.
template <typename In>
constexpr bool kExchangeOnValu = sizeof(In) == 2;

// op(x, x of lane ^ kMask) in both lanes of the pair (op commutative).
template <bool kValu, int kMask, typename T, typename Op>
__device__ __forceinline__ T with_partner(T x, Op op) {
  if constexpr (kValu) {
    return combine_with_partner<kMask>(x, op);
  } else {
    return op(x, __shfl_xor(x, kMask));
  }
}

// op over the 64 lanes, in every lane (op commutative and associative).
template <bool kValu, typename T, typename Op>
__device__ __forceinline__ T over_wave(T x, Op op) {
  x = with_partner<kValu, 32>(x, op);
  x = with_partner<kValu, 16>(x, op);
  x = with_partner<kValu, 8>(x, op);
  x = with_partner<kValu, 4>(x, op);
  x = with_partner<kValu, 2>(x, op);
  return with_partner<kValu, 1>(x, op);
}

// One reduce-scatter step over lane pairs (lane, lane ^ kMask) for an array of
// 2H partials: the lane whose kMask bit is clear keeps the low half, its
// partner the high half, and each combines the partner's copy of the half it
// keeps.
template <bool kValu, int H, int kMask, typename T, typename Op>
__device__ __forceinline__ void reduce_scatter_step(T* p, int lane, Op op) {
#pragma unroll
  for (int i = 0; i < H; ++i) {
    if constexpr (kValu) {
      p[i] = fold_with<kMask>(p[i], p[i + H], lane, op);
    } else {
      const bool up = (lane & kMask) != 0;
      const T send = up ? p[i] : p[i + H];
      const T keep = up ? p[i + H] : p[i];
      p[i] = op(keep, __shfl_xor(send, kMask));
    }
  }
}

// Reduces 16 per-row partials over the 32 lanes of a half-wavefront.  Lane c
// (c = lane % 32) ends holding, in p[0], the total of row (c >> 1) & 15; lanes
// c and c ^ 1 hold the same value.
template <bool kValu, typename T, typename Op>
__device__ __forceinline__ void reduce_rows_over_half_wave(T (&p)[16], int c,
                                                           Op op) {
  reduce_scatter_step<kValu, 8, 16>(p, c, op);
  reduce_scatter_step<kValu, 4, 8>(p, c, op);
  reduce_scatter_step<kValu, 2, 4>(p, c, op);
  reduce_scatter_step<kValu, 1, 2>(p, c, op);
  p[0] = with_partner<kValu, 1>(p[0], op);
}

struct AddOp {
  template <typename T>
  __device__ __forceinline__ T operator()(T a, T b) const {
    return a + b;
  }
};
struct MaxOp {
  __device__ __forceinline__ float operator()(float a, float b) const {
    return fmaxf(a, b);
  }
  __device__ __forceinline__ double operator()(double a, double b) const {
    return fmax(a, b);
  }
};
struct MinOp {
  __device__ __forceinline__ float operator()(float a, float b) const {
    return fminf(a, b);
  }
};
// For operands known not to be NaN: equal to MaxOp there, and it needs no
// canonicalize of shuffled operands.
struct FiniteMaxOp {
  __device__ __forceinline__ float operator()(float a, float b) const {
    return __builtin_elementwise_maximum(a, b);
  }
};

// Exponent that bounds the granularity of a non-negative float: every float
// >= 2^e is a multiple of 2^(e-23), and every float is a multiple of 2^-149.
__device__ __forceinline__ int granularity_exponent(float value) {
  const int biased = static_cast<int>((__float_as_uint(value) >> 23) & 0xFFu);
  return biased == 0 ? -126 : biased - 127;
}

// The reference's sequential double sum of |r| along one key
// (state_capsule.cpp:193-197), read straight from the tile.
template <uint32_t kLayout, typename In>
__device__ double serial_key_sum(const In* tile, int key) {
  double sum = 0.0;
  if constexpr (kLayout == kKeyValue) {
    const In* row = tile + key * kDim;
    for (int value = 0; value < kDim; ++value) sum += fabsf(load1(row + value));
  } else {
    for (int value = 0; value < kDim; ++value) {
      sum += fabsf(load1(tile + value * kDim + key));
    }
  }
  return sum;
}

// code = lround(m / scale * 127), packed four per 32-bit store (one row's
// four consecutive columns).  kFast selects the reciprocal division.
template <uint32_t kLayout, bool kFast>
__device__ __forceinline__ void write_codes(const float (&x)[kRowsPerThread][4],
                                            const float* scale_shared,
                                            const float* scale_inverse,
                                            int group, int c4, int8_t* out) {
#pragma unroll
  for (int j = 0; j < kRowsPerThread; ++j) {
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int value = kLayout == kKeyValue ? 4 * c4 + i : 8 * j + group;
      const float scale = scale_shared[value];
      float q;
      if constexpr (kFast) {
        q = div_by_reciprocal(x[j][i], scale, scale_inverse[value]);
      } else {
        q = scale == 0.0f ? 0.0f : x[j][i] / scale;
      }
      const int code = round_half_away_small(q * kQuantizedMaximum);
      packed |= (static_cast<uint32_t>(code) & 0xFFu) << (8 * i);
    }
    stream_store(reinterpret_cast<uint32_t*>(out + (8 * j + group) * kDim + 4 * c4),
                 packed);
  }
}

// floor of four lifts, each as the low byte of one word: v_cvt_flr_i32_f32
// writes floor(u[0]) as an integer, and its SDWA form with dst_sel BYTE_k and
// UNUSED_PRESERVE writes the low byte of floor(u[k]) into byte k and keeps the
// other bytes.  For |u| < 2^31 the low byte of floor(u) is the two's-complement
// byte of the code.
__device__ __forceinline__ uint32_t pack_lifted_codes(const float (&u)[4]) {
  uint32_t packed;
  asm("v_cvt_flr_i32_f32 %0, %1" : "=v"(packed) : "v"(u[0]));
  asm("v_cvt_flr_i32_f32_sdwa %0, %1 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD"
      : "+v"(packed) : "v"(u[1]));
  asm("v_cvt_flr_i32_f32_sdwa %0, %1 dst_sel:BYTE_2 dst_unused:UNUSED_PRESERVE src0_sel:DWORD"
      : "+v"(packed) : "v"(u[2]));
  asm("v_cvt_flr_i32_f32_sdwa %0, %1 dst_sel:BYTE_3 dst_unused:UNUSED_PRESERVE src0_sel:DWORD"
      : "+v"(packed) : "v"(u[3]));
  return packed;
}

// The same codes from one fma, a fraction and a floor per value (code_lift,
// lift_fraction and lifted_code in codec_math.h), for finite m and scales in
// the reciprocal division's domain.  A row of four values whose smallest lift
// fraction is below the margin is recomputed on the exact path; that branch is
// divergent and taken by about 3% of a wavefront's 256-value rows.
template <uint32_t kLayout>
__device__ __forceinline__ void write_codes_lifted(const float (&x)[kRowsPerThread][4],
                                                   const float* scale_shared,
                                                   const float* scale_inverse,
                                                   const float* code_factor, int group,
                                                   int c4, int8_t* out) {
  float column_factor[4];
  if constexpr (kLayout == kKeyValue) {
#pragma unroll
    for (int i = 0; i < 4; ++i) column_factor[i] = code_factor[4 * c4 + i];
  }
#pragma unroll
  for (int j = 0; j < kRowsPerThread; ++j) {
    const float row_factor = kLayout == kKeyValue ? 0.0f : code_factor[8 * j + group];
    float lift[4];
    float fraction[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float factor = kLayout == kKeyValue ? column_factor[i] : row_factor;
      lift[i] = code_lift(x[j][i], factor);
      fraction[i] = lift_fraction(lift[i]);
    }
    uint32_t packed = pack_lifted_codes(lift);
    if (fminf(fminf(fraction[0], fraction[1]), fminf(fraction[2], fraction[3])) <
        kCodeLiftMargin) {
      packed = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int value = kLayout == kKeyValue ? 4 * c4 + i : 8 * j + group;
        const float q = div_by_reciprocal(x[j][i], scale_shared[value], scale_inverse[value]);
        const int code = round_half_away_small(q * kQuantizedMaximum);
        packed |= (static_cast<uint32_t>(code) & 0xFFu) << (8 * i);
      }
    }
    // An unsigned 32-bit offset from the workgroup's base lets the store use the
    // scalar-base addressing form instead of 64-bit vector address arithmetic.
    const uint32_t offset = static_cast<uint32_t>((8 * j + group) * kDim + 4 * c4);
    stream_store(reinterpret_cast<uint32_t*>(out + offset), packed);
  }
}

// m = r / s in place (kFast: the reciprocal division), with the thread's
// partial maxima of |m|: per row in the [value][key] layout (a row is one
// value), per column over the thread's 16 rows in [key][value] (mx[0..3]).
// On the fast path every m is finite, so the NaN-propagating maximum
// (v_maximum3_f32 with abs modifiers, no canonicalize) equals fmaxf there; the
// IEEE path keeps fmaxf, which like the reference's std::max skips NaNs.
template <bool kFast>
__device__ __forceinline__ float max_abs(float a, float b) {
  if constexpr (kFast) {
    return __builtin_elementwise_maximum(fabsf(a), fabsf(b));
  } else {
    return fmaxf(fabsf(a), fabsf(b));
  }
}

template <uint32_t kLayout, bool kFast, bool kValu>
__device__ __forceinline__ void smooth_and_max(float (&x)[kRowsPerThread][4],
                                               const float* s_shared,
                                               const float* s_inverse, int group,
                                               int c4, float (&mx)[kRowsPerThread]) {
#pragma unroll
  for (int j = 0; j < kRowsPerThread; ++j) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = kLayout == kKeyValue ? 8 * j + group : 4 * c4 + i;
      x[j][i] = kFast ? div_by_reciprocal(x[j][i], s_shared[key], s_inverse[key])
                      : x[j][i] / s_shared[key];
    }
  }
  if constexpr (kLayout == kKeyValue) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float m = 0.0f;
#pragma unroll
      for (int j = 0; j < kRowsPerThread; j += 2) {
        m = max_abs<kFast>(m, max_abs<kFast>(x[j][i], x[j + 1][i]));
      }
      mx[i] = m;
    }
  } else {
#pragma unroll
    for (int j = 0; j < kRowsPerThread; ++j) {
      mx[j] = max_abs<kFast>(max_abs<kFast>(x[j][0], x[j][1]), max_abs<kFast>(x[j][2], x[j][3]));
    }
    // Row maxima over the half-wavefront: mx[0] of lane c holds row (c >> 1) & 15.
    if constexpr (kFast) {
      reduce_rows_over_half_wave<kValu>(mx, c4, FiniteMaxOp{});
    } else {
      reduce_rows_over_half_wave<kValu>(mx, c4, MaxOp{});
    }
  }
}

// bf16 tiles in the [value][key] layout (the slot pool's) keep, on the fast
// domains, the product q0 = RN(r * RN(1/s)) in place of r: it is the first step
// of the reciprocal division of phase 2 and the operand of the code phase's
// lift (wide_code_lift, codec_math.h), which then needs one fma per value.  The
// exact path recovers r from q0 (bf16_input_from_product).  In [key][value] and
// for fp32 tiles phase 2 keeps m = r / s instead.
template <typename In, uint32_t kLayout>
constexpr bool kKeepsProduct = sizeof(In) == 2 && kLayout == kValueKey;

// Phase 2 on the fast domain for kKeepsProduct tiles: x becomes q0; the row
// maxima are those of m = RN(r / s), completed from q0 by the division's two
// remaining steps, with the same reductions as smooth_and_max.
template <bool kValu>
__device__ __forceinline__ void products_and_max(float (&x)[kRowsPerThread][4],
                                                 const float* s_shared,
                                                 const float* s_inverse, int c4,
                                                 float (&mx)[kRowsPerThread]) {
#pragma unroll
  for (int j = 0; j < kRowsPerThread; ++j) {
    float m[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = 4 * c4 + i;
      const float q0 = x[j][i] * s_inverse[key];
      m[i] = quotient_from_product(q0, x[j][i], s_shared[key], s_inverse[key]);
      x[j][i] = q0;
    }
    mx[j] = max_abs<true>(max_abs<true>(m[0], m[1]), max_abs<true>(m[2], m[3]));
  }
  reduce_rows_over_half_wave<kValu>(mx, c4, FiniteMaxOp{});
}

// m = RN(r / s) of a kept product q0, with r recovered from it.
__device__ __forceinline__ float quotient_of_kept_product(float q0, float s, float y) {
  return quotient_from_product(q0, bf16_input_from_product(q0, s), s, y);
}

// Phase 3 for kKeepsProduct tiles on the fast domains: codes from q0 by the
// direct lift; a row of four values whose smallest lift fraction is below the
// margin is recomputed exactly (m from q0, then m / scale by the reciprocal
// division and write_codes' rounding).
__device__ __forceinline__ void write_codes_from_products(
    const float (&x)[kRowsPerThread][4], const float* s_shared, const float* s_inverse,
    const float* scale_shared, const float* scale_inverse, const float* code_factor,
    int group, int c4, int8_t* out) {
#pragma unroll
  for (int j = 0; j < kRowsPerThread; ++j) {
    const int value = 8 * j + group;
    const float factor = code_factor[value];
    float lift[4];
    float fraction[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lift[i] = wide_code_lift(x[j][i], factor);
      fraction[i] = lift_fraction(lift[i]);
    }
    uint32_t packed = pack_lifted_codes(lift);
    if (fminf(fminf(fraction[0], fraction[1]), fminf(fraction[2], fraction[3])) <
        kWideLiftMargin) {
      packed = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = 4 * c4 + i;
        const float m = quotient_of_kept_product(x[j][i], s_shared[key], s_inverse[key]);
        const float q = div_by_reciprocal(m, scale_shared[value], scale_inverse[value]);
        const int code = round_half_away_small(q * kQuantizedMaximum);
        packed |= (static_cast<uint32_t>(code) & 0xFFu) << (8 * i);
      }
    }
    const uint32_t offset = static_cast<uint32_t>(value * kDim + 4 * c4);
    stream_store(reinterpret_cast<uint32_t*>(out + offset), packed);
  }
}

// kKeepsProduct tiles off the fast domains (tiles with a non-zero |r| below
// 2^-100 or a key sum above 2^46, or a scale outside [2^-90, 2^90]; rare) read
// their rows again from memory, one row at a time, and divide by IEEE
// division: these paths hold no tile in registers, which leaves the fast path
// its register budget (4 workgroups per CU).  Row j of the thread: values
// 4*c4 .. 4*c4+3 of value row 8*j + group.
__device__ __forceinline__ void reload_row(const uint16_t* tile, int group, int c4, int j,
                                           float (&r)[4]) {
  const uint32_t bytes = 2u * static_cast<uint32_t>((8 * j + group) * kDim + 4 * c4);
  const uint2 raw =
      stream_load(reinterpret_cast<const uint2*>(reinterpret_cast<const char*>(tile) + bytes));
  r[0] = __uint_as_float(raw.x << 16);
  r[1] = __uint_as_float(raw.x & 0xFFFF0000u);
  r[2] = __uint_as_float(raw.y << 16);
  r[3] = __uint_as_float(raw.y & 0xFFFF0000u);
}

// Phase 2 off the fast domain: the row maxima of |r / s|, as smooth_and_max's
// IEEE path forms them.
template <bool kValu>
__device__ __forceinline__ void reloaded_quotient_max(const uint16_t* tile,
                                                      const float* s_shared, int group,
                                                      int c4, float (&mx)[kRowsPerThread]) {
#pragma unroll
  for (int j = 0; j < kRowsPerThread; ++j) {
    float r[4];
    reload_row(tile, group, c4, j, r);
    float m[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) m[i] = r[i] / s_shared[4 * c4 + i];
    mx[j] = max_abs<false>(max_abs<false>(m[0], m[1]), max_abs<false>(m[2], m[3]));
    __builtin_amdgcn_sched_barrier(0);
  }
  reduce_rows_over_half_wave<kValu>(mx, c4, MaxOp{});
}

// Phase 3 off the fast domains: m = r / s, then write_codes' division by the
// scale (the reciprocal division when fast_scale) and rounding.  fast_scale is
// a run-time argument: two instantiations on the two sides of a branch would
// start with the same address arithmetic, which the compiler hoists above the
// branch and keeps live for all 16 rows.
__device__ __forceinline__ void write_codes_reloaded(const uint16_t* tile,
                                                     const float* s_shared,
                                                     const float* scale_shared,
                                                     const float* scale_inverse, int group,
                                                     int c4, int8_t* out, bool fast_scale) {
#pragma unroll
  for (int j = 0; j < kRowsPerThread; ++j) {
    const int value = 8 * j + group;
    float r[4];
    reload_row(tile, group, c4, j, r);
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float m = r[i] / s_shared[4 * c4 + i];
      const float scale = scale_shared[value];
      float q;
      if (fast_scale) {
        q = div_by_reciprocal(m, scale, scale_inverse[value]);
      } else {
        q = scale == 0.0f ? 0.0f : m / scale;
      }
      const int code = round_half_away_small(q * kQuantizedMaximum);
      packed |= (static_cast<uint32_t>(code) & 0xFFu) << (8 * i);
    }
    stream_store(reinterpret_cast<uint32_t*>(out + value * kDim + 4 * c4), packed);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The scale step of encode_kernel for kKeepsProduct tiles ([value][key]): the
// per-value scales from the row maxima of |m| (mx[0] of lanes with even c4,
// as reduce_rows_over_half_wave leaves them), written to LDS with their
// reciprocals and code factors, and to `scales`.  Returns, for the whole
// workgroup, whether every scale is 0 or in [2^-90, 2^90] (fast_scale).  The
// other tiles keep the step inline in encode_kernel: moved into a call, it
// changed the code generated for the fp32 kernels.
__device__ __forceinline__ bool finish_value_key_scales(const float (&mx)[kRowsPerThread],
                                                        float* scale_shared,
                                                        float* scale_inverse,
                                                        float* code_factor, float* scales,
                                                        int t, int group, int c4) {
  if ((c4 & 1) == 0) scale_shared[8 * ((c4 >> 1) & 15) + group] = mx[0];
  __syncthreads();
  bool scale_ok = true;
  if (t < kDim) {
    const float scale = scale_shared[t];
    scale_inverse[t] = scale == 0.0f ? 0.0f : 1.0f / scale;
    code_factor[t] = scale == 0.0f ? 0.0f : kQuantizedMaximum / scale;
    scales[t] = scale;
    scale_ok = scale == 0.0f || (scale >= 0x1p-90f && scale <= 0x1p90f);
  }
  return __syncthreads_and(scale_ok) != 0;
}

// kKeepsProduct tiles are compiled for 4 wavefronts per SIMD (at most 128
// VGPRs, 4 workgroups per CU); without the bound the allocator spreads the
// kept products over 136.
template <uint32_t kLayout, typename In, int kMode>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(kKeepsProduct<In, kLayout> ? 4 : 1))) void encode_kernel(
    const In* __restrict__ source, int8_t* __restrict__ codes,
    float* __restrict__ smoothing, float* __restrict__ scales,
    const float* __restrict__ given_smoothing, TileMap map) {
  __shared__ double key_sum[kDim];
  __shared__ double sum_part[4][kDim];
  __shared__ float max_part[4][kDim];
  __shared__ float s_shared[kDim];
  __shared__ float s_inverse[kDim];
  __shared__ float scale_shared[kDim];
  __shared__ float scale_inverse[kDim];
  __shared__ float code_factor[kDim];
  __shared__ float min_part[4];
  __shared__ double tmax_part[4];

  constexpr bool kValu = kExchangeOnValu<In>;
  const uint64_t item = work_item(map);
  uint64_t entry;
  if (!pool_entry(map, item, &entry)) return;  // uniform over the workgroup

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int group = t >> 5;  // row offset within each group of 8 rows
  const int c4 = t & 31;     // column quad
  const In* tile = source + entry * kTile;

  // min_abs is the smallest NON-ZERO |r| of the thread's values: zeros add
  // nothing to a key sum and divide exactly on both division paths, so they
  // must not force the slow paths (dequantized states hold many exact zeros,
  // one per code 0).
  // Tiles are held widened in x; phase 2 replaces r in place by m = r / s, or
  // by q0 = RN(r * RN(1/s)) for kKeepsProduct tiles on the fast domain.
  constexpr bool kKeepProduct = kKeepsProduct<In, kLayout>;
  float x[kRowsPerThread][4];
  float min_abs = load_rows(tile, static_cast<uint32_t>(group * kDim + 4 * c4), x);

  bool fast_divide = false;
  if constexpr (kMode != kModeGivenSmoothing) {
    // ---- smoothing: per-key double sums of |r| ------------------------------
    if constexpr (kLayout == kKeyValue) {
      double p[kRowsPerThread];
#pragma unroll
      for (int j = 0; j < kRowsPerThread; ++j) {
        p[j] = (static_cast<double>(fabsf(x[j][0])) + static_cast<double>(fabsf(x[j][1]))) +
               (static_cast<double>(fabsf(x[j][2])) + static_cast<double>(fabsf(x[j][3])));
      }
      reduce_rows_over_half_wave<kValu>(p, c4, AddOp{});
      if ((c4 & 1) == 0) key_sum[8 * ((c4 >> 1) & 15) + group] = p[0];
    } else {
      double p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        double acc = 0.0;
#pragma unroll
        for (int j = 0; j < kRowsPerThread; ++j) {
          acc += static_cast<double>(fabsf(x[j][i]));
        }
        p[i] = with_partner<kValu, 32>(acc, AddOp{});
      }
      if (lane < 32) {
#pragma unroll
        for (int i = 0; i < 4; ++i) sum_part[wave][4 * c4 + i] = p[i];
      }
      __syncthreads();
      if (t < kDim) {
        key_sum[t] = (sum_part[0][t] + sum_part[1][t]) +
                     (sum_part[2][t] + sum_part[3][t]);
      }
    }
    __syncthreads();

    // Tile-wide smallest non-zero |r| and largest key sum decide whether the
    // tree sums are exact: every non-zero |r| >= 2^e is a multiple of
    // 2^(e-23), so every partial sum below 2^(e+29) is a double without
    // rounding and any summation order gives the sequential sum.
    double tmax = t < kDim ? key_sum[t] : 0.0;
    min_abs = over_wave<kValu>(min_abs, MinOp{});
    tmax = over_wave<kValu>(tmax, MaxOp{});
    if (lane == 0) {
      min_part[wave] = min_abs;
      tmax_part[wave] = tmax;
    }
    __syncthreads();
    min_abs = fminf(fminf(min_part[0], min_part[1]),
                    fminf(min_part[2], min_part[3]));
    tmax = fmax(fmax(tmax_part[0], tmax_part[1]),
                fmax(tmax_part[2], tmax_part[3]));
    bool exact = tmax == 0.0;
    if (!exact && min_abs < INFINITY) {
      const int e = granularity_exponent(min_abs) + 29;
      const double bound =
          __longlong_as_double(static_cast<long long>(e + 1023) << 52);
      exact = tmax < bound;
    }
    if (!exact) {
      if (t < kDim) key_sum[t] = serial_key_sum<kLayout>(tile, t);
      __syncthreads();
    }
    if (t < kDim) {
      const float mean = static_cast<float>(key_sum[t] / 128.0);
      const float s = sqrtf(mean < kSmoothingFloor ? kSmoothingFloor : mean);
      s_shared[t] = s;
      s_inverse[t] = 1.0f / s;
      smoothing[item * kDim + t] = s;
    }
    if constexpr (kMode == kModeSmoothingOnly) return;
    // Markstein division is exact for every r / s when the smallest non-zero
    // |r| is at least 2^-100 and s <= 2^20 (key sums <= 2^46): |r/s| <= 128 s
    // stays far from overflow and >= 2^-120 stays normal.  r = +-0 gives +0
    // where IEEE gives +-0; m only feeds max |m| and lround(m / scale * 127),
    // neither of which sees the sign of a zero.
    fast_divide = min_abs >= 0x1p-100f && tmax <= 0x1p46;
  } else {
    if (t < kDim) {
      const float s = given_smoothing[item * kDim + t];
      s_shared[t] = s;
      s_inverse[t] = 1.0f / s;
    }
  }
  __syncthreads();

  // ---- m = r / s and the per-value scales max |m| over keys ----------------
  // The branch is uniform over the workgroup; each side is straight-line code.
  float mx[kRowsPerThread];
  if constexpr (kKeepProduct) {
    if (!fast_divide) {
      // Rare: the whole encode from the rows read again.  Returning here
      // leaves x one path from phase 2 to the codes; a merge of the two paths
      // would tie q0 to the registers of r and cost a copy per value.
      reloaded_quotient_max<kValu>(tile, s_shared, group, c4, mx);
      const bool fast_scale = finish_value_key_scales(mx, scale_shared, scale_inverse,
                                                      code_factor, scales + item * kDim, t,
                                                      group, c4);
      write_codes_reloaded(tile, s_shared, scale_shared, scale_inverse, group, c4,
                           codes + item * kTile, fast_scale);
      return;
    }
    products_and_max<kValu>(x, s_shared, s_inverse, c4, mx);
    int8_t* out = codes + item * kTile;
    if (finish_value_key_scales(mx, scale_shared, scale_inverse, code_factor,
                                scales + item * kDim, t, group, c4)) {
      write_codes_from_products(x, s_shared, s_inverse, scale_shared, scale_inverse,
                                code_factor, group, c4, out);
    } else {
      write_codes_reloaded(tile, s_shared, scale_shared, scale_inverse, group, c4, out, false);
    }
    return;
  } else if (fast_divide) {
    smooth_and_max<kLayout, true, kValu>(x, s_shared, s_inverse, group, c4, mx);
  } else {
    smooth_and_max<kLayout, false, kValu>(x, s_shared, s_inverse, group, c4, mx);
  }
  if constexpr (kLayout == kKeyValue) {
#pragma unroll
    for (int i = 0; i < 4; ++i) mx[i] = with_partner<kValu, 32>(mx[i], MaxOp{});
    if (lane < 32) {
#pragma unroll
      for (int i = 0; i < 4; ++i) max_part[wave][4 * c4 + i] = mx[i];
    }
    __syncthreads();
    if (t < kDim) {
      scale_shared[t] = fmaxf(fmaxf(max_part[0][t], max_part[1][t]),
                              fmaxf(max_part[2][t], max_part[3][t]));
    }
  } else {
    if ((c4 & 1) == 0) scale_shared[8 * ((c4 >> 1) & 15) + group] = mx[0];
  }
  __syncthreads();
  bool scale_ok = true;
  if (t < kDim) {
    const float scale = scale_shared[t];
    scale_inverse[t] = scale == 0.0f ? 0.0f : 1.0f / scale;
    code_factor[t] = scale == 0.0f ? 0.0f : kQuantizedMaximum / scale;
    scales[item * kDim + t] = scale;
    scale_ok = scale == 0.0f || (scale >= 0x1p-90f && scale <= 0x1p90f);
  }
  // Markstein for m / scale: exact when 2^-90 <= scale <= 2^90 and |m| is
  // large enough for the code to be non-zero; smaller |m| give |m/scale*127|
  // < 0.5 on both paths.  scale == 0 gives y = 0 and code 0 like the reference.
  const bool fast_scale = __syncthreads_and(scale_ok) != 0;

  // ---- codes ---------------------------------------------------------------
  int8_t* out = codes + item * kTile;
  if (fast_scale && fast_divide) {  // m finite: every r / s took the fast division
    write_codes_lifted<kLayout>(x, scale_shared, scale_inverse, code_factor, group, c4, out);
  } else if (fast_scale) {
    write_codes<kLayout, true>(x, scale_shared, scale_inverse, group, c4, out);
  } else {
    write_codes<kLayout, false>(x, scale_shared, scale_inverse, group, c4, out);
  }
}

// Decode thread layout: kWaves wavefronts per tile, interleaved.  A lane
// handles rows 2 kWaves j + t / 32 of the tile, j = 0 .. 64 / kWaves - 1, and
// the four columns 4*(t%32)..+3, so every store instruction writes two whole
// rows of contiguous HBM and the wavefronts advance through the tile together.
// (Each wavefront writing its own contiguous band of rows measured slower; see
// launch_decode.)
template <int kWaves>
struct DecodeShape {
  static constexpr int kThreadCount = 64 * kWaves;
  static constexpr int kRows = 64 / kWaves;  // rows per thread
  static constexpr int kRowStep = 2 * kWaves;
  __device__ static int first_row(int t) { return t >> 5; }
};

// dense = ((s[k] * code) / 127) * scale[v] (+ sum_r ck[k][r] * cv[v][r]) for
// the thread's rows x 4 columns.  kFast selects the two-operation division.
template <uint32_t kLayout, bool kFast, bool kCompensated, typename Shape, typename Out>
__device__ __forceinline__ void decode_rows(const int8_t* tile,
                                            const float* s_shared,
                                            const float* scale_shared,
                                            const float* ck_shared,
                                            const float* cv_shared, int first,
                                            int c4, Out* out) {
  constexpr int kRank = 4;
  // The IEEE path (s outside the two-part division's domain) is rare; it
  // stays rolled so that it does not set the kernel's register count.
  constexpr int kUnroll = kFast ? (kCompensated ? 2 : 4) : 1;
#pragma unroll kUnroll
  for (int j = 0; j < Shape::kRows; ++j) {
    const int row = first + Shape::kRowStep * j;
    const uint32_t packed =
        stream_load(reinterpret_cast<const uint32_t*>(tile + row * kDim + 4 * c4));
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = kLayout == kKeyValue ? row : 4 * c4 + i;
      const int value = kLayout == kKeyValue ? 4 * c4 + i : row;
      const float code = static_cast<float>(
          static_cast<int8_t>(static_cast<uint8_t>(packed >> (8 * i))));
      const float a = s_shared[key] * code;
      float d;
      if constexpr (kFast) {
        d = div_by_127(a);
      } else {
        d = a / kQuantizedMaximum;
      }
      float value_out = d * scale_shared[value];
      if constexpr (kCompensated) {
#pragma unroll
        for (int r = 0; r < kRank; ++r) {
          value_out += ck_shared[key * kRank + r] * cv_shared[value * kRank + r];
        }
      }
      v[i] = value_out;
    }
    store4(out + row * kDim + 4 * c4, v);
  }
}

template <uint32_t kLayout, typename Out, bool kCompensated, typename Shape>
__global__ __launch_bounds__(Shape::kThreadCount) void decode_kernel(
    const int8_t* __restrict__ codes, const float* __restrict__ smoothing,
    const float* __restrict__ scales,
    const float* __restrict__ compensator_keys,
    const float* __restrict__ compensator_values, Out* __restrict__ dense,
    TileMap map) {
  constexpr int kRank = 4;
  __shared__ float s_shared[kDim];
  __shared__ float scale_shared[kDim];
  __shared__ float ck_shared[kCompensated ? kDim * kRank : 1];
  __shared__ float cv_shared[kCompensated ? kDim * kRank : 1];

  const uint64_t item = work_item(map);
  uint64_t entry;
  if (!pool_entry(map, item, &entry)) return;  // uniform over the workgroup

  const int t = threadIdx.x;
  const int c4 = t & 31;

  bool ok = true;
  if (t < kDim) {
    const float s = smoothing[item * kDim + t];
    s_shared[t] = s;
    // The two-part division by 127 (div_by_127) is exact for s * code when s
    // is in [2^-90, 2^100]: the product is +-0 or between 2^-90 and 2^107 in
    // magnitude, so its low part a * 2^-35 stays a normal float.
    ok = s >= 0x1p-90f && s <= 0x1p100f;
  } else if (t < 2 * kDim) {
    scale_shared[t - kDim] = scales[item * kDim + (t - kDim)];
  }
  if constexpr (kCompensated) {
    for (int i = t; i < kDim * kRank; i += Shape::kThreadCount) {
      ck_shared[i] = compensator_keys[item * kDim * kRank + i];
      cv_shared[i] = compensator_values[item * kDim * kRank + i];
    }
  }
  const bool fast_divide = __syncthreads_and(ok) != 0;

  const int8_t* tile = codes + item * kTile;
  Out* out = dense + entry * kTile;
  const int first = Shape::first_row(t);
  if (fast_divide) {
    decode_rows<kLayout, true, kCompensated, Shape>(tile, s_shared, scale_shared, ck_shared,
                                                    cv_shared, first, c4, out);
  } else {
    decode_rows<kLayout, false, kCompensated, Shape>(tile, s_shared, scale_shared, ck_shared,
                                                     cv_shared, first, c4, out);
  }
}

// --------------------------------------------------------------- dispatch

template <int kMode>
int32_t launch_encode(void* stream, const void* source, uint32_t dtype,
                      int8_t* codes, float* smoothing, float* scales,
                      const float* given_smoothing, uint64_t items,
                      uint32_t layout, TileMap map) {
  const dim3 grid(static_cast<uint32_t>(items));
  const dim3 block(kThreads);
  if (dtype == kDtypeF32) {
    const float* src = static_cast<const float*>(source);
    return layout == kKeyValue
               ? launch(encode_kernel<kKeyValue, float, kMode>, grid, block,
                        stream, src, codes, smoothing, scales, given_smoothing,
                        map)
               : launch(encode_kernel<kValueKey, float, kMode>, grid, block,
                        stream, src, codes, smoothing, scales, given_smoothing,
                        map);
  }
  const uint16_t* src = static_cast<const uint16_t*>(source);
  return layout == kKeyValue
             ? launch(encode_kernel<kKeyValue, uint16_t, kMode>, grid, block,
                      stream, src, codes, smoothing, scales, given_smoothing,
                      map)
             : launch(encode_kernel<kValueKey, uint16_t, kMode>, grid, block,
                      stream, src, codes, smoothing, scales, given_smoothing,
                      map);
}

template <bool kCompensated, typename Shape, typename Out>
int32_t launch_decode_shaped(void* stream, const int8_t* codes, const float* smoothing,
                             const float* scales, const float* compensator_keys,
                             const float* compensator_values, Out* dense, uint64_t items,
                             uint32_t layout, TileMap map) {
  const dim3 grid(static_cast<uint32_t>(items));
  const dim3 block(Shape::kThreadCount);
  return layout == kKeyValue
             ? launch(decode_kernel<kKeyValue, Out, kCompensated, Shape>, grid, block, stream,
                      codes, smoothing, scales, compensator_keys, compensator_values, dense, map)
             : launch(decode_kernel<kValueKey, Out, kCompensated, Shape>, grid, block, stream,
                      codes, smoothing, scales, compensator_keys, compensator_values, dense, map);
}

// Thread layout per output type, from A/B runs on one box (ms, bit-identical;
// wavefronts per tile, interleaved or in bands):
//   config-2 dequantize (fp32, [key][value]): 4 interleaved 3.647, 4 bands
//     3.543, 8 interleaved 3.584, 8 bands 3.515, 16 bands 3.536,
//     16 interleaved 3.370;
//   config-5 fp32 decode-scatter ([value][key] into slots): 4 interleaved
//     6.234, 8 interleaved 5.928, 8 bands 6.512, 16 bands 5.683,
//     16 interleaved 5.690;
//   config-5 bf16 decode-scatter: 4 interleaved 3.627, 8 interleaved 3.562,
//     8 bands 4.523, 16 bands 3.913, 16 interleaved 3.883.
// fp32 tiles take 16 interleaved wavefronts (1024 threads, 4 rows per thread),
// bf16 tiles 8 (512 threads, 8 rows per thread).
template <bool kCompensated>
int32_t launch_decode(void* stream, const int8_t* codes, const float* smoothing,
                      const float* scales, const float* compensator_keys,
                      const float* compensator_values, void* dense,
                      uint32_t dtype, uint64_t items, uint32_t layout,
                      TileMap map) {
  return dtype == kDtypeF32
             ? launch_decode_shaped<kCompensated, DecodeShape<16>>(
                   stream, codes, smoothing, scales, compensator_keys, compensator_values,
                   static_cast<float*>(dense), items, layout, map)
             : launch_decode_shaped<kCompensated, DecodeShape<8>>(
                   stream, codes, smoothing, scales, compensator_keys, compensator_values,
                   static_cast<uint16_t*>(dense), items, layout, map);
}

constexpr TileMap kIdentityMap{nullptr, 0, 0, 0, false};

bool valid_layout(uint32_t layout) {
  return layout == kKeyValue || layout == kValueKey;
}

// Reference admission for the provider launchers:
// gdn_state_codec_quantize.cpp:207-211, gdn_state_codec_smoothing.cpp:144-147.
bool provider_states_ok(uint32_t states) { return states >= 1 && states <= 64; }

}  // namespace
}  // namespace gdn

using gdn::kStatusInvalidArgument;

// ------------------------------------------------------ reference v1/v2 ABI

extern "C" int32_t statecentric_gdn_state_codec_smoothing_launch_v1(
    void* stream, const float* residual, float* smoothing) {
  if (residual == nullptr || smoothing == nullptr || !gdn::aligned16(residual, smoothing)) {
    return kStatusInvalidArgument;
  }
  return gdn::launch_encode<gdn::kModeSmoothingOnly>(
      stream, residual, gdn::kDtypeF32, nullptr, smoothing, nullptr, nullptr, 1,
      gdn::kKeyValue, gdn::kIdentityMap);
}

extern "C" int32_t statecentric_gdn_state_codec_quantize_launch_v1(
    void* stream, const float* residual, const float* smoothing,
    int8_t* quantized, float* value_scales) {
  if (residual == nullptr || smoothing == nullptr || quantized == nullptr ||
      value_scales == nullptr || !gdn::aligned16(residual, smoothing, quantized, value_scales)) {
    return kStatusInvalidArgument;
  }
  return gdn::launch_encode<gdn::kModeGivenSmoothing>(
      stream, residual, gdn::kDtypeF32, quantized, nullptr, value_scales,
      smoothing, 1, gdn::kKeyValue, gdn::kIdentityMap);
}

extern "C" int32_t statecentric_gdn_state_codec_dequantize_launch_v1(
    void* stream, const int8_t* quantized, const float* smoothing,
    const float* value_scales, const float* compensator_keys,
    const float* compensator_values, float* dense) {
  if (quantized == nullptr || smoothing == nullptr || value_scales == nullptr ||
      compensator_keys == nullptr || compensator_values == nullptr ||
      dense == nullptr ||
      !gdn::aligned16(quantized, smoothing, value_scales, compensator_keys,
                      compensator_values, dense)) {
    return kStatusInvalidArgument;
  }
  return gdn::launch_decode<true>(stream, quantized, smoothing, value_scales,
                                  compensator_keys, compensator_values, dense,
                                  gdn::kDtypeF32, 1, gdn::kKeyValue,
                                  gdn::kIdentityMap);
}

extern "C" int32_t statecentric_gdn_state_codec_provider_smoothing_launch_v2(
    void* stream, const float* provider_state, float* smoothing,
    uint32_t states) {
  if (provider_state == nullptr || smoothing == nullptr ||
      !gdn::provider_states_ok(states) || !gdn::aligned16(provider_state, smoothing)) {
    return kStatusInvalidArgument;
  }
  return gdn::launch_encode<gdn::kModeSmoothingOnly>(
      stream, provider_state, gdn::kDtypeF32, nullptr, smoothing, nullptr,
      nullptr, states, gdn::kValueKey, gdn::kIdentityMap);
}

extern "C" int32_t statecentric_gdn_state_codec_provider_quantize_launch_v2(
    void* stream, const float* provider_state, const float* smoothing,
    int8_t* quantized, float* value_scales, uint32_t states) {
  if (provider_state == nullptr || smoothing == nullptr ||
      quantized == nullptr || value_scales == nullptr ||
      !gdn::provider_states_ok(states) ||
      !gdn::aligned16(provider_state, smoothing, quantized, value_scales)) {
    return kStatusInvalidArgument;
  }
  return gdn::launch_encode<gdn::kModeGivenSmoothing>(
      stream, provider_state, gdn::kDtypeF32, quantized, nullptr, value_scales,
      smoothing, states, gdn::kValueKey, gdn::kIdentityMap);
}

// ------------------------------------------------------------ batched v4 ABI

extern "C" int32_t statecentric_gdn_state_codec_encode_launch_v4(
    void* stream, const float* state, int8_t* quantized, float* smoothing,
    float* value_scales, uint64_t heads, uint32_t layout) {
  if (state == nullptr || quantized == nullptr || smoothing == nullptr ||
      value_scales == nullptr || heads == 0 || heads > gdn::kMaxGrid ||
      !gdn::valid_layout(layout) ||
      !gdn::aligned16(state, quantized, smoothing, value_scales)) {
    return kStatusInvalidArgument;
  }
  return gdn::launch_encode<gdn::kModeEncode>(
      stream, state, gdn::kDtypeF32, quantized, smoothing, value_scales,
      nullptr, heads, layout, gdn::kIdentityMap);
}

extern "C" int32_t statecentric_gdn_state_codec_decode_launch_v4(
    void* stream, const int8_t* quantized, const float* smoothing,
    const float* value_scales, const float* compensator_keys,
    const float* compensator_values, float* state, uint64_t heads,
    uint32_t layout) {
  if (quantized == nullptr || smoothing == nullptr || value_scales == nullptr ||
      state == nullptr || heads == 0 || heads > gdn::kMaxGrid ||
      !gdn::valid_layout(layout) ||
      (compensator_keys == nullptr) != (compensator_values == nullptr) ||
      !gdn::aligned16(quantized, smoothing, value_scales, compensator_keys,
                      compensator_values, state)) {
    return kStatusInvalidArgument;
  }
  if (compensator_keys != nullptr) {
    return gdn::launch_decode<true>(stream, quantized, smoothing, value_scales,
                                    compensator_keys, compensator_values, state,
                                    gdn::kDtypeF32, heads, layout,
                                    gdn::kIdentityMap);
  }
  return gdn::launch_decode<false>(stream, quantized, smoothing, value_scales,
                                   nullptr, nullptr, state, gdn::kDtypeF32,
                                   heads, layout, gdn::kIdentityMap);
}

namespace {
bool pool_args_ok(const int32_t* slot_ids, uint32_t batch, uint32_t layers,
                  uint32_t slots, uint32_t heads, uint32_t layout,
                  uint32_t dtype) {
  if (slot_ids == nullptr || batch == 0 || layers == 0 || slots == 0 ||
      heads == 0 || !gdn::valid_layout(layout) ||
      (dtype != gdn::kDtypeF32 && dtype != gdn::kDtypeBF16)) {
    return false;
  }
  const uint64_t items = static_cast<uint64_t>(layers) * batch * heads;
  return items <= gdn::kMaxGrid;
}
}  // namespace

extern "C" int32_t statecentric_gdn_state_codec_pool_encode_launch_v4(
    void* stream, const void* pool, uint32_t pool_dtype,
    const int32_t* slot_ids, uint32_t batch, uint32_t layers, uint32_t slots,
    uint32_t heads, uint32_t layout, int8_t* quantized, float* smoothing,
    float* value_scales) {
  if (pool == nullptr || quantized == nullptr || smoothing == nullptr ||
      value_scales == nullptr ||
      !pool_args_ok(slot_ids, batch, layers, slots, heads, layout, pool_dtype) ||
      !gdn::aligned16(pool, slot_ids, quantized, smoothing, value_scales)) {
    return kStatusInvalidArgument;
  }
  const gdn::TileMap map{slot_ids, batch, heads, slots, pool_dtype == gdn::kDtypeF32};
  return gdn::launch_encode<gdn::kModeEncode>(
      stream, pool, pool_dtype, quantized, smoothing, value_scales, nullptr,
      static_cast<uint64_t>(layers) * batch * heads, layout, map);
}

extern "C" int32_t statecentric_gdn_state_codec_pool_decode_launch_v4(
    void* stream, const int8_t* quantized, const float* smoothing,
    const float* value_scales, const int32_t* slot_ids, uint32_t batch,
    uint32_t layers, uint32_t slots, uint32_t heads, uint32_t layout,
    void* pool, uint32_t pool_dtype) {
  if (pool == nullptr || quantized == nullptr || smoothing == nullptr ||
      value_scales == nullptr ||
      !pool_args_ok(slot_ids, batch, layers, slots, heads, layout, pool_dtype) ||
      !gdn::aligned16(pool, slot_ids, quantized, smoothing, value_scales)) {
    return kStatusInvalidArgument;
  }
  const gdn::TileMap map{slot_ids, batch, heads, slots, false};
  return gdn::launch_decode<false>(
      stream, quantized, smoothing, value_scales, nullptr, nullptr, pool,
      pool_dtype, static_cast<uint64_t>(layers) * batch * heads, layout, map);
}
