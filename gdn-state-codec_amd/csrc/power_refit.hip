// Rank-4 window-boundary refit (window_boundary_launch_v1 with
// power_iterations in 1..32; native/ascendc/gdn_state_codec/kernel/
// gdn_state_codec_window_boundary.cpp:253-366).
//
// For a state whose 16-record window is full, the window's residual operator
//   R = boundary * S + old compensators * S + sum_j key_j corr_j^T * suffix_j
// is fitted with four rank-one terms by deflated power iteration (the start
// vector of rank r is ((r+1)(c+3)) mod 17 - 8, normalized with a 20-step
// Newton square root), stored as fp16 compensators; R minus the fit is then
// re-encoded with fresh smoothing sqrt(mean |row|), absmax scales and
// round-half-away codes, and the window is cleared.
//
// Every dot product of the reference is a sequential fp32 sum; this kernel
// keeps each one on a single thread in the reference's order (outputs of the
// operator in parallel, one row or column per thread; projections and norms
// on single threads, broadcast through LDS), so the result is bit-identical to
// the CPU statement of the reference kernel.  One 128-thread workgroup per
// state, operands staged in LDS: the codes at a 132-byte row stride so both
// the row walk and the column walk are free of bank conflicts, compensators
// and records as fp16 bits (31,408 bytes: 25 of the CU's 1,280-byte LDS
// granules, five workgroups per CU).  The fitted residual is evaluated once
// per cell, one key row per thread held in registers for the smoothing, scale
// and code passes, and written once to the workspace.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>
#include <type_traits>

#include "pipelined_sum.h"
#include "codec_math.h"
#include "gdn_state_codec_window.h"
#include "lane_exchange.h"
#include "launch.h"
#include "window_common.h"

namespace gdn {
namespace {

constexpr int kThreads = 128;
constexpr int kCodeStride = kDim + 4;
constexpr float kBoundaryFloor = 1.0e-8f;

// f(std::integral_constant<int, c>) for c = 0 .. kDim - 1, expanded at compile
// time: a body that indexes a register array by c keeps the array in VGPRs,
// where a loop the compiler declines to unroll fully would move it to scratch.
template <int kColumn = 0, typename F>
__device__ __forceinline__ void each_column(F&& f) {
  if constexpr (kColumn < kDim) {
    f(std::integral_constant<int, kColumn>{});
    each_column<kColumn + 1>(f);
  }
}

struct PowerArgs {
  const int8_t* residual;
  const float* smoothing;
  const float* scales;
  const uint16_t* comp_keys;
  const uint16_t* comp_values;
  float* record_decay;
  uint16_t* record_keys;
  uint16_t* record_corrections;
  uint32_t* positions;
  int8_t* next_residual;
  float* next_smoothing;
  float* next_scales;
  uint16_t* next_comp_keys;
  uint16_t* next_comp_values;
  float* workspace;
  uint32_t power_iterations;
};

// Compensators and records are fp16 values (the fitted ranks are rounded to
// fp16 when formed), so they are kept as fp16 bits and widened exactly when
// read: 31,408 bytes, five workgroups per CU.
struct PowerShared {
  int8_t code[kDim * kCodeStride];  // [value column][key row]
  alignas(8) uint16_t ck[kDim * kRank];
  alignas(8) uint16_t cv[kDim * kRank];
  alignas(8) uint16_t nk[kDim * kRank];
  alignas(8) uint16_t nv[kDim * kRank];
  // Records as [dimension][record]: a dimension's 16 records are 32
  // contiguous bytes, so the record projections (lane j walks record j)
  // read consecutive words and a cell reads its 16 records as two 16-byte
  // words.
  alignas(16) uint16_t rk[kDim * kWindow];
  alignas(16) uint16_t rc[kDim * kWindow];
  float smoothing[kDim], scales[kDim];
  union {
    float left[kDim];            // power iteration
    float next_smoothing[kDim];  // re-encoding, after the iteration
  };
  float right[kDim];
  float old_projection[kRank], fitted_projection[kRank], record_projection[kWindow];
  float record_suffix[kWindow];
  float scalar;  // norm inverse / singular value broadcast
  int flag;
};
static_assert(workgroups_by_lds(sizeof(PowerShared)) >= 5, "five workgroups per CU");

// window_boundary.cpp:17-23.
__device__ __forceinline__ float newton_sqrt(float value) {
  float estimate = value > 1.0f ? value : 1.0f;
#pragma unroll 1
  for (int i = 0; i < 20; ++i) estimate = 0.5f * (estimate + value / estimate);
  return estimate;
}

__device__ __forceinline__ float h2f(uint16_t h) { return half_bits_to_float(h); }

// code / 127 by the two-part division (div_by_127, exact for every integer in
// [-128, 127]): two VALU instructions, where a table of the 256 quotients
// would cost a second LDS read whose address depends on the first.
__device__ __forceinline__ float code_value_arith(int8_t code) {
  return div_by_127(static_cast<float>(code));
}

// Normalize (:25-37) of v; returns whether the norm was usable.  The squared
// norm is one sequential sum on thread 0.
__device__ bool normalize(PowerShared& sh, float* v, int t) {
  if (t == 0) {
    float squared = 0.0f;
    struct Group {
      float x[16];
    };
    pipelined<kDim / 16, Group>(
        [&](auto g, Group& r) { unrolled<16>([&](auto i) { r.x[i] = v[16 * decltype(g)::value + i]; }); },
        [&](auto, const Group& r) { unrolled<16>([&](auto i) { squared += r.x[i] * r.x[i]; }); });
    sh.flag = squared <= 1.0e-20f ? 0 : 1;
    sh.scalar = sh.flag ? 1.0f / newton_sqrt(squared) : 0.0f;
  }
  __syncthreads();
  const bool ok = sh.flag != 0;
  if (ok) v[t] *= sh.scalar;
  __syncthreads();
  return ok;
}

// Projections of an apply (old compensator side, records, fitted ranks): one
// sequential sum per thread in the reference's loop order.  Wavefront 0 runs
// the compensator sides (lanes 0..3 the old ranks, lanes 4..7 the fitted
// ones: the same loop over a per-lane basis, so no branch divergence) while
// wavefront 1 runs the 16 record sides (its lanes 0..15).
__device__ void projections(PowerShared& sh, const float* vector, const uint16_t* old_basis,
                            const uint16_t* record_basis, const uint16_t* fitted_basis,
                            int fitted, int t) {
  if (t < 2 * kRank) {
    const int r = t & (kRank - 1);
    const bool is_fitted = t >= kRank;
    if (!is_fitted || r < fitted) {
      const uint16_t* basis = is_fitted ? fitted_basis : old_basis;
      float acc = 0.0f;
      for (int i = 0; i < kDim; ++i) acc += h2f(basis[i * kRank + r]) * vector[i];
      if (is_fitted) {
        sh.fitted_projection[r] = acc;
      } else {
        sh.old_projection[r] = acc;
      }
    }
  } else if (t >= 64 && t < 64 + kWindow) {
    const int j = t - 64;
    float acc = 0.0f;
    for (int i = 0; i < kDim; ++i) acc += h2f(record_basis[i * kWindow + j]) * vector[i];
    sh.record_projection[j] = acc;
  }
  __syncthreads();
}

// ApplyRight (:113-166): output[row] = R^T-free form R * vector over columns.
__device__ void apply_right(PowerShared& sh, const float* vector, float* output, float bs,
                            int fitted, int t) {
  projections(sh, vector, sh.cv, sh.rc, sh.nv, fitted, t);
  const int row = t;
  float value = 0.0f;
  const float s = sh.smoothing[row];
  for (int column = 0; column < kDim; ++column) {
    value += code_value_arith(sh.code[column * kCodeStride + row]) * s * sh.scales[column] *
             vector[column] * bs;
  }
  for (int r = 0; r < kRank; ++r) value += h2f(sh.ck[row * kRank + r]) * sh.old_projection[r] * bs;
  for (int j = 0; j < kWindow; ++j) {
    value += h2f(sh.rk[row * kWindow + j]) * sh.record_projection[j] * sh.record_suffix[j];
  }
  for (int r = 0; r < fitted; ++r) value -= h2f(sh.nk[row * kRank + r]) * sh.fitted_projection[r];
  __syncthreads();  // every thread has read `vector` before it may be overwritten
  output[row] = value;
  __syncthreads();
}

// ApplyTranspose (:168-221): output[column] = R^T * vector over rows.
__device__ void apply_transpose(PowerShared& sh, const float* vector, float* output, float bs,
                                int fitted, int t) {
  projections(sh, vector, sh.ck, sh.rk, sh.nk, fitted, t);
  const int column = t;
  float value = 0.0f;
  const float scale = sh.scales[column];
  const int8_t* code = sh.code + column * kCodeStride;
  for (int row = 0; row < kDim; ++row) {
    value += code_value_arith(code[row]) * sh.smoothing[row] * scale * vector[row] * bs;
  }
  for (int r = 0; r < kRank; ++r) value += h2f(sh.cv[column * kRank + r]) * sh.old_projection[r] * bs;
  for (int j = 0; j < kWindow; ++j) {
    value += h2f(sh.rc[column * kWindow + j]) * sh.record_projection[j] * sh.record_suffix[j];
  }
  for (int r = 0; r < fitted; ++r) value -= h2f(sh.nv[column * kRank + r]) * sh.fitted_projection[r];
  __syncthreads();
  output[column] = value;
  __syncthreads();
}

// The re-encode of R minus the fit, for the 128 threads of a workgroup whose
// LDS holds the state (codes [value column][key row] at kCodeStride, the old
// and fitted compensators ck / cv / nk / nv [dim][rank], the records rk / rc
// [dim][record], smoothing, scales and record suffixes):
// thread t owns key row t, whose 128 fitted cells stay in registers through
// the smoothing, scale and code passes.  Writes the fitted residual to
// workspace [key row][value column], next_smoothing[key], next_scales[value],
// and hands every code of row t to sink(integral_constant column, code).  Each
// cell is the reference's ResidualCell (window_boundary.cpp:223-251;
// encoded_requantize.cpp:72-100 is the same expression), evaluated in its
// order.  The column loops are unrolled at compile time (each_column) so that
// cell[] is only ever indexed by constants and lives in VGPRs.  Uses sh.left
// and sh.right as scratch for the column maxima.
template <typename Sink>
__device__ __forceinline__ void reencode_rows(PowerShared& sh, float bs, int t, float* workspace,
                                              float* next_smoothing, float* next_scales,
                                              Sink&& sink) {
  const int row = t;
  float cell[kDim];
  {
    // The row's operands stay as fp16 pairs (widened where used) and the
    // window suffix products, the same for every thread, in scalar
    // registers, leaving the vector registers to the cells.
    const float s = sh.smoothing[row];
    uint32_t ck2[kRank / 2], nk2[kRank / 2], rk2[kWindow / 2];
    float suffix[kWindow];
#pragma unroll
    for (int i = 0; i < kRank / 2; ++i) {
      ck2[i] = reinterpret_cast<const uint32_t*>(sh.ck + row * kRank)[i];
      nk2[i] = reinterpret_cast<const uint32_t*>(sh.nk + row * kRank)[i];
    }
#pragma unroll
    for (int i = 0; i < kWindow / 2; ++i) rk2[i] = reinterpret_cast<const uint32_t*>(sh.rk + row * kWindow)[i];
#pragma unroll
    for (int j = 0; j < kWindow; ++j) {
      suffix[j] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sh.record_suffix[j])));
    }
    // Every compensator and record product is of two fp16 values, exact in
    // fp32: one v_fma_mix_f32 each (half_product), and the fitted ranks'
    // `value -= nk * nv` one fma (minus_half_product), the reference's
    // roundings throughout.
    const float neg_zero = opaque_negative_zero();
    const auto half = [](uint32_t pair, int i) { return i & 1 ? pair >> 16 : pair; };
    // A column's LDS operands; the next column's are read while this one's
    // cell is evaluated, so their latency overlaps the arithmetic.
    struct Operands {
      int code;
      float scale;
      uint2 cv, nv;
      uint4 r0, r1;
    };
    const auto fetch = [&](int column) {
      Operands o;
      o.code = sh.code[column * kCodeStride + row];
      o.scale = sh.scales[column];
      o.cv = *reinterpret_cast<const uint2*>(sh.cv + column * kRank);
      o.nv = *reinterpret_cast<const uint2*>(sh.nv + column * kRank);
      const uint4* const rc4 = reinterpret_cast<const uint4*>(sh.rc + column * kWindow);
      o.r0 = rc4[0];
      o.r1 = rc4[1];
      return o;
    };
    Operands next = fetch(0);
    each_column([&](auto c) {
      constexpr int column = decltype(c)::value;
      // Opaque to the compiler, so the pairs stay packed in registers.
#pragma unroll
      for (int i = 0; i < kRank / 2; ++i) asm volatile("" : "+v"(ck2[i]), "+v"(nk2[i]));
#pragma unroll
      for (int i = 0; i < kWindow / 2; ++i) asm volatile("" : "+v"(rk2[i]));
      const Operands o = next;
      if constexpr (column + 1 < kDim) next = fetch(column + 1);
      // Issued here, ahead of this column's arithmetic, not sunk to its end.
      __builtin_amdgcn_sched_barrier(0);
      // code / 127 by the two-part division (exact for every integer code).
      float value = code_value_arith(static_cast<int8_t>(o.code)) * s * o.scale * bs;
      const uint32_t cvp[kRank / 2] = {o.cv.x, o.cv.y}, nvp[kRank / 2] = {o.nv.x, o.nv.y};
#pragma unroll
      for (int r = 0; r < kRank; ++r) {
        value += half_product(half(ck2[r / 2], r), half(cvp[r / 2], r), neg_zero) * bs;
        value = minus_half_product(value, half(nk2[r / 2], r), half(nvp[r / 2], r));
      }
      const uint32_t rc2[kWindow / 2] = {o.r0.x, o.r0.y, o.r0.z, o.r0.w,
                                         o.r1.x, o.r1.y, o.r1.z, o.r1.w};
#pragma unroll
      for (int j = 0; j < kWindow; ++j) {
        value += half_product(half(rk2[j / 2], j), half(rc2[j / 2], j), neg_zero) * suffix[j];
      }
      cell[column] = value;
      // One column ahead at a time: the scheduler would otherwise hoist the
      // LDS reads of many columns ahead of their use.
      __builtin_amdgcn_sched_barrier(0);
    });
  }
  {
    float4* const work = reinterpret_cast<float4*>(workspace + row * kDim);
#pragma unroll
    for (int q = 0; q < kDim / 4; ++q) {
      work[q] = make_float4(cell[4 * q], cell[4 * q + 1], cell[4 * q + 2], cell[4 * q + 3]);
    }
  }

  // ---- fresh smoothing (row t): sequential sum of |cell| over the columns ----
  float s_new;
  {
    float mean_absolute = 0.0f;
    each_column([&](auto c) { mean_absolute += fabsf(cell[decltype(c)::value]); });
    const float mean = mean_absolute / 128.0f;
    s_new = newton_sqrt(mean > kBoundaryFloor ? mean : kBoundaryFloor);
    next_smoothing[row] = s_new;
  }
  // From here on cell[] holds m = cell / s_new (the cells themselves are in the
  // workspace already): the scale pass divides once and stores m in place.

  // ---- scales: max over rows of |cell / s| per column -------------------------
  // The reference keeps `value > maximum ? value : maximum` from 0 over the
  // rows, which skips NaNs; fmaxf(|m|, 0) maps a NaN to 0 and leaves every
  // other |m| alone, and a maximum of those is exact in any order.  Each
  // wavefront reduces its 64 rows with quarter-width reduce-scatters (32
  // columns across 64 lanes: lane L ends with column L % 32), then the two
  // wavefronts' maxima meet in LDS.
  const int lane = t & 63;
  const int wave = t >> 6;
#pragma unroll
  for (int quarter = 0; quarter < 4; ++quarter) {
#pragma unroll
    for (int i = 0; i < 32; ++i) cell[32 * quarter + i] = cell[32 * quarter + i] / s_new;
    const auto magnitude = [&](int i) { return fmaxf(fabsf(cell[32 * quarter + i]), 0.0f); };
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float lo = fold_max<16>(magnitude(i), magnitude(16 + i), lane);
      const float hi = fold_max<16>(magnitude(8 + i), magnitude(24 + i), lane);
      v[i] = fold_max<8>(lo, hi, lane);
      if (i % 2 == 1) __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = fold_max<4>(v[i], v[i + 4], lane);
#pragma unroll
    for (int i = 0; i < 2; ++i) v[i] = fold_max<2>(v[i], v[i + 2], lane);
    v[0] = fold_max<1>(v[0], v[1], lane);
    v[0] = max_partner<32>(v[0]);
    if (lane < 32) {
      (wave == 0 ? sh.left : sh.right)[32 * quarter + lane] = v[0];
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  __syncthreads();  // both wavefronts' column maxima; every cell has been evaluated
  {
    // Thread t's own slots: no other thread reads them before the barrier.
    const float maximum = fmaxf(sh.left[t], sh.right[t]);
    next_scales[t] = maximum;
    sh.left[t] = maximum;
    // The certified codes' factor RN(127 / maximum) (code_lift in codec_math.h)
    // for a maximum of 0 or in [2^-90, 2^90]; NaN otherwise, which sends every
    // cell of the column to the exact path below.
    sh.right[t] = maximum == 0.0f ? 0.0f
                  : (maximum >= 0x1p-90f && maximum <= 0x1p90f) ? kQuantizedMaximum / maximum
                                                                : __builtin_nanf("");
  }
  __syncthreads();

  // ---- codes: round-half-away (:336-345), handed to the caller's sink ------
  // The reference's q = m / maximum * 127, then trunc(q +- 0.5) clamped to
  // +-127.  Where the lift u = fma(m, RN(127 / maximum), 0.5 + 2^-14) has a
  // fraction of at least 2^-13, q + 0.5 lies at least 2^-15 inside
  // (floor(u), floor(u) + 1), so the rounded q +- 0.5 truncates to floor(u)
  // (the certificate of codec_math.h; |m| <= maximum since the maximum is
  // over these same m).  The other cells, NaN and infinite ones among them,
  // take the reference's expression.
  each_column([&](auto c) {
    constexpr int column = decltype(c)::value;
    const float m = cell[column];
    const float u = code_lift(m, sh.right[column]);
    int code;
    if (lift_fraction(u) >= kCodeLiftMargin) {
      code = lifted_code(u);
    } else {
      const float maximum = sh.left[column];
      float q = maximum == 0.0f ? 0.0f : m / maximum * 127.0f;
      q += q >= 0.0f ? 0.5f : -0.5f;
      q = q > 127.0f ? 127.0f : q;
      q = q < -127.0f ? -127.0f : q;
      code = static_cast<int>(q);
    }
    sink(c, static_cast<int8_t>(code));
    if constexpr (column % 4 == 3) __builtin_amdgcn_sched_barrier(0);
  });
}

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3))) void power_refit_kernel(PowerArgs a) {
  extern __shared__ __align__(16) unsigned char dynamic[];
  PowerShared& sh = *reinterpret_cast<PowerShared*>(dynamic);
  const int t = threadIdx.x;
  const uint64_t state = blockIdx.x;
  if (a.positions[state * kPositionStride] != static_cast<uint32_t>(kWindow)) return;  // uniform
  const uint64_t vb = state * kDim;
  const uint64_t rb = state * kWindow;

  // ---- stage the state in LDS -----------------------------------------------
  for (int i = t; i < kTile / 4; i += kThreads) {
    const uint32_t w = reinterpret_cast<const uint32_t*>(a.residual + state * kTile)[i];
    const int column = (4 * i) / kDim, row = (4 * i) % kDim;
    *reinterpret_cast<uint32_t*>(&sh.code[column * kCodeStride + row]) = w;
  }
  for (int i = t; i < kDim * kRank; i += kThreads) {
    sh.ck[i] = a.comp_keys[vb * kRank + i];
    sh.cv[i] = a.comp_values[vb * kRank + i];
    sh.nk[i] = 0u;
    sh.nv[i] = 0u;
  }
  for (int i = t; i < kWindow * kDim; i += kThreads) {
    const int j = i / kDim, dimension = i % kDim;
    sh.rk[dimension * kWindow + j] = a.record_keys[rb * kDim + i];
    sh.rc[dimension * kWindow + j] = a.record_corrections[rb * kDim + i];
  }
  sh.smoothing[t] = (a.smoothing + vb)[t];
  sh.scales[t] = (a.scales + vb)[t];
  // BuildSuffix (:102-111), computed identically by every thread.
  float bs = 1.0f;
  for (int j = kWindow - 1; j >= 0; --j) {
    if (t == 0) sh.record_suffix[j] = bs;
    bs *= a.record_decay[rb + j];
  }
  // The same value in every lane: keep it in a scalar register.
  bs = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(bs)));
  __syncthreads();

  // ---- deflated power iteration ---------------------------------------------
  for (int rank = 0; rank < kRank; ++rank) {
    sh.right[t] = static_cast<float>(static_cast<int>(((rank + 1) * (t + 3)) % 17) - 8);
    __syncthreads();
    (void)normalize(sh, sh.right, t);
    for (uint32_t it = 0; it < a.power_iterations; ++it) {
      apply_right(sh, sh.right, sh.left, bs, rank, t);
      if (!normalize(sh, sh.left, t)) break;
      apply_transpose(sh, sh.left, sh.right, bs, rank, t);
      if (!normalize(sh, sh.right, t)) break;
    }
    apply_right(sh, sh.right, sh.left, bs, rank, t);
    if (t == 0) {
      float squared = 0.0f;
      for (int i = 0; i < kDim; ++i) squared += sh.left[i] * sh.left[i];
      sh.scalar = newton_sqrt(squared);
    }
    __syncthreads();
    const float singular = sh.scalar;
    if (singular > 1.0e-20f) {
      const float inverse = 1.0f / singular;
      sh.nk[t * kRank + rank] = static_cast<uint16_t>(float_to_half_bits(sh.left[t] * inverse * singular));
      sh.nv[t * kRank + rank] = static_cast<uint16_t>(float_to_half_bits(sh.right[t]));
    }
    __syncthreads();
  }

  // ---- R minus the fit, re-encoded; codes staged in the code area ------------
  // The workspace is written once and never read back.
  reencode_rows(sh, bs, t, a.workspace + state * kTile, a.next_smoothing + vb, a.next_scales + vb,
                [&](auto c, int8_t code) {
                  sh.code[decltype(c)::value * kCodeStride + t] = code;
                });
  __syncthreads();
  // next_residual [value column][key row]: each round of 16 columns, eight
  // lanes write one whole 128-byte column.
#pragma unroll
  for (int round = 0; round < kDim / 16; ++round) {
    const int column = 16 * round + (t >> 3);
    const int offset = 16 * (t & 7);
    const uint32_t* src = reinterpret_cast<const uint32_t*>(&sh.code[column * kCodeStride + offset]);
    *reinterpret_cast<uint4*>(a.next_residual + state * kTile + column * kDim + offset) =
        make_uint4(src[0], src[1], src[2], src[3]);
  }

  // ---- new compensators, cleared window, position ----------------------------
  for (int i = t; i < kDim * kRank; i += kThreads) {
    a.next_comp_keys[vb * kRank + i] = sh.nk[i];
    a.next_comp_values[vb * kRank + i] = sh.nv[i];
  }
  for (int i = t; i < kWindow * kDim / 2; i += kThreads) {
    reinterpret_cast<uint32_t*>(a.record_keys + rb * kDim)[i] = 0u;
    reinterpret_cast<uint32_t*>(a.record_corrections + rb * kDim)[i] = 0u;
  }
  if (t < kWindow) a.record_decay[rb + t] = 0.0f;
  __syncthreads();  // every thread has read the position word above
  if (t == 0) a.positions[state * kPositionStride] = 0u;
}

// ---- encoded_requantize -----------------------------------------------------

struct RequantizeArgs {
  const int8_t* residual;  // [state][row = smoothing axis][column = scale axis]
  const float* smoothing;
  const float* scales;
  const uint16_t* old_left;  // [state][dim][rank]
  const uint16_t* old_right;
  const float* record_decay;
  const uint16_t* record_left;  // [state][record][dim]
  const uint16_t* record_right;
  const uint16_t* new_left;  // [state][rank][dim]
  const uint16_t* new_right;
  int8_t* next_residual;  // [state][row][column]
  float* next_smoothing;
  float* next_scales;
  uint16_t* next_left;  // [state][dim][rank]
  uint16_t* next_right;
  float* workspace;  // [state][row][column]
};

// EncodedRequantize::Process (encoded_requantize.cpp:102-166): the window
// operator minus the committed ranks re-encoded.  The state is staged in the
// power refit's LDS layout (codes transposed to [column][row], the [rank][dim]
// bases to [dim][rank], the records to [dim][record]) and re-encoded by the
// same reencode_rows; the codes go back through the code area to 16-byte
// row stores (168 VGPRs, three wavefronts per SIMD: five workgroups per CU,
// as the LDS allows).
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3))) void encoded_requantize_kernel(
    RequantizeArgs a) {
  extern __shared__ __align__(16) unsigned char dynamic[];
  PowerShared& sh = *reinterpret_cast<PowerShared*>(dynamic);
  const int t = threadIdx.x;
  const uint64_t state = blockIdx.x;
  const uint64_t vb = state * kDim;
  const uint64_t rb = state * kWindow;

  const uint32_t* words = reinterpret_cast<const uint32_t*>(a.residual + state * kTile);
  for (int i = t; i < kTile / 4; i += kThreads) {
    const uint32_t w = words[i];
    const int row = (4 * i) / kDim, column = (4 * i) % kDim;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      sh.code[(column + b) * kCodeStride + row] = static_cast<int8_t>(w >> (8 * b));
    }
  }
  for (int i = t; i < kDim * kRank; i += kThreads) {
    const int dimension = i / kRank, rank = i % kRank;
    sh.ck[i] = a.old_left[vb * kRank + i];
    sh.cv[i] = a.old_right[vb * kRank + i];
    sh.nk[i] = a.new_left[(state * kRank + rank) * kDim + dimension];
    sh.nv[i] = a.new_right[(state * kRank + rank) * kDim + dimension];
  }
  for (int i = t; i < kWindow * kDim; i += kThreads) {
    const int j = i / kDim, dimension = i % kDim;
    sh.rk[dimension * kWindow + j] = a.record_left[rb * kDim + i];
    sh.rc[dimension * kWindow + j] = a.record_right[rb * kDim + i];
  }
  sh.smoothing[t] = (a.smoothing + vb)[t];
  sh.scales[t] = (a.scales + vb)[t];
  // The suffix products (:106-111), computed identically by every thread.
  float bs = 1.0f;
  for (int j = kWindow - 1; j >= 0; --j) {
    if (t == 0) sh.record_suffix[j] = bs;
    bs *= a.record_decay[rb + j];
  }
  bs = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(bs)));
  __syncthreads();

  // The codes of row t, four to a word, staged row-major in the code area
  // (free once every cell has been evaluated; a 132-byte row stride keeps the
  // 64 lanes' word writes in distinct banks), so that only one packed word is
  // live at a time.
  uint32_t quad = 0u;
  reencode_rows(sh, bs, t, a.workspace + state * kTile, a.next_smoothing + vb, a.next_scales + vb,
                [&](auto c, int8_t code) {
                  constexpr int column = decltype(c)::value;
                  quad |= static_cast<uint32_t>(static_cast<uint8_t>(code)) << (8 * (column % 4));
                  if constexpr (column % 4 == 3) {
                    *reinterpret_cast<uint32_t*>(&sh.code[t * kCodeStride + column - 3]) = quad;
                    quad = 0u;
                  }
                });
  __syncthreads();
  // next_residual [row][column]: each round of 16 rows, eight lanes write one
  // whole 128-byte row.
#pragma unroll
  for (int round = 0; round < kDim / 16; ++round) {
    const int row = 16 * round + (t >> 3);
    const int offset = 16 * (t & 7);
    const uint32_t* src = reinterpret_cast<const uint32_t*>(&sh.code[row * kCodeStride + offset]);
    *reinterpret_cast<uint4*>(a.next_residual + state * kTile + row * kDim + offset) =
        make_uint4(src[0], src[1], src[2], src[3]);
  }
  // The committed bases in the [dim][rank] layout: the LDS copies already are.
  for (int i = t; i < kDim * kRank; i += kThreads) {
    a.next_left[vb * kRank + i] = sh.nk[i];
    a.next_right[vb * kRank + i] = sh.nv[i];
  }
}

// The residual workspace of the allocation-free refit entry point: room for
// kNoAllocMaxStates states (32 MiB), one copy per GPU, held by every GPU this
// library runs on until the process ends.  In host code `scratch` names a
// host-side stand-in, never the device array: host code uses only the address
// hipGetSymbolAddress returns for the GPU in question (scratch_on_device).
constexpr uint32_t kNoAllocMaxStates = 512;
static __device__ __align__(256) float scratch[kNoAllocMaxStates * kTile];

constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
float* scratch_address[kMaxDevices] = {};

// The device address of `scratch` on the GPU that `stream` runs on, looked up
// once per GPU with that GPU current (and the caller's current GPU restored).
int32_t scratch_on_device(void* stream, float** address) {
  int device = 0;
  if (hipStreamGetDevice(static_cast<hipStream_t>(stream), &device) != hipSuccess ||
      device < 0 || device >= kMaxDevices) {
    return kStatusLaunchFailed;
  }
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (scratch_address[device] == nullptr) {
    int current = 0;
    if (hipGetDevice(&current) != hipSuccess) return kStatusLaunchFailed;
    if (current != device && hipSetDevice(device) != hipSuccess) return kStatusLaunchFailed;
    void* found = nullptr;
    const hipError_t status = hipGetSymbolAddress(&found, HIP_SYMBOL(scratch));
    if (current != device && hipSetDevice(current) != hipSuccess) return kStatusLaunchFailed;
    if (status != hipSuccess || found == nullptr) return kStatusLaunchFailed;
    scratch_address[device] = static_cast<float*>(found);
  }
  *address = scratch_address[device];
  return kStatusOk;
}

}  // namespace

int32_t launch_power_refit(void* stream, const int8_t* residual, const float* smoothing,
                           const float* scales, const uint16_t* comp_keys,
                           const uint16_t* comp_values, float* record_decay,
                           uint16_t* record_keys, uint16_t* record_corrections,
                           uint32_t* positions, int8_t* next_residual, float* next_smoothing,
                           float* next_scales, uint16_t* next_comp_keys,
                           uint16_t* next_comp_values, float* residual_workspace,
                           uint32_t states, uint32_t power_iterations) {
  const PowerArgs args{residual, smoothing, scales, comp_keys, comp_values, record_decay,
                       record_keys, record_corrections, positions, next_residual, next_smoothing,
                       next_scales, next_comp_keys, next_comp_values, residual_workspace,
                       power_iterations};
  void* pointers[] = {const_cast<PowerArgs*>(&args)};
  const hipError_t status =
      hipLaunchKernel(reinterpret_cast<const void*>(power_refit_kernel), dim3(states),
                      dim3(kThreads), pointers, sizeof(PowerShared),
                      static_cast<hipStream_t>(stream));
  return status == hipSuccess ? kStatusOk : kStatusLaunchFailed;
}

int32_t launch_quant_only_refit(void* stream, const int8_t* residual, const float* smoothing,
                                const float* scales, float* record_decay,
                                uint16_t* record_keys, uint16_t* record_corrections,
                                uint32_t* positions, int8_t* next_residual,
                                float* next_smoothing, float* next_scales,
                                uint16_t* next_comp_keys, uint16_t* next_comp_values,
                                uint32_t states);

}  // namespace gdn

// The window-boundary refit without a caller workspace: the power refit's
// fitted residual goes to the library's own scratch array, so the call
// allocates nothing.  Calls that overlap on one GPU share that array and race.
extern "C" int32_t statecentric_gdn_state_codec_window_boundary_noalloc_launch_v1(
    void* stream, const int8_t* residual, const float* smoothing, const float* scales,
    const uint16_t* compensator_keys, const uint16_t* compensator_values,
    float* record_decay, uint16_t* record_keys, uint16_t* record_corrections,
    uint32_t* positions, int8_t* next_residual, float* next_smoothing, float* next_scales,
    uint16_t* next_compensator_keys, uint16_t* next_compensator_values, uint32_t states,
    uint32_t power_iterations) {
  if (!residual || !smoothing || !scales || !compensator_keys || !compensator_values ||
      !record_decay || !record_keys || !record_corrections || !positions || !next_residual ||
      !next_smoothing || !next_scales || !next_compensator_keys || !next_compensator_values ||
      states == 0 || states > gdn::kMaxWindowStates || power_iterations > 32 ||
      (power_iterations > 0 && states > gdn::kNoAllocMaxStates) ||
      !gdn::aligned16(residual, smoothing, scales, compensator_keys, compensator_values,
                      record_decay, record_keys, record_corrections, positions, next_residual,
                      next_smoothing, next_scales, next_compensator_keys,
                      next_compensator_values)) {
    return gdn::kStatusInvalidArgument;
  }
  if (power_iterations == 0) {  // the quant-only refit uses no workspace
    return gdn::launch_quant_only_refit(stream, residual, smoothing, scales, record_decay,
                                        record_keys, record_corrections, positions,
                                        next_residual, next_smoothing, next_scales,
                                        next_compensator_keys, next_compensator_values, states);
  }
  float* workspace = nullptr;
  const int32_t found = gdn::scratch_on_device(stream, &workspace);
  if (found != gdn::kStatusOk) return found;
  return gdn::launch_power_refit(stream, residual, smoothing, scales, compensator_keys,
                                 compensator_values, record_decay, record_keys,
                                 record_corrections, positions, next_residual, next_smoothing,
                                 next_scales, next_compensator_keys, next_compensator_values,
                                 workspace, states, power_iterations);
}

// encoded_requantize_launch_v1 (encoded_requantize.cpp:102-166, admission
// :189-215): every state re-encoded; see the kernel above.
extern "C" int32_t statecentric_gdn_state_codec_encoded_requantize_launch_v1(
    void* stream, const int8_t* residual, const float* smoothing, const float* scales,
    const uint16_t* old_left, const uint16_t* old_right, const float* record_decay,
    const uint16_t* record_left, const uint16_t* record_right, const uint16_t* new_left,
    const uint16_t* new_right, int8_t* next_residual, float* next_smoothing,
    float* next_scales, uint16_t* next_left, uint16_t* next_right,
    float* residual_workspace, uint32_t states) {
  if (!residual || !smoothing || !scales || !old_left || !old_right || !record_decay ||
      !record_left || !record_right || !new_left || !new_right || !next_residual ||
      !next_smoothing || !next_scales || !next_left || !next_right || !residual_workspace ||
      states == 0 || states > gdn::kMaxWindowStates ||
      !gdn::aligned16(residual, smoothing, scales, old_left, old_right, record_decay,
                      record_left, record_right, new_left, new_right, next_residual,
                      next_smoothing, next_scales, next_left, next_right, residual_workspace)) {
    return gdn::kStatusInvalidArgument;
  }
  const gdn::RequantizeArgs args{residual, smoothing, scales, old_left, old_right,
                                 record_decay, record_left, record_right, new_left, new_right,
                                 next_residual, next_smoothing, next_scales, next_left,
                                 next_right, residual_workspace};
  void* pointers[] = {const_cast<gdn::RequantizeArgs*>(&args)};
  const hipError_t status = hipLaunchKernel(
      reinterpret_cast<const void*>(gdn::encoded_requantize_kernel), dim3(states),
      dim3(gdn::kThreads), pointers, sizeof(gdn::PowerShared), static_cast<hipStream_t>(stream));
  return status == hipSuccess ? gdn::kStatusOk : gdn::kStatusLaunchFailed;
}
