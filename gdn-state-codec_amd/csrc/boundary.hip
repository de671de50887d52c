// Window-boundary refit: once a state's 16-record window is full, its records
// are folded into a new int8 boundary (native/ascendc/gdn_state_codec/kernel/
// gdn_state_codec_window_boundary.cpp).
//
// Quant-only refit (power_iterations == 0, :368-499): for every value column v
// of every state,
//   w[k]   = ((code[v][k] * ((scale[v] * S) / 127)) * s[k]) + records(v, k)
//   m[k]   = w[k] / s[k]                       (the existing smoothing is kept)
//   scale' = max_k |m[k]|
//   code'  = rint_even(fp16(clamp(m[k] * (127 / scale'), +-127)))
// where S is the product of the 16 record gates and records(v, k) is either
// the 16 record terms key_j[k] * (corr_j[v] * suffix_j) added in record order
// (window_boundary_launch_v1) or a precomputed fp32 merge [v][k]
// (window_boundary_cube_finish_launch_v1, fed by the boundary runtime's fp16
// record GEMM).  Compensator outputs are zero and every position is reset.
//
// One workgroup per state; each wavefront owns 32 value columns and each lane
// two keys, so a column is one coalesced 128-byte row read and write.  The
// per-column scalars (corr_j[v] * suffix_j and (scale[v] * S) / 127) are formed
// once per state in LDS, the 32 column maxima come from one reduce-scatter and
// their multipliers from one vector division.  The arithmetic keeps the
// reference's statement order with separately rounded multiplies and adds,
// making the result bit-identical to its CPU statement.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "codec_math.h"
#include "gdn_state_codec_window.h"
#include "launch.h"
#include "stream_memory.h"
#include "window_common.h"

namespace gdn {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kColumnsPerWave = kDim / kWaves;
// The reference's Cube-backed entry points admit at most 128 states
// (window_boundary.cpp:698-703, 724-731; bf16_cube_matmul.cpp:56-60).
constexpr uint32_t kMaxCubeStates = 128;

struct RefitArgs {
  const int8_t* residual;
  const float* smoothing;
  const float* scales;
  const float* record_decay;
  const uint16_t* record_keys;
  const uint16_t* record_corrections;
  uint32_t* positions;
  int8_t* next_residual;
  float* next_smoothing;
  float* next_scales;
  uint16_t* next_comp_keys;
  uint16_t* next_comp_values;
  const float* record_merge;  // nullptr: add the 16 record terms
  uint32_t states;
};

// rint_even(fp16(t)): the Ascend cast to half, then to int8 with CAST_RINT.
__device__ __forceinline__ uint32_t rint_through_half(float t) {
  const float h = half_bits_to_float(float_to_half_bits(t));
  return static_cast<uint32_t>(static_cast<int32_t>(__builtin_rintf(h))) & 0xFFu;
}

// One halving exchange of a max reduce-scatter over lane bit kMask: the lane
// with the bit clear keeps v[0, N/2), its partner v[N/2, N), and each takes
// the max with the partner's copy of the half it keeps.  Recursion (not a
// runtime loop) keeps every array index a constant, so v stays in registers.
template <int N, int kMask>
__device__ __forceinline__ void halve_max(float* v, int lane) {
  if constexpr (N > 1) {
    constexpr int n = N / 2;
    const bool up = (lane & kMask) != 0;
#pragma unroll
    for (int i = 0; i < n; ++i) {
      const float lo = v[i];
      const float hi = v[i + n];
      const float send = up ? lo : hi;
      const float keep = up ? hi : lo;
      v[i] = fmaxf(keep, __shfl_xor(send, kMask));
    }
    halve_max<n, kMask / 2>(v, lane);
  }
}

// Reduce-scatter of per-lane column maxima: v[c] holds this lane's max for
// column c (c < 32); afterwards lane L holds the wave-wide max of column
// L >> 1 (five halvings over lane bits 5..1, one exchange over bit 0; max is
// exact, so the grouping does not change the result).
__device__ __forceinline__ float reduce_scatter_max32(float (&v)[32], int lane) {
  halve_max<32, 32>(v, lane);
  return fmaxf(v[0], __shfl_xor(v[0], 1));
}

template <bool kMerged>
__global__ __launch_bounds__(kThreads) void quant_only_refit_kernel(RefitArgs a) {
  // Per-state tables, formed once: corr_j[v] * suffix_j (the record terms'
  // per-column scalars) and (scale[v] * S) / 127, with the same fp32
  // roundings as evaluating them per element.
  __shared__ __align__(16) float scaled_corrections[kDim][kWindow];
  __shared__ float factors[kDim];
  __shared__ float multipliers[kWaves][kColumnsPerWave];
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const uint64_t state = blockIdx.x;
  const uint64_t vector_base = state * kDim;
  const uint64_t record_base = state * kWindow;

  float gates[kWindow];
#pragma unroll
  for (int j = 0; j < kWindow; ++j) gates[j] = a.record_decay[record_base + j];
  const int k0 = 2 * lane;
  const int column0 = wave * kColumnsPerWave;
  const int8_t* codes = a.residual + state * kTile;
  // This lane's two codes of each of the wave's 32 columns (rows of [v][k]).
  uint32_t pair[kColumnsPerWave];
#pragma unroll
  for (int c = 0; c < kColumnsPerWave; ++c) {
    pair[c] = *reinterpret_cast<const uint16_t*>(codes + (column0 + c) * kDim + k0);
  }
  // Every other load before any arithmetic that waits on one (memory returns
  // in issue order): the record corrections of this thread's column (threads
  // 0..127 take records 0..7 of column t, threads 128..255 records 8..15 of
  // column t - 128: coalesced 256-byte fp16 rows per record), the column's
  // scale, this lane's smoothing pair and its two keys of the 16 records.
  const int own_column = t & (kDim - 1);
  const int j0 = (t >> 7) * (kWindow / 2);
  uint16_t correction_bits[kWindow / 2];
  uint32_t key_words[kWindow];
  if constexpr (!kMerged) {
#pragma unroll
    for (int jj = 0; jj < kWindow / 2; ++jj) {
      correction_bits[jj] = a.record_corrections[(record_base + j0 + jj) * kDim + own_column];
    }
  }
  const float own_scale = t < kDim ? a.scales[vector_base + t] : 0.0f;
  const float2 sm = *reinterpret_cast<const float2*>(a.smoothing + vector_base + k0);
  if constexpr (!kMerged) {
#pragma unroll
    for (int j = 0; j < kWindow; ++j) {
      key_words[j] = *reinterpret_cast<const uint32_t*>(a.record_keys + (record_base + j) * kDim + k0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // Gate suffixes in the reference's order (BuildSuffix, :102-111).
  float suffix[kWindow];
  float boundary_suffix = 1.0f;
#pragma unroll
  for (int j = kWindow - 1; j >= 0; --j) {
    suffix[j] = boundary_suffix;
    boundary_suffix *= gates[j];
  }
  if constexpr (!kMerged) {
#pragma unroll
    for (int jj = 0; jj < kWindow / 2; ++jj) {
      float sfx = suffix[jj];
      if (j0 != 0) sfx = suffix[jj + kWindow / 2];
      scaled_corrections[own_column][j0 + jj] = half_bits_to_float(correction_bits[jj]) * sfx;
    }
  }
  if (t < kDim) factors[t] = own_scale * boundary_suffix / 127.0f;
  float key0[kWindow], key1[kWindow];
  if constexpr (!kMerged) {
#pragma unroll
    for (int j = 0; j < kWindow; ++j) {
      key0[j] = half_bits_to_float(key_words[j] & 0xFFFFu);
      key1[j] = half_bits_to_float(key_words[j] >> 16);
    }
  }
  __syncthreads();

  // m[k] = w[k] / s[k] for the wave's 32 columns, kept in registers.
  // Markstein's division by the lane's two smoothing values (div_by_reciprocal)
  // equals IEEE division when s lies in [2^-20, 2^20] and every w is 0 or in
  // [2^-100, 2^100], so that |w/s| lies in [2^-120, 2^120]; -0 gives +0, which
  // neither max|m| nor the code rounding can see.  The loop divides that way
  // and checks the domain as it goes (the smallest non-zero |w| as an unsigned
  // minimum of (bits << 1) - 1, where a zero becomes the largest value); a
  // wavefront with a lane outside it computes w again and divides with IEEE
  // division.
  const auto boundary_value = [&](int c, float& w0, float& w1) {
    const int v = column0 + c;
    const float factor = factors[v];
    w0 = static_cast<float>(static_cast<int8_t>(pair[c] & 0xFFu)) * factor * sm.x;
    w1 = static_cast<float>(static_cast<int8_t>(pair[c] >> 8)) * factor * sm.y;
    if constexpr (kMerged) {
      const float2 merge = *reinterpret_cast<const float2*>(a.record_merge + state * kTile + v * kDim + k0);
      w0 = w0 + merge.x;
      w1 = w1 + merge.y;
    } else {
      float scalar[kWindow];
#pragma unroll
      for (int q = 0; q < kWindow; q += 4) {
        const float4 x = *reinterpret_cast<const float4*>(&scaled_corrections[v][q]);
        scalar[q] = x.x;
        scalar[q + 1] = x.y;
        scalar[q + 2] = x.z;
        scalar[q + 3] = x.w;
      }
#pragma unroll
      for (int j = 0; j < kWindow; ++j) {
        w0 = key0[j] * scalar[j] + w0;
        w1 = key1[j] * scalar[j] + w1;
      }
    }
  };
  const float y0 = 1.0f / sm.x, y1 = 1.0f / sm.y;
  uint32_t min_key = 0xFFFFFFFFu;
  float max_abs = 0.0f;
  float m0[kColumnsPerWave], m1[kColumnsPerWave];
#pragma unroll
  for (int c = 0; c < kColumnsPerWave; ++c) {
    float w0, w1;
    boundary_value(c, w0, w1);
    min_key = min(min_key, min((__float_as_uint(w0) << 1) - 1u, (__float_as_uint(w1) << 1) - 1u));
    max_abs = fmaxf(max_abs, fmaxf(fabsf(w0), fabsf(w1)));
    m0[c] = div_by_reciprocal(w0, sm.x, y0);
    m1[c] = div_by_reciprocal(w1, sm.y, y1);
  }
  const float min_abs =
      min_key == 0xFFFFFFFFu ? INFINITY : __uint_as_float((min_key + 1u) >> 1);
  const bool lane_fast = min_abs >= 0x1p-100f && max_abs <= 0x1p100f &&
                         sm.x >= 0x1p-20f && sm.x <= 0x1p20f &&
                         sm.y >= 0x1p-20f && sm.y <= 0x1p20f;
  if (!__all(lane_fast)) {
#pragma unroll
    for (int c = 0; c < kColumnsPerWave; ++c) {
      float w0, w1;
      boundary_value(c, w0, w1);
      m0[c] = w0 / sm.x;
      m1[c] = w1 / sm.y;
    }
  }

  // Column maxima (scale'), then every column's multiplier 127 / scale' in one
  // vector division: lane 2c holds column c.
  float column_max[kColumnsPerWave];
#pragma unroll
  for (int c = 0; c < kColumnsPerWave; ++c) column_max[c] = fmaxf(fabsf(m0[c]), fabsf(m1[c]));
  const float maximum = reduce_scatter_max32(column_max, lane);
  if ((lane & 1) == 0) {
    a.next_scales[vector_base + column0 + (lane >> 1)] = maximum;
    multipliers[wave][lane >> 1] = maximum > 0.0f ? 127.0f / maximum : 0.0f;
  }
  wave_lds_sync();

  int8_t* out = a.next_residual + state * kTile;
#pragma unroll
  for (int c = 0; c < kColumnsPerWave; ++c) {
    const float multiplier = multipliers[wave][c];
    float t0 = m0[c] * multiplier, t1 = m1[c] * multiplier;
    t0 = fminf(fmaxf(t0, -127.0f), 127.0f);
    t1 = fminf(fmaxf(t1, -127.0f), 127.0f);
    const uint32_t packed = rint_through_half(t0) | (rint_through_half(t1) << 8);
    *reinterpret_cast<uint16_t*>(out + (column0 + c) * kDim + k0) = static_cast<uint16_t>(packed);
  }
  // Smoothing kept, compensators zero, position reset (the finalize kernel).
  if (t < kDim) a.next_smoothing[vector_base + t] = a.smoothing[vector_base + t];
  for (int i = t; i < kDim * kRank / 2; i += kThreads) {
    reinterpret_cast<uint32_t*>(a.next_comp_keys + vector_base * kRank)[i] = 0u;
    reinterpret_cast<uint32_t*>(a.next_comp_values + vector_base * kRank)[i] = 0u;
  }
  if (t == 0) a.positions[state * kPositionStride] = 0u;
}

// scaled[j][k] = fp16(key_j[k] * fp16(suffix_j)), suffix_j the product of the
// later gates in ascending order (:550-580).  One thread per (record, key pair).
__global__ __launch_bounds__(kThreads) void scale_records_kernel(
    const float* __restrict__ record_decay, const uint16_t* __restrict__ record_keys,
    uint16_t* __restrict__ scaled, uint32_t states) {
  const uint64_t index = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const uint64_t pairs = static_cast<uint64_t>(states) * kWindow * (kDim / 2);
  if (index >= pairs) return;
  const uint64_t record = index / (kDim / 2);  // state * 16 + j
  const uint64_t state = record / kWindow;
  const int j = static_cast<int>(record % kWindow);
  float suffix = 1.0f;
  for (int later = j + 1; later < kWindow; ++later) suffix *= record_decay[state * kWindow + later];
  const float hs = half_bits_to_float(float_to_half_bits(suffix));
  const uint32_t w = reinterpret_cast<const uint32_t*>(record_keys)[index];
  const uint32_t lo = float_to_half_bits(half_bits_to_float(w & 0xFFFFu) * hs);
  const uint32_t hi = float_to_half_bits(half_bits_to_float(w >> 16) * hs);
  reinterpret_cast<uint32_t*>(scaled)[index] = lo | (hi << 16);
}

// C[s][m][n] = sum_{k<16} A[s][k][m] * B[s][k][n] in ascending k (fp16 products
// are exact in fp32).  One workgroup per state; thread t owns row m = t / 2,
// columns 64 * (t % 2)..+63.
__global__ __launch_bounds__(kThreads) void f16_at_b_kernel(const uint16_t* __restrict__ a,
                                                            const uint16_t* __restrict__ b,
                                                            float* __restrict__ c) {
  __shared__ float sa[kWindow][kDim];
  __shared__ float sb[kWindow][kDim];
  const int t = threadIdx.x;
  const uint64_t state = blockIdx.x;
  for (int i = t; i < kWindow * kDim; i += kThreads) {
    sa[i / kDim][i % kDim] = half_bits_to_float(a[state * kWindow * kDim + i]);
    sb[i / kDim][i % kDim] = half_bits_to_float(b[state * kWindow * kDim + i]);
  }
  __syncthreads();
  const int m = t >> 1;
  const int n0 = 64 * (t & 1);
  float* row = c + state * kTile + static_cast<uint64_t>(m) * kDim + n0;
  for (int n4 = 0; n4 < 64; n4 += 4) {
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < kWindow; ++k) {
      const float x = sa[k][m];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] += x * sb[k][n0 + n4 + i];
    }
    *reinterpret_cast<float4*>(row + n4) = make_float4(acc[0], acc[1], acc[2], acc[3]);
  }
}

int32_t launch_refit(void* stream, const RefitArgs& args) {
  if (args.record_merge != nullptr) {
    return launch(quant_only_refit_kernel<true>, dim3(args.states), dim3(kThreads), stream, args);
  }
  return launch(quant_only_refit_kernel<false>, dim3(args.states), dim3(kThreads), stream, args);
}

}  // namespace

// The quant-only refit (records folded, existing smoothing) of `states` slot states.
int32_t launch_quant_only_refit(void* stream, const int8_t* residual, const float* smoothing,
                                const float* scales, float* record_decay,
                                uint16_t* record_keys, uint16_t* record_corrections,
                                uint32_t* positions, int8_t* next_residual,
                                float* next_smoothing, float* next_scales,
                                uint16_t* next_comp_keys, uint16_t* next_comp_values,
                                uint32_t states) {
  const RefitArgs args{residual, smoothing, scales, record_decay, record_keys,
                       record_corrections, positions, next_residual, next_smoothing,
                       next_scales, next_comp_keys, next_comp_values, nullptr, states};
  return launch_refit(stream, args);
}

int32_t launch_power_refit(void* stream, const int8_t* residual, const float* smoothing,
                           const float* scales, const uint16_t* comp_keys,
                           const uint16_t* comp_values, float* record_decay,
                           uint16_t* record_keys, uint16_t* record_corrections,
                           uint32_t* positions, int8_t* next_residual, float* next_smoothing,
                           float* next_scales, uint16_t* next_comp_keys,
                           uint16_t* next_comp_values, float* residual_workspace,
                           uint32_t states, uint32_t power_iterations);

int32_t launch_scale_records(void* stream, const float* record_decay, const uint16_t* record_keys,
                             uint16_t* scaled, uint32_t states) {
  const uint64_t pairs = static_cast<uint64_t>(states) * kWindow * (kDim / 2);
  return launch(scale_records_kernel, dim3(static_cast<uint32_t>((pairs + kThreads - 1) / kThreads)),
                dim3(kThreads), stream, record_decay, record_keys, scaled, states);
}

int32_t launch_f16_at_b(void* stream, const uint16_t* a, const uint16_t* b, float* c,
                        uint32_t states) {
  return launch(f16_at_b_kernel, dim3(states), dim3(kThreads), stream, a, b, c);
}

}  // namespace gdn

extern "C" int32_t statecentric_gdn_state_codec_window_boundary_launch_v1(
    void* stream, const int8_t* residual, const float* smoothing, const float* scales,
    const uint16_t* compensator_keys, const uint16_t* compensator_values,
    float* record_decay, uint16_t* record_keys, uint16_t* record_corrections,
    uint32_t* positions, int8_t* next_residual, float* next_smoothing, float* next_scales,
    uint16_t* next_compensator_keys, uint16_t* next_compensator_values,
    float* residual_workspace, uint32_t states, uint32_t power_iterations) {
  if (!residual || !smoothing || !scales || !compensator_keys || !compensator_values ||
      !record_decay || !record_keys || !record_corrections || !positions || !next_residual ||
      !next_smoothing || !next_scales || !next_compensator_keys || !next_compensator_values ||
      !residual_workspace || states == 0 || states > gdn::kMaxWindowStates ||
      power_iterations > 32 ||
      !gdn::aligned16(residual, smoothing, scales, compensator_keys, compensator_values,
                      record_decay, record_keys, record_corrections, positions, next_residual,
                      next_smoothing, next_scales, next_compensator_keys,
                      next_compensator_values, residual_workspace)) {
    return gdn::kStatusInvalidArgument;
  }
  if (power_iterations > 0) {
    return gdn::launch_power_refit(stream, residual, smoothing, scales, compensator_keys,
                                   compensator_values, record_decay, record_keys,
                                   record_corrections, positions, next_residual, next_smoothing,
                                   next_scales, next_compensator_keys, next_compensator_values,
                                   residual_workspace, states, power_iterations);
  }
  return gdn::launch_quant_only_refit(stream, residual, smoothing, scales, record_decay,
                                      record_keys, record_corrections, positions, next_residual,
                                      next_smoothing, next_scales, next_compensator_keys,
                                      next_compensator_values, states);
}

extern "C" int32_t statecentric_gdn_state_codec_window_boundary_cube_finish_launch_v1(
    void* stream, const int8_t* residual, const float* smoothing, const float* scales,
    const uint16_t* compensator_keys, const uint16_t* compensator_values,
    float* record_decay, uint16_t* record_keys, uint16_t* record_corrections,
    uint32_t* positions, int8_t* next_residual, float* next_smoothing, float* next_scales,
    uint16_t* next_compensator_keys, uint16_t* next_compensator_values, float* record_merge,
    uint32_t states) {
  if (!residual || !smoothing || !scales || !compensator_keys || !compensator_values ||
      !record_decay || !record_keys || !record_corrections || !positions || !next_residual ||
      !next_smoothing || !next_scales || !next_compensator_keys || !next_compensator_values ||
      !record_merge || states == 0 || states > gdn::kMaxCubeStates ||
      !gdn::aligned16(residual, smoothing, scales, compensator_keys, compensator_values,
                      record_decay, record_keys, record_corrections, positions, next_residual,
                      next_smoothing, next_scales, next_compensator_keys,
                      next_compensator_values, record_merge)) {
    return gdn::kStatusInvalidArgument;
  }
  const gdn::RefitArgs args{residual, smoothing, scales, record_decay, record_keys,
                            record_corrections, positions, next_residual, next_smoothing,
                            next_scales, next_compensator_keys, next_compensator_values,
                            record_merge, states};
  return gdn::launch_refit(stream, args);
}

extern "C" int32_t statecentric_gdn_state_codec_boundary_scale_records_launch_v1(
    void* stream, const float* record_decay, const uint16_t* record_keys,
    uint16_t* scaled_record_keys, uint32_t states) {
  if (!record_decay || !record_keys || !scaled_record_keys || states == 0 ||
      states > gdn::kMaxCubeStates ||
      !gdn::aligned16(record_decay, record_keys, scaled_record_keys)) {
    return gdn::kStatusInvalidArgument;
  }
  return gdn::launch_scale_records(stream, record_decay, record_keys, scaled_record_keys, states);
}

extern "C" int32_t statecentric_gdn_state_codec_bf16_cube_matmul_launch_v1(
    void* stream, const uint16_t* a, const uint16_t* b, float* c, uint32_t states,
    void* workspace, void* tiling, uint32_t blocks) {
  if (!a || !b || !c || !workspace || !tiling || blocks == 0 || blocks > 64 || states == 0 ||
      states > gdn::kMaxCubeStates || blocks != (states + 1u) / 2u ||
      !gdn::aligned16(a, b, c)) {
    return gdn::kStatusInvalidArgument;
  }
  return gdn::launch_f16_at_b(stream, a, b, c, states);
}

// ---- boundary runtime (host/gdn_state_codec_boundary_runtime.cpp:60-128) ----
// One process-wide handle for a fixed state count (1..128), reference-counted;
// step = scale the record keys by their gate suffixes, then the fp16 record
// GEMM record_merge[v][k] = sum_j corr_j[v] * scaled_key_j[k].  The kernels
// need no workspace, so the handle owns no device memory.

namespace {

struct BoundaryRuntime {
  uint32_t states = 0;
  uint32_t references = 0;
};

std::mutex boundary_mutex;
BoundaryRuntime* boundary_runtime = nullptr;

}  // namespace

extern "C" void* statecentric_gdn_state_codec_boundary_runtime_create_v1(uint32_t states) {
  if (states == 0 || states > gdn::kMaxCubeStates) return nullptr;
  std::lock_guard<std::mutex> lock(boundary_mutex);
  if (boundary_runtime != nullptr) {
    if (boundary_runtime->states != states) return nullptr;
    ++boundary_runtime->references;
    return boundary_runtime;
  }
  boundary_runtime = new BoundaryRuntime{states, 1};
  return boundary_runtime;
}

extern "C" void statecentric_gdn_state_codec_boundary_runtime_destroy_v1(void* opaque) {
  std::lock_guard<std::mutex> lock(boundary_mutex);
  auto* runtime = static_cast<BoundaryRuntime*>(opaque);
  if (runtime == nullptr || runtime != boundary_runtime) return;
  if (--runtime->references != 0) return;
  boundary_runtime = nullptr;
  delete runtime;
}

extern "C" int32_t statecentric_gdn_state_codec_boundary_runtime_step_v1(
    void* opaque, void* stream, const float* record_decay, const uint16_t* record_keys,
    const uint16_t* record_corrections, uint16_t* scaled_record_keys, float* record_merge,
    uint32_t states) {
  {
    std::lock_guard<std::mutex> lock(boundary_mutex);
    auto* runtime = static_cast<BoundaryRuntime*>(opaque);
    if (runtime == nullptr || runtime != boundary_runtime || !record_decay || !record_keys ||
        !record_corrections || !scaled_record_keys || !record_merge ||
        states != runtime->states ||
        !gdn::aligned16(record_decay, record_keys, record_corrections, scaled_record_keys,
                        record_merge)) {
      return 1;
    }
  }
  if (gdn::launch_scale_records(stream, record_decay, record_keys, scaled_record_keys, states) !=
      gdn::kStatusOk) {
    return 2;
  }
  if (gdn::launch_f16_at_b(stream, record_corrections, scaled_record_keys, record_merge, states) !=
      gdn::kStatusOk) {
    return 3;
  }
  return 0;
}
