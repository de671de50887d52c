// The reference's device rank-4 chain over an encoded boundary: the two
// per-state finishing kernels that run after prepare_int8_vector and the int8
// GEMM (kernel/gdn_state_codec_encoded_projection.cpp, EncodedProjection
// :43-175, finish_encoded_projection :778-820, commit_encoded_rank :822-865).
//
// For state s, with the input vector x = column 0 of `input` (fp16
// [128][16]) and the int32 projection p = column 0 of `projected`, each row
// of the window operator (transpose == 0) or of its transpose is
//   value[row] = p[row] * dyn / 127 * axis[row] * B
//              + sum_r out_old[row][r] * (sum_a in_old[a][r] x[a]) * B
//              - sum_{r < fitted} out_new[r][row] * (sum_a in_new[r][a] x[a])
//              + sum_j out_rec[j][row] * (sum_a in_rec[j][a] x[a]) * suffix_j
// (B the product of the 16 record gates, suffix_j that of the records after
// j); finish writes value / |value| as fp16 to column 0 of `output` (columns
// 1..15 zero), commit writes value to column 0 of `corrected`, fp16(value) to
// new_left[rank] and x's fp16 bits to new_right[rank].
//
// One 64-lane wavefront per state.  The 24 coefficient sums are sequential
// fp32 sums in the reference's order, one per lane (lanes 0..3 the old ranks,
// 4..7 the fitted ones, 8..23 the records), over the input vector and the
// input-side bases staged in LDS (records first, then the rank bases in the
// same area); the coefficients are then broadcast through
// scalar registers and every lane evaluates two rows.  The squared norm is the
// reference's sequential sum, evaluated identically by every lane from LDS.
// Operations and their order are the reference's, so results are
// bit-identical to its scalar code restated on the CPU.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gdn_state_codec_window.h"
#include "launch.h"
#include "window_common.h"

namespace gdn {
namespace {

constexpr int kLanes = 64;
constexpr int kVectorColumns = 16;  // vector operands are [128][16], column 0 used
constexpr int kScalarStride = 8;    // dynamic_scale is [S][8], element 0 used
constexpr int kCoefficients = 2 * kRank + kWindow;

struct RankArgs {
  const int32_t* projected;
  const float* dynamic_scale;
  const uint16_t* input;
  const float* smoothing;
  const float* scales;
  const uint16_t* old_left;   // [S][dim][rank]
  const uint16_t* old_right;
  const float* record_decay;  // [S][16]
  const uint16_t* record_left;   // [S][record][dim]
  const uint16_t* record_right;
  uint16_t* new_left;   // [S][rank][dim]; commit writes rank `ranks`
  uint16_t* new_right;
  uint16_t* output;     // finish: fp16 [S][128][16]
  float* corrected;     // commit: fp32 [S][128][16], column 0 written
  uint32_t ranks;       // finish: fitted ranks (0..4); commit: the rank committed (0..3)
  uint32_t transpose;   // finish only
};

// window_boundary.cpp:17-23 / encoded_projection.cpp:36-42.
__device__ __forceinline__ float newton_sqrt(float value) {
  float estimate = value > 1.0f ? value : 1.0f;
#pragma unroll 1
  for (int i = 0; i < 20; ++i) estimate = 0.5f * (estimate + value / estimate);
  return estimate;
}

__device__ __forceinline__ float readlane(float value, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(value), lane));
}

// LDS: x as fp16 bits and one 4 KiB staging area, 4,352 bytes in all.  The
// CU allocates LDS in 1,280-byte granules, so that is four granules and 32
// of these one-wavefront workgroups fit on a CU, where the wave slots allow
// 32; six granules (the bases and the records staged side by side) allowed 21.
struct RowsShared {
  uint16_t x[kDim];
  union {
    __align__(16) uint16_t records[kWindow * kDim];  // [record][dim]
    struct {
      __align__(16) uint16_t old_in[kDim * kRank];  // [dim][rank]
      __align__(16) uint16_t new_in[kRank * kDim];  // [rank][dim]
    } ranks;
    float values[kDim];  // finish: the rows, for the squared norm
  };
};
static_assert(workgroups_by_lds(sizeof(RowsShared)) == 32, "32 one-wavefront workgroups per CU");

template <bool kCommit>
__global__ __launch_bounds__(kLanes) void encoded_rows_kernel(RankArgs a) {
  __shared__ RowsShared sh;

  const int lane = threadIdx.x;
  const uint64_t state = blockIdx.x;
  const uint32_t ranks = a.ranks;
  // transpose == 0: the input vector lives on the right (scale) axis.
  const bool left_in = !kCommit && a.transpose != 0;
  const uint64_t basis = state * kDim * kRank;
  const uint64_t records = state * kWindow * kDim;
  const uint16_t* const old_out = (left_in ? a.old_right : a.old_left) + basis;
  const uint16_t* const new_out = (left_in ? a.new_right : a.new_left) + basis;
  const uint16_t* const record_out = (left_in ? a.record_right : a.record_left) + records;
  const float* const axis = (left_in ? a.scales : a.smoothing) + state * kDim;
  const uint16_t* const input = a.input + state * kDim * kVectorColumns;

  // ---- stage x and the input-side records; the rank bases wait in registers
  for (int row = lane; row < kDim; row += kLanes) sh.x[row] = input[row * kVectorColumns];
  const uint4 old_words =
      reinterpret_cast<const uint4*>((left_in ? a.old_left : a.old_right) + basis)[lane];
  const uint4 new_words =
      reinterpret_cast<const uint4*>((left_in ? a.new_left : a.new_right) + basis)[lane];
  const uint4* const record_src =
      reinterpret_cast<const uint4*>((left_in ? a.record_left : a.record_right) + records);
#pragma unroll
  for (int i = 0; i < kWindow * kDim / 8 / kLanes; ++i) {
    reinterpret_cast<uint4*>(sh.records)[i * kLanes + lane] = record_src[i * kLanes + lane];
  }
  wave_lds_sync();

  // ---- PrepareState (:82-123): one sequential sum per coefficient lane ------
  // Lanes 8..23 sum the records first; the rank bases then replace the
  // records in the staging area and lanes 0..7 sum them.  Each term is an
  // fp16 basis value times an fp16 input value, a product exact in fp32, so
  // `total += b * x` rounds exactly what fma(b, x, total) rounds: one
  // v_fma_mix_f32 per term, widening both halves itself.
  const auto sum = [&](const uint16_t* basis_lds, int stride) {
    float total = 0.0f;
    for (int i = 0; i < kDim; ++i) {
      total = __builtin_fmaf(half_bits_to_float(basis_lds[i * stride]),
                             half_bits_to_float(sh.x[i]), total);
    }
    return total;
  };
  float coefficient = 0.0f;
  if (lane >= 2 * kRank && lane < kCoefficients) {
    coefficient = sum(sh.records + (lane - 2 * kRank) * kDim, 1);
  }
  wave_lds_sync();
  reinterpret_cast<uint4*>(sh.ranks.old_in)[lane] = old_words;
  reinterpret_cast<uint4*>(sh.ranks.new_in)[lane] = new_words;
  wave_lds_sync();
  if (lane < kRank) {
    coefficient = sum(sh.ranks.old_in + lane, kRank);
  } else if (lane < 2 * kRank) {
    coefficient = sum(sh.ranks.new_in + (lane - kRank) * kDim, 1);
  }
  // Record coefficients times their suffixes, and the whole window's product.
  const float* const decay = a.record_decay + state * kWindow;
  float suffix = 1.0f;
  for (int j = kWindow - 1; j >= 0; --j) {
    if (lane == 2 * kRank + j) coefficient *= suffix;
    suffix *= decay[j];
  }
  const float boundary_suffix = suffix;
  float old_coefficient[kRank], new_coefficient[kRank], record_coefficient[kWindow];
#pragma unroll
  for (int r = 0; r < kRank; ++r) {
    old_coefficient[r] = readlane(coefficient, r);
    new_coefficient[r] = readlane(coefficient, kRank + r);
  }
#pragma unroll
  for (int j = 0; j < kWindow; ++j) record_coefficient[j] = readlane(coefficient, 2 * kRank + j);

  // ---- Value (:125-163) for rows lane and lane + 64 -------------------------
  const float dynamic = a.dynamic_scale[state * kScalarStride];
  float row_value[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int row = lane + h * kLanes;
    float value = static_cast<float>(a.projected[(state * kDim + row) * kVectorColumns]) *
                  dynamic / 127.0f * axis[row] * boundary_suffix;
#pragma unroll
    for (int r = 0; r < kRank; ++r) {
      value += half_bits_to_float(old_out[row * kRank + r]) * old_coefficient[r] *
               boundary_suffix;
      if (static_cast<uint32_t>(r) < ranks) {
        value -= half_bits_to_float(new_out[r * kDim + row]) * new_coefficient[r];
      }
    }
#pragma unroll
    for (int j = 0; j < kWindow; ++j) {
      value += half_bits_to_float(record_out[j * kDim + row]) * record_coefficient[j];
    }
    row_value[h] = value;
  }

  if constexpr (kCommit) {
    const uint64_t committed = (state * kRank + ranks) * kDim;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int row = lane + h * kLanes;
      a.corrected[(state * kDim + row) * kVectorColumns] = row_value[h];
      a.new_left[committed + row] = static_cast<uint16_t>(float_to_half_bits(row_value[h]));
      a.new_right[committed + row] = input[row * kVectorColumns];
    }
  } else {
    // Squared norm: the reference's sequential sum over the rows, evaluated
    // identically in every lane from LDS.
    sh.values[lane] = row_value[0];
    sh.values[lane + kLanes] = row_value[1];
    wave_lds_sync();
    float squared_norm = 0.0f;
    for (int row = 0; row < kDim; ++row) squared_norm += sh.values[row] * sh.values[row];
    const float inverse = squared_norm > 1.0e-20f ? 1.0f / newton_sqrt(squared_norm) : 0.0f;
    uint16_t* const output = a.output + state * kDim * kVectorColumns;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int row = lane + h * kLanes;
      const uint32_t bits = float_to_half_bits(row_value[h] * inverse);
      uint4* const out = reinterpret_cast<uint4*>(output + row * kVectorColumns);
      out[0] = make_uint4(bits, 0u, 0u, 0u);
      out[1] = make_uint4(0u, 0u, 0u, 0u);
    }
  }
}

int32_t launch_rows(bool commit, const RankArgs& args, uint32_t states, void* stream) {
  return commit ? launch(encoded_rows_kernel<true>, dim3(states), dim3(kLanes), stream, args)
                : launch(encoded_rows_kernel<false>, dim3(states), dim3(kLanes), stream, args);
}

}  // namespace
}  // namespace gdn

// finish_encoded_projection_launch_v1 (encoded_projection.cpp:964-990).
extern "C" int32_t statecentric_gdn_state_codec_finish_encoded_projection_launch_v1(
    void* stream, const int32_t* projected, const float* dynamic_scale, const uint16_t* input,
    const float* smoothing, const float* scales, const uint16_t* old_left,
    const uint16_t* old_right, const float* record_decay, const uint16_t* record_left,
    const uint16_t* record_right, const uint16_t* new_left, const uint16_t* new_right,
    uint16_t* output, uint32_t states, uint32_t fitted_ranks, uint32_t transpose) {
  if (!projected || !dynamic_scale || !input || !smoothing || !scales || !old_left ||
      !old_right || !record_decay || !record_left || !record_right || !new_left ||
      !new_right || !output || states == 0 || states > gdn::kMaxWindowStates ||
      fitted_ranks > static_cast<uint32_t>(gdn::kRank) || transpose > 1u ||
      !gdn::aligned16(projected, dynamic_scale, input, smoothing, scales, old_left, old_right,
                      record_decay, record_left, record_right, new_left, new_right, output)) {
    return gdn::kStatusInvalidArgument;
  }
  const gdn::RankArgs args{projected, dynamic_scale, input, smoothing, scales, old_left,
                           old_right, record_decay, record_left, record_right,
                           const_cast<uint16_t*>(new_left), const_cast<uint16_t*>(new_right),
                           output, nullptr, fitted_ranks, transpose};
  return gdn::launch_rows(false, args, states, stream);
}

// commit_encoded_rank_launch_v1 (encoded_projection.cpp:992-1015).
extern "C" int32_t statecentric_gdn_state_codec_commit_encoded_rank_launch_v1(
    void* stream, const int32_t* projected, const float* dynamic_scale, const uint16_t* input,
    const float* smoothing, const float* scales, const uint16_t* old_left,
    const uint16_t* old_right, const float* record_decay, const uint16_t* record_left,
    const uint16_t* record_right, uint16_t* new_left, uint16_t* new_right, float* corrected,
    uint32_t states, uint32_t rank) {
  if (!projected || !dynamic_scale || !input || !smoothing || !scales || !old_left ||
      !old_right || !record_decay || !record_left || !record_right || !new_left ||
      !new_right || !corrected || states == 0 || states > gdn::kMaxWindowStates ||
      rank >= static_cast<uint32_t>(gdn::kRank) ||
      !gdn::aligned16(projected, dynamic_scale, input, smoothing, scales, old_left, old_right,
                      record_decay, record_left, record_right, new_left, new_right,
                      corrected)) {
    return gdn::kStatusInvalidArgument;
  }
  const gdn::RankArgs args{projected, dynamic_scale, input, smoothing, scales, old_left,
                           old_right, record_decay, record_left, record_right, new_left,
                           new_right, nullptr, corrected, rank, 0u};
  return gdn::launch_rows(true, args, states, stream);
}
