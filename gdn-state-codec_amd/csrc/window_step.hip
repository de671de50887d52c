// Windowed GDN decode step: one token of the gated delta rule evaluated against
// the encoded state (int8 boundary + rank-4 fp16 compensators + up to 15 fp16
// rank-one records), without materializing the dense state.
//
// For a state S (boundary B decayed by the records' gates, plus the records),
// read vector r, output vector y and write key w, the step computes
//   state_read  = S^T r,   output_read = S^T y,
//   correction  = value - state_read,
//   out         = output_read + correction * (w . q),
// and appends the record {gate, w, correction} at the state's window position
// (native/src/gdn_state_codec_state_capsule.cpp:354-397 is the semantics;
// native/ascendc/gdn_state_codec/kernel/gdn_state_codec_windowed_gdn_step.cpp:
// 34-187 (fp16) and :189-619 (bf16) the device entry points).  S^T x expands to
//   (sum_k code[k][v] * s[k] * x[k]) / 127 * scale[v] * suffix
//   + sum_r cv[v][r] * (ck[:, r] . x) * suffix
//   + sum_j corr_j[v] * (key_j . x) * suffix_j,
// where suffix_j is the product of the gates recorded after record j and
// suffix the product of all of them.
//
// One wavefront per state.  Phase 1 spreads the 128 keys over the 64 lanes (two
// each) to form w*s for both readouts, the update, compensator and record
// projections (wave reductions).  Phase 2 reads the 16 KiB of codes once,
// feeding both readouts from the same registers (the decode projection's
// layout), and phase 3 finishes two values per lane.  Everything is fp32; the
// only roundings to 16 bits are the stored records and bf16 outputs, where the
// reference's Ascend kernel also rounds its products and partial sums to fp16.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "codec_math.h"
#include "gdn_state_codec_window.h"
#include "lane_exchange.h"
#include "launch.h"
#include "stream_memory.h"
#include "window_common.h"

namespace gdn {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

enum : int { kStepF16 = 0, kStepBF16 = 1, kStepBF16QuantOnly = 2 };

struct StepArgs {
  const int8_t* residual;
  const float* smoothing;
  const float* scales;
  const uint16_t* comp_keys;
  const uint16_t* comp_values;
  float* record_decay;
  uint16_t* record_keys;
  uint16_t* record_corrections;
  uint32_t* positions;
  const float* decay;      // linear (fp16 step) or log (bf16 steps)
  const uint16_t* beta;    // bf16 steps
  const uint16_t* keys;    // fp16: write keys [S][128]; bf16: keys [S/2][128]
  const uint16_t* reads;   // fp16 step only
  const uint16_t* queries; // fp16: [S][128]; bf16: [S/2][128]
  const uint16_t* values;
  void* outputs;           // fp16 step: float; bf16 steps: bf16 bits
  uint32_t states;
};

__device__ __forceinline__ float code_byte(uint32_t word, int byte) {
  return static_cast<float>(
      static_cast<int8_t>(static_cast<uint8_t>(word >> (8 * byte))));
}

__device__ __forceinline__ uint32_t word_of(const uint4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Pairwise combination over 3 lane bits: 16 partials per lane become 2 per
// lane holding entries 2 * idx + {0, 1}, idx = 4*bit(M2) + 2*bit(M1) + bit(M0).
template <int M2, int M1, int M0>
__device__ __forceinline__ void reduce16_over_8_lanes(float (&p)[16], int lane) {
#pragma unroll
  for (int i = 0; i < 8; ++i) p[i] = fold<M2>(p[i], p[i + 8], lane);
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = fold<M1>(p[i], p[i + 4], lane);
#pragma unroll
  for (int i = 0; i < 2; ++i) p[i] = fold<M0>(p[i], p[i + 2], lane);
}

// Reduce-scatter of N partial sums over the 64 lanes: log2(N) halving steps
// over lane bits 5, 4, ... followed by a plain sum over the remaining low bits
// leave lane L holding the total of value L >> (6 - log2(N)).
template <int N, int kMask>
__device__ __forceinline__ void halve(float* v, int lane) {
  if constexpr (N > 1) {
    constexpr int n = N / 2;
#pragma unroll
    for (int i = 0; i < n; ++i) v[i] = fold<kMask>(v[i], v[i + n], lane);
    halve<n, kMask / 2>(v, lane);
  }
}

template <int kMask>
__device__ __forceinline__ float sum_low_bits(float x) {
  if constexpr (kMask >= 1) return sum_low_bits<kMask / 2>(add_partner<kMask>(x));
  return x;
}

template <int N>
__device__ __forceinline__ float reduce_scatter(float (&v)[N], int lane) {
  halve<N, 32>(v, lane);
  return sum_low_bits<32 / N>(v[0]);
}

constexpr int kEarlyRows = 12;  // code rows issued before phase 1 (of 16)

template <int kVariant>
__global__ __launch_bounds__(kThreads) void window_step_kernel(StepArgs a) {
  constexpr bool kValueKey = kVariant != kStepF16;
  constexpr bool kCompensated = kVariant != kStepBF16QuantOnly;
  __shared__ __align__(16) float weights[kWaves][2][kDim];  // s*read, s*output vector
  __shared__ __align__(16) float readouts[kWaves][2][kDim]; // boundary readouts by value
  // [0, 16): record read-side coefficients, [16, 32): output side,
  // [32, 36) / [36, 40): compensator read / output projections.
  __shared__ float coefficients[kWaves][2 * kWindow + 2 * kRank];
  // Record corrections j < p of this lane's two values, parked from phase 1
  // to phase 3 so that they hold no registers during phase 2.
  __shared__ uint32_t parked_corrections[kWaves][kWindow - 1][64];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const uint32_t state = blockIdx.x * kWaves + wave;
  if (state >= a.states) return;  // whole wavefront; only wave-level syncs below
  const uint32_t p = a.positions[static_cast<uint64_t>(state) * kPositionStride];
  if (p >= kWindow) return;  // full window: the boundary refit comes first

  const uint64_t vector_base = static_cast<uint64_t>(state) * kDim;
  const uint64_t record_base = static_cast<uint64_t>(state) * kWindow;
  const int k0 = 2 * lane;  // this lane's two keys, and (phase 3) its two values

  // ---- loads, in the order they are consumed: memory returns in issue order,
  // so phase 1 waits only for its own operands while the 16 KiB of codes is
  // still in flight.
  uint32_t vec_a, vec_b, vec_c = 0;
  float g, beta = 0.0f;
  if constexpr (kVariant == kStepF16) {
    g = a.decay[state];
    vec_a = *reinterpret_cast<const uint32_t*>(a.keys + vector_base + k0);     // write keys
    vec_b = *reinterpret_cast<const uint32_t*>(a.queries + vector_base + k0);
    vec_c = *reinterpret_cast<const uint32_t*>(a.reads + vector_base + k0);
  } else {
    g = decay_gate(a.decay[state]);
    beta = bf16_to_float(a.beta[state]);
    const uint64_t head = static_cast<uint64_t>(state >> 1) * kDim + k0;
    vec_a = *reinterpret_cast<const uint32_t*>(a.keys + head);
    vec_b = *reinterpret_cast<const uint32_t*>(a.queries + head);
  }
  const float2 sm = *reinterpret_cast<const float2*>(a.smoothing + vector_base + k0);
  uint32_t record_key[kWindow];
#pragma unroll
  for (int j = 0; j < kWindow; ++j) {
    record_key[j] = j < static_cast<int>(p)
        ? *reinterpret_cast<const uint32_t*>(a.record_keys + (record_base + j) * kDim + k0)
        : 0u;
  }
  uint4 comp_key = make_uint4(0u, 0u, 0u, 0u);
  if constexpr (kCompensated) {
    comp_key = *reinterpret_cast<const uint4*>(a.comp_keys + (vector_base + k0) * kRank);
  }
  // Lane j < p holds gate j (one load, issued before the codes so that phase 1
  // does not wait for them); the other lanes hold 1.0.
  const float gate_lane = lane < static_cast<int>(p) ? a.record_decay[record_base + lane] : 1.0f;
  // Phase-3 record corrections for values k0, k0+1: loaded before the codes
  // too, and parked in LDS by phase 1.
  uint32_t correction_word[kWindow - 1];
#pragma unroll
  for (int j = 0; j < kWindow - 1; ++j) {
    correction_word[j] = j < static_cast<int>(p)
        ? *reinterpret_cast<const uint32_t*>(a.record_corrections + (record_base + j) * kDim + k0)
        : 0u;
  }
  // Lane (c, r) = (lane & 7, lane >> 3) reads bytes 16c..16c+15 of rows r + 8j.
  const int8_t* codes = a.residual + static_cast<uint64_t>(state) * kTile;
  const int chunk = lane & 7;
  const int row8 = lane >> 3;
  // Rows 0..11 now, rows 12..15 after phase 1: with all 16 in flight through
  // phase 1 the kernel needs more than 128 VGPRs and runs 3 wavefronts per
  // SIMD instead of 4.
  uint4 row[16];
#pragma unroll
  for (int j = 0; j < kEarlyRows; ++j) {
    row[j] = stream_load(reinterpret_cast<const uint4*>(codes + (row8 + 8 * j) * kDim + 16 * chunk));
  }
  // The loads above are issued before any phase-1 arithmetic: without this barrier
  // the scheduler hoists phase-1 math, with its waits for the small operands,
  // above the code loads, and the 16 KiB stream starts a round trip late.
  __builtin_amdgcn_sched_barrier(0);

  // ---- phase 1: vectors, update, compensator and record projections --------
#pragma unroll
  for (int j = 0; j < kWindow - 1; ++j) {
    if (j < static_cast<int>(p)) parked_corrections[wave][j][lane] = correction_word[j];
  }
  float read0, read1, out0, out1, write0, write1, query0, query1;
  uint32_t record_key_bits;
  if constexpr (kVariant == kStepF16) {
    write0 = half_bits_to_float(vec_a & 0xFFFFu);
    write1 = half_bits_to_float(vec_a >> 16);
    query0 = half_bits_to_float(vec_b & 0xFFFFu);
    query1 = half_bits_to_float(vec_b >> 16);
    read0 = half_bits_to_float(vec_c & 0xFFFFu);
    read1 = half_bits_to_float(vec_c >> 16);
    record_key_bits = vec_a;
  } else {
    const float key0 = bf16_to_float(vec_a & 0xFFFFu);
    const float key1 = bf16_to_float(vec_a >> 16);
    query0 = kQueryScale * bf16_to_float(vec_b & 0xFFFFu);
    query1 = kQueryScale * bf16_to_float(vec_b >> 16);
    read0 = g * key0;
    read1 = g * key1;
    write0 = beta * key0;
    write1 = beta * key1;
    record_key_bits = float_to_half_bits(write0) | (float_to_half_bits(write1) << 16);
  }
  out0 = query0 * g;
  out1 = query1 * g;
  *reinterpret_cast<float2*>(&weights[wave][0][k0]) = make_float2(sm.x * read0, sm.y * read1);
  *reinterpret_cast<float2*>(&weights[wave][1][k0]) = make_float2(sm.x * out0, sm.y * out1);
  const float update = wave_sum_valu(write0 * query0 + write1 * query1);

  // Gate products in descending record order, the 1.0 of lanes j >= p leaving
  // every product unchanged: boundary_suffix = prod_i gate_i, and
  // lane_suffix = prod_{i > j} gate_i for the record j = (lane >> 1) & 15
  // whose coefficient this lane scales.
  const int lane_record = (lane >> 1) & (kWindow - 1);
  float boundary_suffix = 1.0f;
  float lane_suffix = 1.0f;
#pragma unroll
  for (int j = kWindow - 1; j >= 0; --j) {
    if (j == lane_record) lane_suffix = boundary_suffix;
    boundary_suffix *= __builtin_bit_cast(
        float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, gate_lane), j));
  }

  // Record projections key_j . read and key_j . (q*g): 32 partials, one
  // reduce-scatter; lane L ends with value L >> 1.
  {
    float partial[2 * kWindow];
#pragma unroll
    for (int j = 0; j < kWindow; ++j) {
      const float b0 = half_bits_to_float(record_key[j] & 0xFFFFu);
      const float b1 = half_bits_to_float(record_key[j] >> 16);
      partial[j] = b0 * read0 + b1 * read1;
      partial[kWindow + j] = b0 * out0 + b1 * out1;
    }
    const float total = reduce_scatter(partial, lane);
    if ((lane & 1) == 0) coefficients[wave][lane >> 1] = total * lane_suffix;
  }
  if constexpr (kCompensated) {
    const uint32_t words[4] = {comp_key.x, comp_key.y, comp_key.z, comp_key.w};
    float partial[2 * kRank];
#pragma unroll
    for (int r = 0; r < kRank; ++r) {
      const float b0 = half_bits_to_float((words[r >> 1] >> (16 * (r & 1))) & 0xFFFFu);
      const float b1 = half_bits_to_float((words[2 + (r >> 1)] >> (16 * (r & 1))) & 0xFFFFu);
      partial[r] = b0 * read0 + b1 * read1;
      partial[kRank + r] = b0 * out0 + b1 * out1;
    }
    const float total = reduce_scatter(partial, lane);  // lane L: value L >> 3
    if ((lane & 7) == 0) coefficients[wave][2 * kWindow + (lane >> 3)] = total * boundary_suffix;
  }

#pragma unroll
  for (int j = kEarlyRows; j < 16; ++j) {
    row[j] = stream_load(reinterpret_cast<const uint4*>(codes + (row8 + 8 * j) * kDim + 16 * chunk));
  }
  // Phase-3 operands for values k0, k0+1, in flight during phase 2.
  const float2 scale = *reinterpret_cast<const float2*>(a.scales + vector_base + k0);
  const uint32_t value_word = *reinterpret_cast<const uint32_t*>(a.values + vector_base + k0);
  uint4 comp_value = make_uint4(0u, 0u, 0u, 0u);
  if constexpr (kCompensated) {
    comp_value = *reinterpret_cast<const uint4*>(a.comp_values + (vector_base + k0) * kRank);
  }
  wave_lds_sync();

  // ---- phase 2: both boundary readouts from the codes in registers ---------
  float acc_read[16], acc_out[16];
  if constexpr (kValueKey) {
    // codes [value][key]: lane owns keys 16*chunk..+15 of value rows row8 + 8j.
    float wr[16], wo[16];
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      const float4 x = *reinterpret_cast<const float4*>(&weights[wave][0][16 * chunk + i]);
      const float4 y = *reinterpret_cast<const float4*>(&weights[wave][1][16 * chunk + i]);
      wr[i] = x.x; wr[i + 1] = x.y; wr[i + 2] = x.z; wr[i + 3] = x.w;
      wo[i] = y.x; wo[i + 1] = y.y; wo[i + 2] = y.z; wo[i + 3] = y.w;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      float ar = 0.0f, ao = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float c = code_byte(word_of(row[j], i >> 2), i & 3);
        ar = fmaf(c, wr[i], ar);
        ao = fmaf(c, wo[i], ao);
      }
      acc_read[j] = ar;
      acc_out[j] = ao;
    }
    reduce16_over_8_lanes<4, 2, 1>(acc_read, lane);
    reduce16_over_8_lanes<4, 2, 1>(acc_out, lane);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int v = row8 + 8 * (2 * chunk + e);
      readouts[wave][0][v] = acc_read[e];
      readouts[wave][1][v] = acc_out[e];
    }
  } else {
    // codes [key][value]: lane owns values 16*chunk..+15 of key rows row8 + 8j.
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      acc_read[i] = 0.0f;
      acc_out[i] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float wr = weights[wave][0][row8 + 8 * j];
      const float wo = weights[wave][1][row8 + 8 * j];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float c = code_byte(word_of(row[j], i >> 2), i & 3);
        acc_read[i] = fmaf(c, wr, acc_read[i]);
        acc_out[i] = fmaf(c, wo, acc_out[i]);
      }
    }
    reduce16_over_8_lanes<32, 16, 8>(acc_read, lane);
    reduce16_over_8_lanes<32, 16, 8>(acc_out, lane);
    // values 16*chunk + 2*row8 + {0, 1}: adjacent, one 8-byte LDS store each.
    const int v = 16 * chunk + 2 * row8;
    *reinterpret_cast<float2*>(&readouts[wave][0][v]) = make_float2(acc_read[0], acc_read[1]);
    *reinterpret_cast<float2*>(&readouts[wave][1][v]) = make_float2(acc_out[0], acc_out[1]);
  }
  wave_lds_sync();

  // ---- phase 3: finish values k0, k0+1 --------------------------------------
  const float2 sr = *reinterpret_cast<const float2*>(&readouts[wave][0][k0]);
  const float2 so = *reinterpret_cast<const float2*>(&readouts[wave][1][k0]);
  const float boundary_read[2] = {sr.x, sr.y};
  const float boundary_out[2] = {so.x, so.y};
  const float value_scale[2] = {scale.x, scale.y};
  const uint32_t comp_words[4] = {comp_value.x, comp_value.y, comp_value.z, comp_value.w};
  uint32_t output_bits = 0, correction_bits = 0;
  float output_f32[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const float factor = value_scale[e] * boundary_suffix * kInvQuantizedMaximum;
    float state_read = boundary_read[e] * factor;
    float output_read = boundary_out[e] * factor;
    if constexpr (kCompensated) {
#pragma unroll
      for (int r = 0; r < kRank; ++r) {
        const float b = half_bits_to_float(
            (comp_words[2 * e + (r >> 1)] >> (16 * (r & 1))) & 0xFFFFu);
        state_read = fmaf(b, coefficients[wave][2 * kWindow + r], state_read);
        output_read = fmaf(b, coefficients[wave][2 * kWindow + kRank + r], output_read);
      }
    }
#pragma unroll
    for (int j = 0; j < kWindow - 1; ++j) {
      if (j < static_cast<int>(p)) {
        const uint32_t word = parked_corrections[wave][j][lane];
        const float c = half_bits_to_float((word >> (16 * e)) & 0xFFFFu);
        state_read = fmaf(c, coefficients[wave][j], state_read);
        output_read = fmaf(c, coefficients[wave][kWindow + j], output_read);
      }
    }
    float value;
    if constexpr (kVariant == kStepF16) {
      value = half_bits_to_float((value_word >> (16 * e)) & 0xFFFFu);
    } else {
      value = bf16_to_float((value_word >> (16 * e)) & 0xFFFFu);
    }
    const float correction = value - state_read;
    const float out = fmaf(correction, update, output_read);
    output_f32[e] = out;
    output_bits |= static_cast<uint32_t>(float_to_bf16(out)) << (16 * e);
    correction_bits |= float_to_half_bits(correction) << (16 * e);
  }
  if constexpr (kVariant == kStepF16) {
    *reinterpret_cast<float2*>(static_cast<float*>(a.outputs) + vector_base + k0) =
        make_float2(output_f32[0], output_f32[1]);
  } else {
    *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(a.outputs) + vector_base + k0) =
        output_bits;
  }
  *reinterpret_cast<uint32_t*>(a.record_corrections + (record_base + p) * kDim + k0) =
      correction_bits;
  *reinterpret_cast<uint32_t*>(a.record_keys + (record_base + p) * kDim + k0) = record_key_bits;
  if (lane == 0) {
    a.record_decay[record_base + p] = g;
    a.positions[static_cast<uint64_t>(state) * kPositionStride] = p + 1;
  }
}

template <int kVariant>
int32_t launch_step(void* stream, const StepArgs& args) {
  const dim3 grid((args.states + kWaves - 1) / kWaves);
  return launch(window_step_kernel<kVariant>, grid, dim3(kThreads), stream, args);
}

}  // namespace
}  // namespace gdn

using gdn::StepArgs;

extern "C" int32_t statecentric_gdn_state_codec_windowed_gdn_step_launch_v1(
    void* stream, const int8_t* residual, const float* smoothing,
    const float* scales, const uint16_t* compensator_keys,
    const uint16_t* compensator_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    const float* decay, const uint16_t* write_keys, const uint16_t* reads,
    const uint16_t* queries, const uint16_t* values, float* outputs,
    uint32_t states) {
  if (!residual || !smoothing || !scales || !compensator_keys ||
      !compensator_values || !record_decay || !record_keys ||
      !record_corrections || !positions || !decay || !write_keys || !reads ||
      !queries || !values || !outputs || states == 0 ||
      states > gdn::kMaxWindowStates ||
      !gdn::aligned16(residual, smoothing, scales, compensator_keys, compensator_values,
                      record_decay, record_keys, record_corrections, positions, decay,
                      write_keys, reads, queries, values, outputs)) {
    return gdn::kStatusInvalidArgument;
  }
  const StepArgs args{residual, smoothing, scales, compensator_keys,
                      compensator_values, record_decay, record_keys,
                      record_corrections, positions, decay, nullptr, write_keys,
                      reads, queries, values, outputs, states};
  return gdn::launch_step<gdn::kStepF16>(stream, args);
}

namespace {

int32_t bf16_step(void* stream, const int8_t* residual, const float* smoothing,
                  const float* scales, const uint16_t* compensator_keys,
                  const uint16_t* compensator_values, float* record_decay,
                  uint16_t* record_keys, uint16_t* record_corrections,
                  uint32_t* positions, const float* decay, const uint16_t* beta,
                  const uint16_t* keys, const uint16_t* queries,
                  const uint16_t* values, uint16_t* outputs, uint32_t states,
                  bool quant_only) {
  if (!residual || !smoothing || !scales || !compensator_keys ||
      !compensator_values || !record_decay || !record_keys ||
      !record_corrections || !positions || !decay || !beta || !keys ||
      !queries || !values || !outputs || states == 0 ||
      states > gdn::kMaxWindowStates || states % 2 != 0 ||
      !gdn::aligned16(residual, smoothing, scales, compensator_keys, compensator_values,
                      record_decay, record_keys, record_corrections, positions, decay, beta,
                      keys, queries, values, outputs)) {
    return gdn::kStatusInvalidArgument;
  }
  const StepArgs args{residual, smoothing, scales, compensator_keys,
                      compensator_values, record_decay, record_keys,
                      record_corrections, positions, decay, beta, keys,
                      nullptr, queries, values, outputs, states};
  return quant_only ? gdn::launch_step<gdn::kStepBF16QuantOnly>(stream, args)
                    : gdn::launch_step<gdn::kStepBF16>(stream, args);
}

}  // namespace

extern "C" int32_t statecentric_gdn_state_codec_windowed_gdn_step_bf16_launch_v1(
    void* stream, const int8_t* residual, const float* smoothing,
    const float* scales, const uint16_t* compensator_keys,
    const uint16_t* compensator_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    const float* decay, const uint16_t* beta, const uint16_t* keys,
    const uint16_t* queries, const uint16_t* values, uint16_t* outputs,
    uint32_t states) {
  return bf16_step(stream, residual, smoothing, scales, compensator_keys,
                   compensator_values, record_decay, record_keys,
                   record_corrections, positions, decay, beta, keys, queries,
                   values, outputs, states, false);
}

extern "C" int32_t
statecentric_gdn_state_codec_windowed_gdn_step_bf16_quant_only_launch_v1(
    void* stream, const int8_t* residual, const float* smoothing,
    const float* scales, const uint16_t* compensator_keys,
    const uint16_t* compensator_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    const float* decay, const uint16_t* beta, const uint16_t* keys,
    const uint16_t* queries, const uint16_t* values, uint16_t* outputs,
    uint32_t states) {
  return bf16_step(stream, residual, smoothing, scales, compensator_keys,
                   compensator_values, record_decay, record_keys,
                   record_corrections, positions, decay, beta, keys, queries,
                   values, outputs, states, true);
}
