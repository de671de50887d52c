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
// lane holding entries 2 * idx + {0, 1}, idx = 4*bit(m2) + 2*bit(m1) + bit(m0).
__device__ __forceinline__ void reduce16_over_8_lanes(float (&p)[16], int lane,
                                                      int m2, int m1, int m0) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const bool up = (lane & m2) != 0;
    const float send = up ? p[i] : p[i + 8];
    const float keep = up ? p[i + 8] : p[i];
    p[i] = keep + __shfl_xor(send, m2);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool up = (lane & m1) != 0;
    const float send = up ? p[i] : p[i + 4];
    const float keep = up ? p[i + 4] : p[i];
    p[i] = keep + __shfl_xor(send, m1);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const bool up = (lane & m0) != 0;
    const float send = up ? p[i] : p[i + 2];
    const float keep = up ? p[i + 2] : p[i];
    p[i] = keep + __shfl_xor(send, m0);
  }
}

template <int kVariant>
__global__ __launch_bounds__(kThreads) void window_step_kernel(StepArgs a) {
  constexpr bool kValueKey = kVariant != kStepF16;
  constexpr bool kCompensated = kVariant != kStepBF16QuantOnly;
  __shared__ __align__(16) float weights[kWaves][2][kDim];  // s*read, s*output vector
  __shared__ float coefficients[kWaves][2][kWindow];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const uint32_t state = blockIdx.x * kWaves + wave;
  if (state >= a.states) return;  // whole wavefront; only wave-level syncs below
  const uint32_t p = a.positions[static_cast<uint64_t>(state) * kPositionStride];
  if (p >= kWindow) return;  // full window: the boundary refit comes first

  const uint64_t vector_base = static_cast<uint64_t>(state) * kDim;
  const uint64_t record_base = static_cast<uint64_t>(state) * kWindow;

  // ---- phase 1: vectors, update, compensator and record projections --------
  const int k0 = 2 * lane;
  float g, read0, read1, out0, out1, write0, write1, query0, query1;
  uint32_t record_key_bits;
  if constexpr (kVariant == kStepF16) {
    g = a.decay[state];
    const uint32_t wk = *reinterpret_cast<const uint32_t*>(a.keys + vector_base + k0);
    const uint32_t rd = *reinterpret_cast<const uint32_t*>(a.reads + vector_base + k0);
    const uint32_t qr = *reinterpret_cast<const uint32_t*>(a.queries + vector_base + k0);
    write0 = half_bits_to_float(wk & 0xFFFFu);
    write1 = half_bits_to_float(wk >> 16);
    read0 = half_bits_to_float(rd & 0xFFFFu);
    read1 = half_bits_to_float(rd >> 16);
    query0 = half_bits_to_float(qr & 0xFFFFu);
    query1 = half_bits_to_float(qr >> 16);
    out0 = query0 * g;
    out1 = query1 * g;
    record_key_bits = wk;
  } else {
    g = decay_gate(a.decay[state]);
    const float beta = bf16_to_float(a.beta[state]);
    const uint64_t head = static_cast<uint64_t>(state >> 1) * kDim + k0;
    const uint32_t kw = *reinterpret_cast<const uint32_t*>(a.keys + head);
    const uint32_t qw = *reinterpret_cast<const uint32_t*>(a.queries + head);
    const float key0 = bf16_to_float(kw & 0xFFFFu);
    const float key1 = bf16_to_float(kw >> 16);
    query0 = kQueryScale * bf16_to_float(qw & 0xFFFFu);
    query1 = kQueryScale * bf16_to_float(qw >> 16);
    read0 = g * key0;
    read1 = g * key1;
    out0 = query0 * g;
    out1 = query1 * g;
    write0 = beta * key0;
    write1 = beta * key1;
    record_key_bits = float_to_half_bits(write0) | (float_to_half_bits(write1) << 16);
  }
  {
    const float2 sm = *reinterpret_cast<const float2*>(a.smoothing + vector_base + k0);
    *reinterpret_cast<float2*>(&weights[wave][0][k0]) = make_float2(sm.x * read0, sm.y * read1);
    *reinterpret_cast<float2*>(&weights[wave][1][k0]) = make_float2(sm.x * out0, sm.y * out1);
  }
  const float update = wave_sum(write0 * query0 + write1 * query1);

  // Gate products: suffix_j = prod_{i > j} gate_i over the p stored records.
  float boundary_suffix = 1.0f;
  float suffix[kWindow];
#pragma unroll
  for (int j = kWindow - 1; j >= 0; --j) {
    suffix[j] = boundary_suffix;
    if (j < static_cast<int>(p)) boundary_suffix *= a.record_decay[record_base + j];
  }

  float comp_read[kRank], comp_out[kRank];
  if constexpr (kCompensated) {
    // comp_keys [state][key][4]: this lane's two keys are 8 contiguous halves.
    const uint4 ck = *reinterpret_cast<const uint4*>(a.comp_keys + (vector_base + k0) * kRank);
    const uint32_t words[4] = {ck.x, ck.y, ck.z, ck.w};
#pragma unroll
    for (int r = 0; r < kRank; ++r) {
      const float b0 = half_bits_to_float((words[r >> 1] >> (16 * (r & 1))) & 0xFFFFu);
      const float b1 = half_bits_to_float((words[2 + (r >> 1)] >> (16 * (r & 1))) & 0xFFFFu);
      comp_read[r] = wave_sum(b0 * read0 + b1 * read1) * boundary_suffix;
      comp_out[r] = wave_sum(b0 * out0 + b1 * out1) * boundary_suffix;
    }
  }
#pragma unroll
  for (int j = 0; j < kWindow; ++j) {
    if (j < static_cast<int>(p)) {
      const uint32_t rk = *reinterpret_cast<const uint32_t*>(
          a.record_keys + (record_base + j) * kDim + k0);
      const float b0 = half_bits_to_float(rk & 0xFFFFu);
      const float b1 = half_bits_to_float(rk >> 16);
      const float pr = wave_sum(b0 * read0 + b1 * read1) * suffix[j];
      const float po = wave_sum(b0 * out0 + b1 * out1) * suffix[j];
      if (lane == 0) {
        coefficients[wave][0][j] = pr;
        coefficients[wave][1][j] = po;
      }
    }
  }
  wave_lds_sync();

  // ---- phase 2: both boundary readouts from one pass over the codes --------
  float acc_read[16], acc_out[16];
  int value_of[2];
  const int8_t* codes = a.residual + static_cast<uint64_t>(state) * kTile;
  if constexpr (kValueKey) {
    // codes [value][key]: lane owns keys 16*kq..+15 of value rows r8 + 8j.
    const int kq = lane & 7;
    const int r8 = lane >> 3;
    uint4 row[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      row[j] = stream_load(reinterpret_cast<const uint4*>(codes + (r8 + 8 * j) * kDim + 16 * kq));
    }
    float wr[16], wo[16];
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      const float4 x = *reinterpret_cast<const float4*>(&weights[wave][0][16 * kq + i]);
      const float4 y = *reinterpret_cast<const float4*>(&weights[wave][1][16 * kq + i]);
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
    reduce16_over_8_lanes(acc_read, lane, 4, 2, 1);
    reduce16_over_8_lanes(acc_out, lane, 4, 2, 1);
    value_of[0] = r8 + 8 * (2 * kq);
    value_of[1] = r8 + 8 * (2 * kq + 1);
  } else {
    // codes [key][value]: lane owns values 16*vc..+15 of key rows kr + 8j.
    const int vc = lane & 7;
    const int kr = lane >> 3;
    uint4 row[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      row[j] = stream_load(reinterpret_cast<const uint4*>(codes + (kr + 8 * j) * kDim + 16 * vc));
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      acc_read[i] = 0.0f;
      acc_out[i] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float wr = weights[wave][0][kr + 8 * j];
      const float wo = weights[wave][1][kr + 8 * j];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float c = code_byte(word_of(row[j], i >> 2), i & 3);
        acc_read[i] = fmaf(c, wr, acc_read[i]);
        acc_out[i] = fmaf(c, wo, acc_out[i]);
      }
    }
    reduce16_over_8_lanes(acc_read, lane, 32, 16, 8);
    reduce16_over_8_lanes(acc_out, lane, 32, 16, 8);
    value_of[0] = 16 * vc + 2 * kr;
    value_of[1] = 16 * vc + 2 * kr + 1;
  }

  // ---- phase 3: finish two values per lane ----------------------------------
  uint16_t* correction_out = a.record_corrections + (record_base + p) * kDim;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int v = value_of[e];
    const float factor = a.scales[vector_base + v] * boundary_suffix * kInvQuantizedMaximum;
    float state_read = acc_read[e] * factor;
    float output_read = acc_out[e] * factor;
    if constexpr (kCompensated) {
      const uint2 cv = *reinterpret_cast<const uint2*>(a.comp_values + (vector_base + v) * kRank);
#pragma unroll
      for (int r = 0; r < kRank; ++r) {
        const float b = half_bits_to_float(((r < 2 ? cv.x : cv.y) >> (16 * (r & 1))) & 0xFFFFu);
        state_read = fmaf(b, comp_read[r], state_read);
        output_read = fmaf(b, comp_out[r], output_read);
      }
    }
#pragma unroll
    for (int j = 0; j < kWindow; ++j) {
      if (j < static_cast<int>(p)) {
        const float c = half_bits_to_float(a.record_corrections[(record_base + j) * kDim + v]);
        state_read = fmaf(c, coefficients[wave][0][j], state_read);
        output_read = fmaf(c, coefficients[wave][1][j], output_read);
      }
    }
    float value;
    if constexpr (kVariant == kStepF16) {
      value = half_bits_to_float(a.values[vector_base + v]);
    } else {
      value = bf16_to_float(a.values[vector_base + v]);
    }
    const float correction = value - state_read;
    const float out = fmaf(correction, update, output_read);
    if constexpr (kVariant == kStepF16) {
      static_cast<float*>(a.outputs)[vector_base + v] = out;
    } else {
      static_cast<uint16_t*>(a.outputs)[vector_base + v] = float_to_bf16(out);
    }
    correction_out[v] = static_cast<uint16_t>(float_to_half_bits(correction));
  }
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
      states > gdn::kMaxWindowStates) {
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
      states > gdn::kMaxWindowStates || states % 2 != 0) {
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
