// The reference's "cube" decode chain for the windowed step, bit-exact:
//   prepare : the read vector r*s and the output vector y*s of a state are each
//             split into a high and a low int8 code with per-state dynamic
//             scales (kernel/gdn_state_codec_encoded_projection.cpp:236-479);
//   project : int32 P[v][c] = sum_k code[v][k] * q[k][c] over the [value][key]
//             boundary codes (kernel/gdn_state_codec_int8_cube_matmul.cpp);
//   finish  : rescale P, add compensator and record terms, correction, output,
//             record append and position update (encoded_projection.cpp:
//             482-776).
// prepare and finish are the reference's scalar fp32 statements: maxima are
// order-free wave reductions, every sequential sum of the reference is run by
// one lane in the reference's row order, and -ffp-contract=off keeps each
// multiply and add separately rounded, so the results equal the CPU statement
// of those kernels bit for bit.  The projection is exact integer arithmetic
// (v_dot4_i32_i8).
//
// decode_runtime_step_v1 runs the three stages as ONE kernel per state: the
// quantized vectors never leave LDS and the codes are read once, the decode
// projection's single-pass layout.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "codec_math.h"
#include "decode_pair.h"
#include "gdn_state_codec_window.h"
#include "lane_exchange.h"
#include "launch.h"
#include "stream_memory.h"
#include "window_common.h"

namespace gdn {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kPairColumns = 16;  // quantized / projected row width

// Vector quantizer rounding of the reference: add +-0.5, clamp, truncate.
__device__ __forceinline__ int pair_round(float value) {
  float r = value + (value >= 0.0f ? 0.5f : -0.5f);
  r = r > 127.0f ? 127.0f : r;
  r = r < -127.0f ? -127.0f : r;
  return static_cast<int>(r);
}

// Two-level split of pair[c][e] (vector c, this lane's rows 2*lane + e).
// codes[c][e] packs the high code in byte 0 and the low code in byte 1;
// scale = {hi0, hi1, lo0, lo1}.
__device__ __forceinline__ void split_pair(const float (&pair)[2][2],
                                           int (&high)[2][2], int (&low)[2][2],
                                           float (&scale)[4]) {
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const float m = wave_max_valu(fmaxf(fabsf(pair[c][0]), fabsf(pair[c][1])));
    scale[c] = m > 1.0e-20f ? m / 127.0f : 1.0f;
  }
  float residual_max[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    float m = 0.0f;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      high[c][e] = pair_round(pair[c][e] / scale[c]);
      const float residual = pair[c][e] - static_cast<float>(high[c][e]) * scale[c];
      m = fmaxf(m, fabsf(residual));
    }
    residual_max[c] = wave_max_valu(m);
  }
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    scale[c + 2] = residual_max[c] > 1.0e-20f ? residual_max[c] / 127.0f : 1.0f;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      low[c][e] = pair_round((pair[c][e] - static_cast<float>(high[c][e]) * scale[c]) /
                             scale[c + 2]);
    }
  }
}

// The vectors one decode step reads: per row, read[k], query[k] (the output
// side before the gate), write[k] (the write key) and the gate.
struct StepVectors {
  float read[2], query[2], write[2];
  float query_raw[2];  // the query before query_scale (bf16) / as given (fp16)
  float gate;
  uint32_t record_key_bits;  // the record key this lane stores (rows 2*lane..+1)
};

// The raw words one lane reads for a step's vectors (rows 2*lane, 2*lane+1),
// without arithmetic, so a kernel can issue them ahead of its bulk loads.
struct VectorWords {
  float decay;     // log decay (bf16 chain) or linear decay (fp16 chain)
  uint32_t beta;   // bf16 bits; 0 when the chain has no beta
  uint32_t key;    // bf16 keys (bf16 chain) or fp16 write keys (fp16 chain)
  uint32_t read;   // fp16 reads (fp16 chain)
  uint32_t query;
};

__device__ __forceinline__ StepVectors bf16_vectors(const VectorWords& w) {
  StepVectors v;
  v.gate = decay_gate(w.decay);
  const float b = bf16_to_float(static_cast<uint16_t>(w.beta));
  uint32_t bits = 0;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const float key = bf16_to_float((w.key >> (16 * e)) & 0xFFFFu);
    v.query_raw[e] = bf16_to_float((w.query >> (16 * e)) & 0xFFFFu);
    v.query[e] = kQueryScale * v.query_raw[e];
    v.read[e] = v.gate * key;
    v.write[e] = b * key;
    bits |= float_to_half_bits(v.write[e]) << (16 * e);
  }
  v.record_key_bits = bits;
  return v;
}

__device__ __forceinline__ StepVectors f16_vectors(const VectorWords& w) {
  StepVectors v;
  v.gate = w.decay;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    v.write[e] = half_bits_to_float((w.key >> (16 * e)) & 0xFFFFu);
    v.read[e] = half_bits_to_float((w.read >> (16 * e)) & 0xFFFFu);
    v.query[e] = half_bits_to_float((w.query >> (16 * e)) & 0xFFFFu);
    v.query_raw[e] = v.query[e];
  }
  v.record_key_bits = w.key;
  return v;
}

// prepare: pair0 = r*s and pair1 = y*s in the reference's expression order:
// bf16 ((g*k)*s, ((query_scale*g)*q)*s; encoded_projection.cpp:390-396),
// fp16 (r*s, (q*g)*s; :265-270).
__device__ __forceinline__ void prepare_pairs(const StepVectors& v, bool bf16, float2 sm,
                                              float (&pair)[2][2]) {
  const float s[2] = {sm.x, sm.y};
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    pair[0][e] = v.read[e] * s[e];
    pair[1][e] = bf16 ? kQueryScale * v.gate * v.query_raw[e] * s[e]
                      : v.query_raw[e] * v.gate * s[e];
  }
}

__device__ __forceinline__ void store_quantized(int8_t* quantized, float* dynamic_scale,
                                                uint32_t state, int lane,
                                                const int (&high)[2][2],
                                                const int (&low)[2][2],
                                                const float (&scale)[4]) {
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const uint32_t word = (static_cast<uint32_t>(high[0][e]) & 0xFFu) |
                          ((static_cast<uint32_t>(low[0][e]) & 0xFFu) << 8) |
                          ((static_cast<uint32_t>(high[1][e]) & 0xFFu) << 16) |
                          ((static_cast<uint32_t>(low[1][e]) & 0xFFu) << 24);
    *reinterpret_cast<uint4*>(quantized + (static_cast<uint64_t>(state) * kDim + 2 * lane + e) *
                                              kPairColumns) = make_uint4(word, 0u, 0u, 0u);
  }
  if (lane == 0) {
    *reinterpret_cast<float4*>(dynamic_scale + static_cast<uint64_t>(state) * kPositionStride) =
        make_float4(scale[0], scale[1], scale[2], scale[3]);
  }
}

// ------------------------------------------------------------------ finish

struct FinishArgs {
  const float* scales;
  const uint16_t* comp_keys;
  const uint16_t* comp_values;
  float* record_decay;
  uint16_t* record_keys;
  uint16_t* record_corrections;
  uint32_t* positions;
  const uint16_t* values;
  void* outputs;
  bool bf16;
};

// Basis rows are padded to 272 bytes: in the sums every lane reads its own
// row at the same column, and a 256-byte stride would put all of them in one
// LDS bank; at 272 bytes any 16 consecutive lanes fall in distinct banks.
constexpr int kBasisStride = kDim + 8;

// LDS a wavefront needs for the finish: the three vectors, the compensator
// and record keys (rows 0..3 and 4..4+p-1), and the 41 sums.
struct FinishShared {
  float read[kDim];
  float query[kDim];
  float write[kDim];
  // Compensator then record keys as fp16 bits (exact; widened when read).
  uint16_t basis[kRank + kWindow][kBasisStride];
  float sums[1 + 2 * kRank + 2 * kWindow];
};

// The key words of one lane: its two keys' four compensator halves and, for
// records j < p, its two record-key halves.
struct KeyWords {
  uint4 comp;
  uint32_t record[kWindow];
};

__device__ __forceinline__ KeyWords load_key_words(const FinishArgs& a, uint32_t state,
                                                   uint32_t p, int lane) {
  const uint64_t vector_base = static_cast<uint64_t>(state) * kDim;
  const uint64_t record_base = static_cast<uint64_t>(state) * kWindow;
  KeyWords k;
  // comp_keys [state][key][4]: this lane's two keys are 8 contiguous halves.
  k.comp = *reinterpret_cast<const uint4*>(a.comp_keys + (vector_base + 2 * lane) * kRank);
#pragma unroll
  for (int j = 0; j < kWindow; ++j) {
    k.record[j] = j < static_cast<int>(p)
        ? *reinterpret_cast<const uint32_t*>(a.record_keys + (record_base + j) * kDim + 2 * lane)
        : 0u;
  }
  return k;
}

// Basis rows 0..3 (compensator keys, transposed to [rank][key]) and
// 4..4+p-1 (record keys).
__device__ __forceinline__ void stage_keys(FinishShared& sh, const KeyWords& k, uint32_t p,
                                           int lane) {
  const uint32_t words[4] = {k.comp.x, k.comp.y, k.comp.z, k.comp.w};
#pragma unroll
  for (int r = 0; r < kRank; ++r) {
    const uint32_t k0 = (words[r >> 1] >> (16 * (r & 1))) & 0xFFFFu;
    const uint32_t k1 = (words[2 + (r >> 1)] >> (16 * (r & 1))) & 0xFFFFu;
    *reinterpret_cast<uint32_t*>(&sh.basis[r][2 * lane]) = k0 | (k1 << 16);
  }
#pragma unroll
  for (int j = 0; j < kWindow; ++j) {
    if (j < static_cast<int>(p)) {
      *reinterpret_cast<uint32_t*>(&sh.basis[kRank + j][2 * lane]) = k.record[j];
    }
  }
}

// Finishes one state at position p < 16 for this lane's two values
// 2*lane, 2*lane+1, given the int32 projections P[e][c] (c = hi0, lo0, hi1,
// lo1) and the dynamic scales.  The per-value operands (scales, compensator
// values, values and the p record corrections) are loaded first, so they are
// in flight during the key staging and the sequential sums.
// kKeysStaged: the caller has already written the basis rows (stage_keys).
template <bool kKeysStaged>
__device__ __forceinline__ void finish_state(const FinishArgs& a, FinishShared& sh,
                             const StepVectors& v, uint32_t state, uint32_t p,
                             int lane, const int32_t (&P)[2][4], const float (&ds)[4],
                             float gate_lane) {
  const uint64_t vector_base = static_cast<uint64_t>(state) * kDim;
  const uint64_t record_base = static_cast<uint64_t>(state) * kWindow;
  const int column0 = 2 * lane;
  const float2 scale = *reinterpret_cast<const float2*>(a.scales + vector_base + column0);
  const uint4 cv = *reinterpret_cast<const uint4*>(a.comp_values + (vector_base + column0) * kRank);
  const uint32_t value_word = *reinterpret_cast<const uint32_t*>(a.values + vector_base + column0);
  uint32_t correction_word[kWindow];
#pragma unroll
  for (int j = 0; j < kWindow; ++j) {
    correction_word[j] = j < static_cast<int>(p)
        ? *reinterpret_cast<const uint32_t*>(a.record_corrections + (record_base + j) * kDim + column0)
        : 0u;
  }
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    sh.read[2 * lane + e] = v.read[e];
    sh.query[2 * lane + e] = v.query[e];
    sh.write[2 * lane + e] = v.write[e];
  }
  if constexpr (!kKeysStaged) stage_keys(sh, load_key_words(a, state, p, lane), p, lane);
  wave_lds_sync();
  // Sequential sums in row order, one per lane: 0 = update, 1..4 = old read
  // projections, 5..8 = old output projections, 9.. = record read projections
  // then record output projections.  Each is the reference's
  // acc += basis * x (read side) or acc += basis * query * gate (output side).
  const int sums = 1 + 2 * kRank + 2 * static_cast<int>(p);
  if (lane < sums) {
    const uint16_t* basis;
    const float* x;
    bool gated;
    if (lane == 0) {
      basis = nullptr;  // the update sum w . q reads sh.write
      x = sh.query;
      gated = false;
    } else if (lane <= 2 * kRank) {
      basis = sh.basis[(lane - 1) & (kRank - 1)];
      gated = lane > kRank;
      x = gated ? sh.query : sh.read;
    } else {
      const int index = lane - 1 - 2 * kRank;
      gated = index >= static_cast<int>(p);
      basis = sh.basis[kRank + (gated ? index - static_cast<int>(p) : index)];
      x = gated ? sh.query : sh.read;
    }
    float acc = 0.0f;
    if (lane == 0) {
#pragma unroll 16
      for (int row = 0; row < kDim; ++row) acc += sh.write[row] * x[row];
    } else {
      // One loop for the read and the output sides (divergent loops would
      // run one after the other): the read side multiplies by 1.0, which
      // leaves every product unchanged.
      const float g = gated ? v.gate : 1.0f;
#pragma unroll 16
      for (int row = 0; row < kDim; ++row) acc += half_bits_to_float(basis[row]) * x[row] * g;
    }
    sh.sums[lane] = acc;
  }
  wave_lds_sync();
  const float update = sh.sums[0];
  // Gate products in descending record order; the 1.0 of lanes j >= p
  // leaves every product unchanged.
  float suffix[kWindow];
  float boundary_suffix = 1.0f;
#pragma unroll
  for (int j = kWindow - 1; j >= 0; --j) {
    suffix[j] = boundary_suffix;
    boundary_suffix *= __builtin_bit_cast(
        float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, gate_lane), j));
  }
  const float value_scale[2] = {scale.x, scale.y};
  const uint32_t comp_words[4] = {cv.x, cv.y, cv.z, cv.w};
  uint32_t output_bits = 0, correction_bits = 0;
  float output_f32[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    float state_read = (static_cast<float>(P[e][0]) * ds[0] +
                        static_cast<float>(P[e][1]) * ds[2]) / 127.0f * value_scale[e] *
                       boundary_suffix;
    float output_read = (static_cast<float>(P[e][2]) * ds[1] +
                         static_cast<float>(P[e][3]) * ds[3]) / 127.0f * value_scale[e] *
                        boundary_suffix;
#pragma unroll
    for (int r = 0; r < kRank; ++r) {
      const float b = half_bits_to_float((comp_words[2 * e + (r >> 1)] >> (16 * (r & 1))) & 0xFFFFu);
      state_read += b * sh.sums[1 + r] * boundary_suffix;
      output_read += b * sh.sums[1 + kRank + r] * boundary_suffix;
    }
#pragma unroll
    for (int j = 0; j < kWindow; ++j) {
      if (j < static_cast<int>(p)) {
        const float b = half_bits_to_float((correction_word[j] >> (16 * e)) & 0xFFFFu);
        state_read += b * sh.sums[1 + 2 * kRank + j] * suffix[j];
        output_read += b * sh.sums[1 + 2 * kRank + p + j] * suffix[j];
      }
    }
    const uint32_t value_bits = (value_word >> (16 * e)) & 0xFFFFu;
    const float value = a.bf16 ? bf16_to_float(static_cast<uint16_t>(value_bits))
                               : half_bits_to_float(value_bits);
    const float correction = value - state_read;
    const float out = output_read + correction * update;
    output_f32[e] = out;
    output_bits |= static_cast<uint32_t>(float_to_bf16(out)) << (16 * e);
    correction_bits |= float_to_half_bits(correction) << (16 * e);
  }
  if (a.bf16) {
    *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(a.outputs) + vector_base + column0) =
        output_bits;
  } else {
    *reinterpret_cast<float2*>(static_cast<float*>(a.outputs) + vector_base + column0) =
        make_float2(output_f32[0], output_f32[1]);
  }
  *reinterpret_cast<uint32_t*>(a.record_corrections + (record_base + p) * kDim + column0) =
      correction_bits;
  *reinterpret_cast<uint32_t*>(a.record_keys + (record_base + p) * kDim + 2 * lane) =
      v.record_key_bits;
  if (lane == 0) {
    a.record_decay[record_base + p] = v.gate;
    a.positions[static_cast<uint64_t>(state) * kPositionStride] = p + 1;
  }
}

// ---------------------------------------------------------------- kernels

struct VectorArgs {
  const uint16_t* keys;     // bf16 keys [S/2][128] or fp16 write keys [S][128]
  const uint16_t* reads;    // fp16 chain only
  const uint16_t* queries;
  const float* decay;       // log (bf16) or linear (fp16)
  const uint16_t* beta;     // bf16 finish only
  uint32_t states;
  bool bf16;
};

__device__ __forceinline__ VectorWords load_vector_words(const VectorArgs& in, uint32_t state,
                                                         int lane) {
  VectorWords w{};
  w.decay = in.decay[state];
  if (in.bf16) {
    w.beta = in.beta != nullptr ? in.beta[state] : 0u;
    const uint64_t head = static_cast<uint64_t>(state >> 1) * kDim + 2 * lane;
    w.key = *reinterpret_cast<const uint32_t*>(in.keys + head);
    w.query = *reinterpret_cast<const uint32_t*>(in.queries + head);
  } else {
    const uint64_t base = static_cast<uint64_t>(state) * kDim + 2 * lane;
    w.key = in.keys != nullptr ? *reinterpret_cast<const uint32_t*>(in.keys + base) : 0u;
    w.read = *reinterpret_cast<const uint32_t*>(in.reads + base);
    w.query = *reinterpret_cast<const uint32_t*>(in.queries + base);
  }
  return w;
}

__device__ __forceinline__ StepVectors vectors_of(const VectorWords& w, bool bf16) {
  return bf16 ? bf16_vectors(w) : f16_vectors(w);
}

__device__ __forceinline__ StepVectors load_vectors(const VectorArgs& in, uint32_t state,
                                                    int lane) {
  return vectors_of(load_vector_words(in, state, lane), in.bf16);
}

__device__ __forceinline__ float2 load_smoothing(const float* smoothing, uint32_t state,
                                                 int lane) {
  return *reinterpret_cast<const float2*>(smoothing + static_cast<uint64_t>(state) * kDim +
                                          2 * lane);
}

// Lane j < p holds record gate j, the other lanes 1.0 (the finish's suffix
// products read it back by readlane).
__device__ __forceinline__ float load_gate_lane(const FinishArgs& a, uint32_t state, uint32_t p,
                                                int lane) {
  return lane < static_cast<int>(p)
             ? a.record_decay[static_cast<uint64_t>(state) * kWindow + lane]
             : 1.0f;
}

__global__ __launch_bounds__(kThreads) void prepare_pair_kernel(
    VectorArgs in, const float* __restrict__ smoothing, int8_t* __restrict__ quantized,
    float* __restrict__ dynamic_scale) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const uint32_t state = blockIdx.x * kWaves + wave;
  if (state >= in.states) return;
  const StepVectors v = load_vectors(in, state, lane);
  float pair[2][2];
  prepare_pairs(v, in.bf16, load_smoothing(smoothing, state, lane), pair);
  int high[2][2], low[2][2];
  float scale[4];
  split_pair(pair, high, low, scale);
  store_quantized(quantized, dynamic_scale, state, lane, high, low, scale);
}

__global__ __launch_bounds__(kThreads) void prepare_vector_kernel(
    const uint16_t* __restrict__ input, const float* __restrict__ axis_scale,
    int8_t* __restrict__ quantized, float* __restrict__ dynamic_scale, uint32_t states) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const uint32_t state = blockIdx.x * kWaves + wave;
  if (state >= states) return;
  float x[2];
  float m = 0.0f;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const uint64_t row = static_cast<uint64_t>(state) * kDim + 2 * lane + e;
    x[e] = half_bits_to_float(input[row * kPairColumns]) * axis_scale[row];
    m = fmaxf(m, fabsf(x[e]));
  }
  m = wave_max_valu(m);
  const float scale = m > 1.0e-20f ? m / 127.0f : 1.0f;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const uint64_t row = static_cast<uint64_t>(state) * kDim + 2 * lane + e;
    const uint32_t code = static_cast<uint32_t>(pair_round(x[e] / scale)) & 0xFFu;
    *reinterpret_cast<uint4*>(quantized + row * kPairColumns) = make_uint4(code, 0u, 0u, 0u);
  }
  if (lane == 0) dynamic_scale[static_cast<uint64_t>(state) * kPositionStride] = scale;
}

// c[s] = a[s] (or a[s]^T) x b[s]: one workgroup per state, thread t computes
// row t/2, columns 8*(t%2)..+7 with v_dot4_i32_i8 over LDS-staged operands.
__global__ __launch_bounds__(kThreads) void int8_matmul_kernel(
    const int8_t* __restrict__ a, const int8_t* __restrict__ b, int32_t* __restrict__ c,
    uint32_t transpose_a) {
  __shared__ __align__(16) uint32_t a_rows[kDim][kDim / 4];        // [m][k/4]
  __shared__ __align__(16) uint32_t b_columns[kPairColumns][kDim / 4];  // [n][k/4]
  const int t = threadIdx.x;
  const uint64_t state = blockIdx.x;
  const int8_t* A = a + state * kTile;
  const int8_t* B = b + state * kDim * kPairColumns;
  // B [k][16] -> b_columns[n][k/4]: thread t packs column n = t & 15, keys
  // 4*(t >> 4)..+3 and 4*(t >> 4) + 64..+3.
  {
    const int n = t & 15;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int k4 = (t >> 4) + 16 * half;
      uint32_t word = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        word |= (static_cast<uint32_t>(static_cast<uint8_t>(B[(4 * k4 + i) * kPairColumns + n]))) << (8 * i);
      }
      b_columns[n][k4] = word;
    }
  }
  if (transpose_a == 0) {
    for (int i = t; i < kDim * kDim / 16; i += kThreads) {
      const uint4 w = reinterpret_cast<const uint4*>(A)[i];
      const int m = i / 8, k16 = i % 8;
      a_rows[m][4 * k16] = w.x;
      a_rows[m][4 * k16 + 1] = w.y;
      a_rows[m][4 * k16 + 2] = w.z;
      a_rows[m][4 * k16 + 3] = w.w;
    }
  } else {
    // a_rows[m][k/4] packs A[k..k+3][m].
    for (int i = t; i < kDim * kDim / 4; i += kThreads) {
      const int m = i % kDim, k4 = i / kDim;
      uint32_t word = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        word |= static_cast<uint32_t>(static_cast<uint8_t>(A[(4 * k4 + j) * kDim + m])) << (8 * j);
      }
      a_rows[m][k4] = word;
    }
  }
  __syncthreads();
  const int m = t >> 1;
  const int n0 = 8 * (t & 1);
  int32_t acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int k4 = 0; k4 < kDim / 4; ++k4) {
    const int aw = static_cast<int>(a_rows[m][k4]);
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      acc[n] = __builtin_amdgcn_sdot4(aw, static_cast<int>(b_columns[n0 + n][k4]), acc[n], false);
    }
  }
  int4* out = reinterpret_cast<int4*>(c + (state * kDim + m) * kPairColumns + n0);
  out[0] = make_int4(acc[0], acc[1], acc[2], acc[3]);
  out[1] = make_int4(acc[4], acc[5], acc[6], acc[7]);
}

__global__ __launch_bounds__(kThreads) void finish_pair_kernel(
    VectorArgs in, FinishArgs fa, const int32_t* __restrict__ projected,
    const float* __restrict__ dynamic_scale) {
  __shared__ FinishShared shared[kWaves];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const uint32_t state = blockIdx.x * kWaves + wave;
  if (state >= in.states) return;
  const uint32_t p = fa.positions[static_cast<uint64_t>(state) * kPositionStride];
  if (p >= kWindow) return;
  const float gate_lane = load_gate_lane(fa, state, p, lane);
  const StepVectors v = load_vectors(in, state, lane);
  int32_t P[2][4];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int4 w = *reinterpret_cast<const int4*>(
        projected + (static_cast<uint64_t>(state) * kDim + 2 * lane + e) * kPairColumns);
    P[e][0] = w.x; P[e][1] = w.y; P[e][2] = w.z; P[e][3] = w.w;
  }
  const float4 d = *reinterpret_cast<const float4*>(dynamic_scale + static_cast<uint64_t>(state) * kPositionStride);
  const float ds[4] = {d.x, d.y, d.z, d.w};
  finish_state<false>(fa, shared[wave], v, state, p, lane, P, ds, gate_lane);
}

// Integer analogue of the decode projection's pairwise lane reduction.
__device__ __forceinline__ void reduce16_over_8_lanes_int(int32_t (&p)[16], int lane) {
#pragma unroll
  for (int i = 0; i < 8; ++i) p[i] = fold<4>(p[i], p[i + 8], lane);
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = fold<2>(p[i], p[i + 4], lane);
#pragma unroll
  for (int i = 0; i < 2; ++i) p[i] = fold<1>(p[i], p[i + 2], lane);
}

// prepare + projection + finish for one state per wavefront.
__global__ __launch_bounds__(kThreads) void fused_decode_pair_kernel(
    VectorArgs in, FinishArgs fa, const int8_t* __restrict__ residual,
    const float* __restrict__ smoothing) {
  __shared__ FinishShared shared[kWaves];
  __shared__ __align__(16) uint32_t qwords[kWaves][4][kDim / 4];  // [c][k/4]
  __shared__ __align__(16) int32_t projected[kWaves][kDim][4];    // [value][c]
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const uint32_t state = blockIdx.x * kWaves + wave;
  if (state >= in.states) return;
  const uint32_t p = fa.positions[static_cast<uint64_t>(state) * kPositionStride];
  if (p >= kWindow) return;

  // The small operands first, then the codes (the bulk of the traffic):
  // memory returns in issue order, so the prepare and the key staging wait
  // only for the small operands while the codes are in flight.  Lane owns
  // keys 16*kq..+15 of value rows r8 + 8j.
  const VectorWords words = load_vector_words(in, state, lane);
  const float2 sm = load_smoothing(smoothing, state, lane);
  const float gate_lane = load_gate_lane(fa, state, p, lane);
  const KeyWords keys = load_key_words(fa, state, p, lane);
  const int kq = lane & 7;
  const int r8 = lane >> 3;
  const int8_t* codes = residual + static_cast<uint64_t>(state) * kTile;
  uint4 row[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    row[j] = stream_load(reinterpret_cast<const uint4*>(codes + (r8 + 8 * j) * kDim + 16 * kq));
  }
  // Keeps the prepare's arithmetic (and its waits) below the code loads.
  __builtin_amdgcn_sched_barrier(0);

  const StepVectors v = vectors_of(words, in.bf16);
  float pair[2][2];
  prepare_pairs(v, in.bf16, sm, pair);
  int high[2][2], low[2][2];
  float ds[4];
  split_pair(pair, high, low, ds);
  stage_keys(shared[wave], keys, p, lane);
  // Column c of the quantized vectors: 0 = hi0, 1 = lo0, 2 = hi1, 3 = lo1.
  // Lane owns rows 2*lane, 2*lane+1: two bytes of word (2*lane)/4.
  {
    uint8_t* bytes = reinterpret_cast<uint8_t*>(&qwords[wave][0][0]);
    const int col_codes[4][2] = {{high[0][0], high[0][1]}, {low[0][0], low[0][1]},
                                 {high[1][0], high[1][1]}, {low[1][0], low[1][1]}};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t pairbits = (static_cast<uint32_t>(col_codes[c][0]) & 0xFFu) |
                                ((static_cast<uint32_t>(col_codes[c][1]) & 0xFFu) << 8);
      *reinterpret_cast<uint16_t*>(bytes + c * kDim + 2 * lane) = static_cast<uint16_t>(pairbits);
    }
  }
  wave_lds_sync();

  // Projection of the codes against the four quantized vectors.
  int qv[4][4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const uint4 w = *reinterpret_cast<const uint4*>(&qwords[wave][c][4 * kq]);
    qv[c][0] = static_cast<int>(w.x);
    qv[c][1] = static_cast<int>(w.y);
    qv[c][2] = static_cast<int>(w.z);
    qv[c][3] = static_cast<int>(w.w);
  }
  int32_t acc[4][16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int words[4] = {static_cast<int>(row[j].x), static_cast<int>(row[j].y),
                          static_cast<int>(row[j].z), static_cast<int>(row[j].w)};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      int s = 0;
#pragma unroll
      for (int m = 0; m < 4; ++m) s = __builtin_amdgcn_sdot4(words[m], qv[c][m], s, false);
      acc[c][j] = s;
    }
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) reduce16_over_8_lanes_int(acc[c], lane);
  // Lane holds values r8 + 8 * (2 * kq + e); the finish wants 2 * lane + e.
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    *reinterpret_cast<int4*>(&projected[wave][r8 + 8 * (2 * kq + e)][0]) =
        make_int4(acc[0][e], acc[1][e], acc[2][e], acc[3][e]);
  }
  wave_lds_sync();
  int32_t P[2][4];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int4 w = *reinterpret_cast<const int4*>(&projected[wave][2 * lane + e][0]);
    P[e][0] = w.x; P[e][1] = w.y; P[e][2] = w.z; P[e][3] = w.w;
  }
  finish_state<true>(fa, shared[wave], v, state, p, lane, P, ds, gate_lane);
}

}  // namespace

int32_t launch_fused_decode_pair_bf16(
    void* stream, const int8_t* residual, const float* smoothing, const float* scales,
    const uint16_t* comp_keys, const uint16_t* comp_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    const float* decay, const uint16_t* beta, const uint16_t* keys,
    const uint16_t* queries, const uint16_t* values, uint16_t* outputs, uint32_t states) {
  const VectorArgs in{keys, nullptr, queries, decay, beta, states, true};
  const FinishArgs fa{scales, comp_keys, comp_values, record_decay, record_keys,
                      record_corrections, positions, values, outputs, true};
  return launch(fused_decode_pair_kernel, dim3((states + kWaves - 1) / kWaves),
                dim3(kThreads), stream, in, fa, residual, smoothing);
}

namespace {

int32_t launch_prepare(void* stream, const VectorArgs& in, const float* smoothing,
                       int8_t* quantized, float* dynamic_scale) {
  return launch(prepare_pair_kernel, dim3((in.states + kWaves - 1) / kWaves), dim3(kThreads),
                stream, in, smoothing, quantized, dynamic_scale);
}

int32_t launch_finish(void* stream, const VectorArgs& in, const FinishArgs& fa,
                      const int32_t* projected, const float* dynamic_scale) {
  return launch(finish_pair_kernel, dim3((in.states + kWaves - 1) / kWaves), dim3(kThreads),
                stream, in, fa, projected, dynamic_scale);
}

}  // namespace
}  // namespace gdn

extern "C" int32_t statecentric_gdn_state_codec_prepare_int8_vector_launch_v1(
    void* stream, const uint16_t* input, const float* axis_scale, int8_t* quantized,
    float* dynamic_scale, uint32_t states) {
  if (!input || !axis_scale || !quantized || !dynamic_scale || states == 0 ||
      states > gdn::kMaxWindowStates ||
      !gdn::aligned16(input, axis_scale, quantized, dynamic_scale)) {
    return gdn::kStatusInvalidArgument;
  }
  return gdn::launch(gdn::prepare_vector_kernel, dim3((states + gdn::kWaves - 1) / gdn::kWaves),
                     dim3(gdn::kThreads), stream, input, axis_scale, quantized,
                     dynamic_scale, states);
}

extern "C" int32_t statecentric_gdn_state_codec_prepare_decode_pair_launch_v1(
    void* stream, const uint16_t* reads, const uint16_t* queries, const float* decay,
    const float* smoothing, int8_t* quantized, float* dynamic_scale, uint32_t states) {
  if (!reads || !queries || !decay || !smoothing || !quantized || !dynamic_scale ||
      states == 0 || states > gdn::kMaxWindowStates ||
      !gdn::aligned16(reads, queries, decay, smoothing, quantized, dynamic_scale)) {
    return gdn::kStatusInvalidArgument;
  }
  const gdn::VectorArgs in{nullptr, reads, queries, decay, nullptr, states, false};
  return gdn::launch_prepare(stream, in, smoothing, quantized, dynamic_scale);
}

extern "C" int32_t statecentric_gdn_state_codec_prepare_decode_pair_bf16_launch_v1(
    void* stream, const uint16_t* keys, const uint16_t* queries, const float* decay,
    const float* smoothing, int8_t* quantized, float* dynamic_scale, uint32_t states) {
  if (!keys || !queries || !decay || !smoothing || !quantized || !dynamic_scale ||
      states == 0 || states > gdn::kMaxWindowStates || states % 2 != 0 ||
      !gdn::aligned16(keys, queries, decay, smoothing, quantized, dynamic_scale)) {
    return gdn::kStatusInvalidArgument;
  }
  const gdn::VectorArgs in{keys, nullptr, queries, decay, nullptr, states, true};
  return gdn::launch_prepare(stream, in, smoothing, quantized, dynamic_scale);
}

extern "C" int32_t statecentric_gdn_state_codec_int8_cube_matmul_launch_v1(
    void* stream, const int8_t* a, const int8_t* b, int32_t* c, uint32_t states,
    uint32_t transpose_a, void* workspace, void* tiling, uint32_t blocks) {
  if (!a || !b || !c || !workspace || !tiling || blocks == 0 || blocks > 64 ||
      states == 0 || states > 128 || blocks != (states + 1u) / 2u || transpose_a > 1u ||
      !gdn::aligned16(a, b, c)) {
    return gdn::kStatusInvalidArgument;
  }
  return gdn::launch(gdn::int8_matmul_kernel, dim3(states), dim3(gdn::kThreads), stream,
                     a, b, c, transpose_a);
}

extern "C" int32_t statecentric_gdn_state_codec_int8_matmul_launch_v4(
    void* stream, const int8_t* a, const int8_t* b, int32_t* c, uint32_t states,
    uint32_t transpose_a) {
  if (!a || !b || !c || states == 0 || states > gdn::kMaxWindowStates || transpose_a > 1u ||
      !gdn::aligned16(a, b, c)) {
    return gdn::kStatusInvalidArgument;
  }
  return gdn::launch(gdn::int8_matmul_kernel, dim3(states), dim3(gdn::kThreads), stream,
                     a, b, c, transpose_a);
}

extern "C" int32_t statecentric_gdn_state_codec_finish_decode_pair_launch_v1(
    void* stream, const int32_t* projected, const float* dynamic_scale, const float* scales,
    const uint16_t* compensator_keys, const uint16_t* compensator_values,
    float* record_decay, uint16_t* record_keys, uint16_t* record_corrections,
    uint32_t* positions, const float* decay, const uint16_t* write_keys,
    const uint16_t* reads, const uint16_t* queries, const uint16_t* values, float* outputs,
    uint32_t states) {
  if (!projected || !dynamic_scale || !scales || !compensator_keys || !compensator_values ||
      !record_decay || !record_keys || !record_corrections || !positions || !decay ||
      !write_keys || !reads || !queries || !values || !outputs || states == 0 ||
      states > gdn::kMaxWindowStates ||
      !gdn::aligned16(projected, dynamic_scale, scales, compensator_keys, compensator_values,
                      record_decay, record_keys, record_corrections, positions, decay,
                      write_keys, reads, queries, values, outputs)) {
    return gdn::kStatusInvalidArgument;
  }
  const gdn::VectorArgs in{write_keys, reads, queries, decay, nullptr, states, false};
  const gdn::FinishArgs fa{scales, compensator_keys, compensator_values, record_decay,
                           record_keys, record_corrections, positions, values, outputs,
                           false};
  return gdn::launch_finish(stream, in, fa, projected, dynamic_scale);
}

extern "C" int32_t statecentric_gdn_state_codec_finish_decode_pair_bf16_launch_v1(
    void* stream, const int32_t* projected, const float* dynamic_scale, const float* scales,
    const uint16_t* compensator_keys, const uint16_t* compensator_values,
    float* record_decay, uint16_t* record_keys, uint16_t* record_corrections,
    uint32_t* positions, const float* decay, const uint16_t* beta, const uint16_t* keys,
    const uint16_t* queries, const uint16_t* values, uint16_t* outputs, uint32_t states) {
  if (!projected || !dynamic_scale || !scales || !compensator_keys || !compensator_values ||
      !record_decay || !record_keys || !record_corrections || !positions || !decay ||
      !beta || !keys || !queries || !values || !outputs || states == 0 ||
      states > gdn::kMaxWindowStates || states % 2 != 0 ||
      !gdn::aligned16(projected, dynamic_scale, scales, compensator_keys, compensator_values,
                      record_decay, record_keys, record_corrections, positions, decay, beta,
                      keys, queries, values, outputs)) {
    return gdn::kStatusInvalidArgument;
  }
  const gdn::VectorArgs in{keys, nullptr, queries, decay, beta, states, true};
  const gdn::FinishArgs fa{scales, compensator_keys, compensator_values, record_decay,
                           record_keys, record_corrections, positions, values, outputs,
                           true};
  return gdn::launch_finish(stream, in, fa, projected, dynamic_scale);
}
