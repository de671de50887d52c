// The device rank-4 chain over an encoded boundary, whole, in one launch.
//
// The reference drives this chain from the host, one stage per launch
// (host/gdn_state_codec_encoded_projection_probe.cpp:611-636): for each rank
// r = 0..3 the seed vector is copied in, then `iterations` times the vector
// is projected through the int8 boundary and finished forward and transposed
// (prepare_int8_vector -> int8_cube_matmul -> finish_encoded_projection, with
// r fitted ranks), and the last vector is projected once more and committed
// as rank r (commit_encoded_rank).  Every stage reads and writes [S][128][16]
// device vectors of which one column is used.
//
// Here one 256-thread workgroup owns one state for the whole chain.  The
// state's int8 boundary is read from HBM once, into registers in both
// orientations (thread t holds 64 codes of row t/2 and 64 codes of column
// t/2); the bases, records, scales and the vector live in LDS; and each stage
// is the reference's arithmetic in the reference's order, so every output is
// bit-identical to the launch-per-stage chain (the stages are restated from
// the kernels in decode_pair.hip and encoded_rank.hip):
//   prepare : x = fp16(v) * axis, scale = max|x| > 1e-20 ? max|x| / 127 : 1,
//             q = round(x / scale) (add +-0.5, clamp to +-127, truncate);
//   product : p = A q or A^T q, exact in int32 (v_dot4_i32_i8);
//   finish  : the 24 coefficient sums (old ranks, fitted ranks, records) as
//             sequential fp32 sums, the rows' value with the window's gates,
//             the sequential squared norm, its 20-step Newton square root and
//             the fp16 output v / |v|;
//   commit  : the rows' value written as the rank's left basis (fp16) and as
//             the corrected vector (fp32), the vector as its right basis.
// The sequential stages (prepare, finish, commit) run in one wavefront, and
// the role moves to the next wavefront at every stage so that the four SIMDs
// of a CU share them; the product uses all four.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gdn_state_codec_window.h"
#include "lane_exchange.h"
#include "launch.h"
#include "window_common.h"

namespace gdn {
namespace {

constexpr int kChainThreads = 256;
constexpr int kChainWaves = kChainThreads / 64;
constexpr int kChainLanes = 64;
constexpr int kCoefficientRows = 2 * kRank + kWindow;  // old, fitted, records
constexpr uint32_t kMaxChainIterations = 64;

struct ChainArgs {
  const int8_t* residual;       // [S][128 left][128 right]
  const float* smoothing;       // [S][128] (left axis)
  const float* scales;          // [S][128] (right axis)
  const uint16_t* old_left;     // fp16 [S][128][4]
  const uint16_t* old_right;    // fp16 [S][128][4]
  const float* record_decay;    // [S][16]
  const uint16_t* record_left;  // fp16 [S][16][128]
  const uint16_t* record_right;
  const uint16_t* seeds;        // fp16 [S][4][128]
  uint16_t* new_left;           // fp16 [S][4][128]
  uint16_t* new_right;          // fp16 [S][4][128]
  float* corrected;             // [S][4][128]
  uint32_t iterations;
};

// Side 0 is the right (value / scale) axis, side 1 the left (key / smoothing)
// axis.  A finish with transpose T takes its input on side T and writes on
// side 1 - T; the forward product (T = 0) maps a right-side vector to the
// left side.
// Basis rows are padded to 132 fp16 (66 words): the 24 coefficient lanes,
// each reading 8 bytes of its own row, then start on banks 2c and hit 48
// distinct banks; unpadded 256-byte rows put all 24 on one bank.
constexpr int kBasisStride = kDim + 4;

struct ChainShared {
  // basis[side][row][dim], fp16: rows 0..3 the old compensators of that side
  // (transposed from [dim][rank]), 4..7 the fitted ranks, 8..23 the records.
  uint16_t basis[2][kCoefficientRows][kBasisStride];
  float axis[2][kDim];
  float decay[kWindow];
  __attribute__((aligned(16))) uint16_t vector[kDim];  // the current vector, fp16 bits
  __attribute__((aligned(16))) uint32_t q[kDim / 4];  // the quantized vector
  int32_t p[kDim];        // the projection
  __attribute__((aligned(16))) float values[kDim];  // the rows' values, for the norm
  float dynamic_scale;
};

// Vector quantizer rounding of the reference: add +-0.5, clamp, truncate.
__device__ __forceinline__ int chain_round(float value) {
  float r = value + (value >= 0.0f ? 0.5f : -0.5f);
  r = r > 127.0f ? 127.0f : r;
  r = r < -127.0f ? -127.0f : r;
  return static_cast<int>(r);
}

// window_boundary.cpp:17-23 / encoded_projection.cpp:36-42.
__device__ __forceinline__ float chain_newton_sqrt(float value) {
  float estimate = value > 1.0f ? value : 1.0f;
#pragma unroll 1
  for (int i = 0; i < 20; ++i) estimate = 0.5f * (estimate + value / estimate);
  return estimate;
}

// prepare_int8_vector of the current vector on input side `side`
// (decode_pair.hip prepare_vector_kernel): one wavefront, rows 2l, 2l + 1.
__device__ void chain_prepare(ChainShared& sh, int side, int lane) {
  float x[2];
  float m = 0.0f;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int row = 2 * lane + e;
    x[e] = half_bits_to_float(sh.vector[row]) * sh.axis[side][row];
    m = fmaxf(m, fabsf(x[e]));
  }
  m = wave_max_valu(m);
  const float scale = m > 1.0e-20f ? m / 127.0f : 1.0f;
  const uint32_t c0 = static_cast<uint32_t>(chain_round(x[0] / scale)) & 0xFFu;
  const uint32_t c1 = static_cast<uint32_t>(chain_round(x[1] / scale)) & 0xFFu;
  // Rows 2l, 2l + 1 are bytes 2 (l & 1), +1 of word l / 2.
  reinterpret_cast<uint16_t*>(sh.q)[lane] = static_cast<uint16_t>(c0 | (c1 << 8));
  if (lane == 0) sh.dynamic_scale = scale;
}

// The rows' value of finish_encoded_projection / commit_encoded_rank
// (encoded_rank.hip encoded_rows_kernel) for a vector on side `in_side`,
// `ranks` fitted ranks; one wavefront, rows lane and lane + 64.  Returns the
// two rows' values.
__device__ void chain_rows(ChainShared& sh, int in_side, uint32_t ranks, int lane,
                           float (&row_value)[2]) {
  const int out_side = 1 - in_side;
  // The sequential coefficient sums, one per lane 0..23, over the vector.
  // Each term is an fp16 basis value times an fp16 vector value, a product
  // exact in fp32, so `coefficient += b * x` rounds exactly what
  // fma(b, x, coefficient) rounds: one v_fma_mix_f32 per term, reading both
  // halves of the packed words itself.
  float coefficient = 0.0f;
  if (lane < kCoefficientRows) {
    const uint16_t* const basis = sh.basis[in_side][lane];
    const auto term = [](uint32_t b, uint32_t x, float total) {
      return __builtin_fmaf(half_bits_to_float(b), half_bits_to_float(x), total);
    };
    for (int i = 0; i < kDim; i += 4) {
      const uint2 b = *reinterpret_cast<const uint2*>(basis + i);
      const uint2 x = *reinterpret_cast<const uint2*>(sh.vector + i);
      coefficient = term(b.x, x.x, coefficient);
      coefficient = term(b.x >> 16, x.x >> 16, coefficient);
      coefficient = term(b.y, x.y, coefficient);
      coefficient = term(b.y >> 16, x.y >> 16, coefficient);
    }
  }
  // Record coefficients times their suffixes, and the whole window's product.
  float suffix = 1.0f;
  for (int j = kWindow - 1; j >= 0; --j) {
    if (lane == 2 * kRank + j) coefficient *= suffix;
    suffix *= sh.decay[j];
  }
  const float boundary_suffix = suffix;
  float old_coefficient[kRank], new_coefficient[kRank], record_coefficient[kWindow];
#pragma unroll
  for (int r = 0; r < kRank; ++r) {
    old_coefficient[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(coefficient), r));
    new_coefficient[r] =
        __int_as_float(__builtin_amdgcn_readlane(__float_as_int(coefficient), kRank + r));
  }
#pragma unroll
  for (int j = 0; j < kWindow; ++j) {
    record_coefficient[j] =
        __int_as_float(__builtin_amdgcn_readlane(__float_as_int(coefficient), 2 * kRank + j));
  }
  const float dynamic = sh.dynamic_scale;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int row = lane + h * kChainLanes;
    float value = static_cast<float>(sh.p[row]) * dynamic / 127.0f * sh.axis[out_side][row] *
                  boundary_suffix;
#pragma unroll
    for (int r = 0; r < kRank; ++r) {
      value += half_bits_to_float(sh.basis[out_side][r][row]) * old_coefficient[r] *
               boundary_suffix;
      if (static_cast<uint32_t>(r) < ranks) {
        value -= half_bits_to_float(sh.basis[out_side][kRank + r][row]) * new_coefficient[r];
      }
    }
#pragma unroll
    for (int j = 0; j < kWindow; ++j) {
      value += half_bits_to_float(sh.basis[out_side][2 * kRank + j][row]) * record_coefficient[j];
    }
    row_value[h] = value;
  }
}

// finish_encoded_projection: the new vector v / |v| in fp16.
__device__ void chain_finish(ChainShared& sh, int in_side, uint32_t ranks, int lane) {
  float row_value[2];
  chain_rows(sh, in_side, ranks, lane, row_value);
  sh.values[lane] = row_value[0];
  sh.values[lane + kChainLanes] = row_value[1];
  wave_lds_sync();
  float squared_norm = 0.0f;
  for (int row = 0; row < kDim; row += 4) {
    const float4 v = *reinterpret_cast<const float4*>(sh.values + row);
    squared_norm += v.x * v.x;
    squared_norm += v.y * v.y;
    squared_norm += v.z * v.z;
    squared_norm += v.w * v.w;
  }
  const float inverse = squared_norm > 1.0e-20f ? 1.0f / chain_newton_sqrt(squared_norm) : 0.0f;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int row = lane + h * kChainLanes;
    sh.vector[row] = static_cast<uint16_t>(float_to_half_bits(row_value[h] * inverse));
  }
}

// commit_encoded_rank of rank `rank` (its vector on the right side).
__device__ void chain_commit(ChainShared& sh, const ChainArgs& a, uint64_t state, uint32_t rank,
                             int lane) {
  float row_value[2];
  chain_rows(sh, 0, rank, lane, row_value);
  const uint64_t base = (state * kRank + rank) * kDim;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int row = lane + h * kChainLanes;
    const uint16_t left = static_cast<uint16_t>(float_to_half_bits(row_value[h]));
    const uint16_t right = sh.vector[row];
    a.corrected[base + row] = row_value[h];
    a.new_left[base + row] = left;
    a.new_right[base + row] = right;
    sh.basis[1][kRank + rank][row] = left;
    sh.basis[0][kRank + rank][row] = right;
  }
}

// sum over i < 16 of the signed byte dot products of codes[i] and q[i].
__device__ __forceinline__ int dot64(const uint32_t (&codes)[16], const uint32_t* q) {
  int acc = 0;
#pragma unroll
  for (int i = 0; i < 16; i += 4) {
    const uint4 qw = *reinterpret_cast<const uint4*>(q + i);
    acc = __builtin_amdgcn_sdot4(static_cast<int>(codes[i]), static_cast<int>(qw.x), acc, false);
    acc = __builtin_amdgcn_sdot4(static_cast<int>(codes[i + 1]), static_cast<int>(qw.y), acc,
                                 false);
    acc = __builtin_amdgcn_sdot4(static_cast<int>(codes[i + 2]), static_cast<int>(qw.z), acc,
                                 false);
    acc = __builtin_amdgcn_sdot4(static_cast<int>(codes[i + 3]), static_cast<int>(qw.w), acc,
                                 false);
  }
  return acc;
}

// Eight waves per SIMD (64 VGPRs): two states per SIMD at a time and 2,048 in
// flight, so 8,192 states run in four full rounds.  The compiler spills about
// half of the column words to scratch and reloads them in each transposed
// product; measured at 8,192 states and 8 iterations (ms): 2.20 at five waves
// per SIMD without spills, 1.99 at six, 1.76 at eight, bit-identical.
__global__ __launch_bounds__(kChainThreads, 8) void encoded_chain_kernel(ChainArgs a) {
  __shared__ ChainShared sh;
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const uint64_t state = blockIdx.x;

  // ---- the boundary in registers, both orientations ------------------------
  // rows[i]: codes A[t/2][64 (t&1) + 4i ..+3]; columns[i]: codes
  // A[64 (t&1) + 4i + j][t/2], j = 0..3, one word each.
  const int line = t >> 1;
  const int part = t & 1;
  const int8_t* const tile = a.residual + state * kTile;
  uint32_t rows[16], columns[16];
  {
    const uint4* src = reinterpret_cast<const uint4*>(tile + line * kDim + 64 * part);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 w = src[i];
      rows[4 * i] = w.x, rows[4 * i + 1] = w.y, rows[4 * i + 2] = w.z, rows[4 * i + 3] = w.w;
    }
    // The columns through LDS, half the tile at a time, staged in the basis
    // area before the bases are loaded: rows 64h..64h+63 (8 KiB) are written
    // by the threads that hold them and read down the columns by the threads
    // of part h.
    uint8_t* const stage = reinterpret_cast<uint8_t*>(&sh.basis[0][0][0]);
    static_assert(sizeof(sh.basis) >= 64 * kDim, "staging area");
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      __syncthreads();
      if ((line >> 6) == h) {
        uint4* const to = reinterpret_cast<uint4*>(stage + (line - 64 * h) * kDim + 64 * part);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          to[i] = make_uint4(rows[4 * i], rows[4 * i + 1], rows[4 * i + 2], rows[4 * i + 3]);
        }
      }
      __syncthreads();
      if (part == h) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          uint32_t word = 0;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            word |= static_cast<uint32_t>(stage[(4 * i + j) * kDim + line]) << (8 * j);
          }
          columns[i] = word;
        }
      }
    }
    __syncthreads();  // the staging area becomes the bases
  }

  // ---- bases, records, scales, gates, zero fitted ranks --------------------
  const uint64_t basis_base = state * kDim * kRank;
  const uint64_t record_base = state * kWindow * kDim;
  for (int i = t; i < kDim * kRank; i += kChainThreads) {
    const int dim = i >> 2, r = i & 3;  // [dim][rank] -> [rank][dim]
    sh.basis[0][r][dim] = a.old_right[basis_base + i];
    sh.basis[1][r][dim] = a.old_left[basis_base + i];
    sh.basis[0][kRank + r][dim] = 0;
    sh.basis[1][kRank + r][dim] = 0;
  }
  for (int i = t; i < kWindow * kDim; i += kChainThreads) {
    const int j = i >> 7, dim = i & (kDim - 1);
    sh.basis[0][2 * kRank + j][dim] = a.record_right[record_base + i];
    sh.basis[1][2 * kRank + j][dim] = a.record_left[record_base + i];
  }
  if (t < kDim) {
    sh.axis[0][t] = a.scales[state * kDim + t];
    sh.axis[1][t] = a.smoothing[state * kDim + t];
  }
  if (t < kWindow) sh.decay[t] = a.record_decay[state * kWindow + t];

  // ---- the chain -----------------------------------------------------------
  int role = 0;  // the wavefront that runs the next sequential stage
  for (uint32_t rank = 0; rank < static_cast<uint32_t>(kRank); ++rank) {
    __syncthreads();  // the previous rank's commit has read the vector
    if (t < kDim) sh.vector[t] = a.seeds[(state * kRank + rank) * kDim + t];
    const uint32_t steps = 2 * a.iterations + 1;  // forward, transposed, ..., commit
    for (uint32_t step = 0; step < steps; ++step) {
      const int side = static_cast<int>(step & 1u);  // input side: 0 forward, 1 transposed
      __syncthreads();
      if (wave == role) chain_prepare(sh, side, lane);
      __syncthreads();
      // p[line] over the thread's 64 codes of the line and its partner's 64
      // (a uniform branch: one straight loop per orientation, no selects).
      int acc = 0;
      if (side == 0) {
        acc = dot64(rows, sh.q + 16 * part);
      } else {
        acc = dot64(columns, sh.q + 16 * part);
      }
      acc += __builtin_amdgcn_update_dpp(0, acc, 0xB1, 0xF, 0xF, false);  // partner lane t ^ 1
      if (part == 0) sh.p[line] = acc;
      __syncthreads();
      if (wave == role) {
        if (step + 1 < steps) {
          chain_finish(sh, side, rank, lane);
        } else {
          chain_commit(sh, a, state, rank, lane);
        }
      }
      role = (role + 1) & (kChainWaves - 1);
    }
  }
}

}  // namespace
}  // namespace gdn

extern "C" int32_t statecentric_gdn_state_codec_encoded_rank_chain_launch_v4(
    void* stream, const int8_t* residual, const float* smoothing, const float* scales,
    const uint16_t* old_left, const uint16_t* old_right, const float* record_decay,
    const uint16_t* record_left, const uint16_t* record_right, const uint16_t* seeds,
    uint16_t* new_left, uint16_t* new_right, float* corrected, uint32_t states,
    uint32_t iterations) {
  if (!residual || !smoothing || !scales || !old_left || !old_right || !record_decay ||
      !record_left || !record_right || !seeds || !new_left || !new_right || !corrected ||
      states == 0 || states > gdn::kMaxWindowStates || iterations == 0 ||
      iterations > gdn::kMaxChainIterations ||
      !gdn::aligned16(residual, smoothing, scales, old_left, old_right, record_decay,
                      record_left, record_right, seeds, new_left, new_right, corrected)) {
    return gdn::kStatusInvalidArgument;
  }
  const gdn::ChainArgs args{residual, smoothing, scales, old_left, old_right, record_decay,
                            record_left, record_right, seeds, new_left, new_right, corrected,
                            iterations};
  return gdn::launch(gdn::encoded_chain_kernel, dim3(states), dim3(gdn::kChainThreads), stream,
                     args);
}
