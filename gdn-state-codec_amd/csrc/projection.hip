// Encoded projection: queries read against the int8 state with dequantization
// fused in, never materializing the fp32 state.
//
// For one head tile (codes, s = smoothing[key], scale[value]) and one query
// x[k] = query_scale * q[k] (q bf16), the boundary readout of the reference
// (native/src/gdn_state_codec_state_capsule.cpp:281-290, records and
// compensators absent) is
//   out[v] = (sum_k code(v, k) * s[k] * x[k]) / 127 * scale[v].
// Value head h reads query head h / (value_heads / query_heads): Qwen's GQA
// pairs consecutive value heads on one query/key head
// (kernel/gdn_state_codec_windowed_gdn_step.cpp:340,
// kernel/gdn_state_codec_encoded_projection.cpp:351-353).
//
// Decode (one query per tile) is a batched GEMV bound by HBM reads of the
// codes: one wavefront per tile, w[k] = s[k] * x[k] held in registers, codes
// converted in registers and accumulated with fp32 FMAs.
//
// Chunked (T queries per tile) is a [T x 128] x [128 x 128] contraction per
// tile on bf16 MFMA (v_mfma_f32_16x16x32_bf16).  Codes are exact in bf16; the
// fp32 operand w[t][k] = s[k] * x_t[k] is split into two bf16 parts
// w ~ hi + lo (each rounded to nearest, remainder below 2^-16 |w| for every
// finite |w| >= 2^-110: hi is clamped to the largest finite bf16, so the top
// of fp32's range splits into finite parts), staged in LDS in the MFMA
// operand order.  The products with the codes are exact, so
// the result differs from the exact readout by at most 2^-16 of sum |terms|
// from the split plus the fp32 accumulation of 256 products (at most
// 256 * 2^-24 of sum |terms|) and the epilogue's rounding: within
// 2^-14 * sum |terms|.  The scale[v] / 127 factor is applied in the epilogue.
// (A third part would make the products exact; it costs a third more MFMA
// and LDS work and measured 7% slower at config 4.)
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "codec_math.h"
#include "bf16_operands.h"
#include "lane_exchange.h"
#include "launch.h"
#include "stream_memory.h"

namespace gdn {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float code_byte(uint32_t word, int byte) {
  return static_cast<float>(
      static_cast<int8_t>(static_cast<uint8_t>(word >> (8 * byte))));
}

__device__ __forceinline__ uint32_t word_of(const uint4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// ------------------------------------------------------------------ decode

// Adds partner halves so that, over the 3 lane bits M2 > M1 > M0, 16 partials
// reduce to 2 per lane: the lane keeps entries 2 * idx + {0, 1} where
// idx = 4*bit(M2) + 2*bit(M1) + bit(M0).
template <int M2, int M1, int M0>
__device__ __forceinline__ void reduce16_over_8_lanes(float (&p)[16], int lane) {
#pragma unroll
  for (int i = 0; i < 8; ++i) p[i] = fold<M2>(p[i], p[i + 8], lane);
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = fold<M1>(p[i], p[i + 4], lane);
#pragma unroll
  for (int i = 0; i < 2; ++i) p[i] = fold<M0>(p[i], p[i + 2], lane);
}

// The same reduction through ds_bpermute, for the [key][value] decode kernel:
// at its 64-VGPR limit the VALU exchanges spill.
__device__ __forceinline__ void reduce16_over_8_lanes_shuffle(float (&p)[16], int lane,
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

template <uint32_t kLayout>
// 64 VGPRs: all 8192 wavefronts of a B=256, 32-head batch are resident at once.
__global__ __launch_bounds__(kThreads, 8) void decode_projection_kernel(
    const int8_t* __restrict__ codes, const float* __restrict__ smoothing,
    const float* __restrict__ scales, const uint16_t* __restrict__ queries,
    float* __restrict__ out, uint64_t tiles, uint32_t value_heads,
    uint32_t group, uint32_t query_heads, float query_scale) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const uint64_t tile = static_cast<uint64_t>(blockIdx.x) * 4 + wave;
  if (tile >= tiles) return;  // whole wavefront; the kernel has no barriers
  const uint64_t b = tile / value_heads;
  const uint64_t h = tile % value_heads;
  const uint16_t* q = queries + (b * query_heads + h / group) * kDim;
  const float* s = smoothing + tile * kDim;
  const int8_t* c = codes + tile * kTile;
  const float* scale = scales + tile * kDim;
  float* o = out + tile * kDim;

  if constexpr (kLayout == kValueKey) {
    // Lane owns keys 16*kq..+15 of value rows r8 + 8j: each load instruction
    // reads 8 whole 128-byte rows.
    const int kq = lane & 7;
    const int r8 = lane >> 3;
    uint4 row[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      row[j] = stream_load(reinterpret_cast<const uint4*>(c + (r8 + 8 * j) * kDim + 16 * kq));
    }
    float w[16];
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      const float4 sv = *reinterpret_cast<const float4*>(s + 16 * kq + i);
      const uint2 qv = *reinterpret_cast<const uint2*>(q + 16 * kq + i);
      w[i + 0] = sv.x * (query_scale * bf16_to_float(qv.x & 0xFFFFu));
      w[i + 1] = sv.y * (query_scale * bf16_to_float(qv.x >> 16));
      w[i + 2] = sv.z * (query_scale * bf16_to_float(qv.y & 0xFFFFu));
      w[i + 3] = sv.w * (query_scale * bf16_to_float(qv.y >> 16));
    }
    float acc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      float a = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        a = fmaf(code_byte(word_of(row[j], i >> 2), i & 3), w[i], a);
      }
      acc[j] = a;
    }
    // Sum the 8 key chunks (lane bits 0..2); the lane keeps rows j = 2kq + e.
    reduce16_over_8_lanes<4, 2, 1>(acc, lane);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int v = r8 + 8 * (2 * kq + e);
      stream_store(o + v, acc[e] / kQuantizedMaximum * scale[v]);
    }
  } else {
    // [key][value] codes: lane owns values 16*vc..+15 of key rows kr + 8j.
    const int vc = lane & 7;
    const int kr = lane >> 3;
    uint4 row[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      row[j] = stream_load(reinterpret_cast<const uint4*>(c + (kr + 8 * j) * kDim + 16 * vc));
    }
    float w[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int k = kr + 8 * j;
      w[j] = s[k] * (query_scale * bf16_to_float(q[k]));
    }
    float acc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        acc[i] = fmaf(code_byte(word_of(row[j], i >> 2), i & 3), w[j], acc[i]);
      }
    }
    // Sum the 8 key groups (lane bits 3..5); the lane keeps values 2kr + e.
    reduce16_over_8_lanes_shuffle(acc, lane, 32, 16, 8);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int v = 16 * vc + 2 * kr + e;
      stream_store(o + v, acc[e] / kQuantizedMaximum * scale[v]);
    }
  }
}

// ----------------------------------------------------------------- chunked

// v_mfma_f32_16x16x32_bf16 operands: lane l holds row (A) or column (B)
// l % 16 and 8 consecutive elements of the contraction; the accumulator lane l
// holds column l % 16, rows 4 * (l / 16) + r.  The logical key order used for
// both operands is: k-step s (0..3), lane group g = l / 16 (0..3), element i
// -> key 32g + 8s + i, so a lane's codes for all four steps are one contiguous
// 32-byte run and the contraction covers every key exactly once.
//
// A workgroup owns one (sequence, head) tile; wavefront w owns the 32 values
// 32w..32w+31 (two 16-column MFMA tiles) and keeps their codes in registers as
// bf16 for every token block.  The tokens are taken kSub blocks of 16 rows at a
// time: the two bf16 parts of w[t][k] = s[k] * x_t[k] of each 16-row block are
// staged in LDS in operand order (8 KiB per block), behind one barrier pair per
// kSub blocks.  With kSub = 2 (17 KiB of LDS, 64 VGPRs) all 2048 workgroups of
// a 64 x 32-head batch are still resident at once, and each runs half as many
// barrier-separated rounds of query loads as with kSub = 1: config 4 measured
// 24.9 -> 23.6 us ([key][value]: 30.8 -> 27.6 us), bit-identical.  kSub = 4
// (33 KiB) leaves half the grid to a second round (24.6 us).
//
// kTail = false requires tokens % (16 * kSub) == 0.  kTail = true handles any
// token count: rows past the last token are computed from a clamped token
// (each output row depends only on its own query row) and never stored.
// Query and output addresses are a per-workgroup base plus a 32-bit lane byte
// offset, so one sequence's output rows must span fewer than 2^32 bytes
// (tokens * value_heads * 512; the launcher checks).
// The [value][key] form fits 64 VGPRs (8 wavefronts per SIMD); the byte gathers
// of the [key][value] form need more.
template <uint32_t kLayout, int kSub, bool kTail>
__global__ __launch_bounds__(kThreads, kLayout == kValueKey ? 8 : 4) void chunked_projection_kernel(
    const int8_t* __restrict__ codes, const float* __restrict__ smoothing,
    const float* __restrict__ scales, const uint16_t* __restrict__ queries,
    float* __restrict__ out, uint32_t tokens, uint32_t value_heads,
    uint32_t group, uint32_t query_heads, float query_scale) {
  constexpr int kBlockTokens = 16;
  __shared__ uint4 a_lds[kSub][2][4][64];  // [block][part][k-step][lane] x 8 bf16
  __shared__ float s_lds[kDim];
  __shared__ __align__(16) float e_lds[kDim];  // scale[v] / 127

  const uint64_t pair = blockIdx.x;  // sequence * value_heads + head
  const uint64_t n = pair / value_heads;
  const uint64_t h = pair % value_heads;
  const uint64_t qh = h / group;
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int col = lane & 15;
  const int g = lane >> 4;

  // B operands: for column tile c (0, 1) value v = 32 wave + 16 c + col and
  // keys 32g + 8s + i, s = 0..3.
  bf16x8 b[2][4];
  const int8_t* tile = codes + pair * kTile;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int v = 32 * wave + 16 * c + col;
    if constexpr (kLayout == kValueKey) {
      const int8_t* run = tile + v * kDim + 32 * g;
      const uint4 lo = stream_load(reinterpret_cast<const uint4*>(run));
      const uint4 hi = stream_load(reinterpret_cast<const uint4*>(run + 16));
      b[c][0] = codes_to_bf16x8(lo.x, lo.y);
      b[c][1] = codes_to_bf16x8(lo.z, lo.w);
      b[c][2] = codes_to_bf16x8(hi.x, hi.y);
      b[c][3] = codes_to_bf16x8(hi.z, hi.w);
    } else {
#pragma unroll
      for (int step = 0; step < 4; ++step) {
        uint32_t w0 = 0, w1 = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          w0 |= static_cast<uint32_t>(static_cast<uint8_t>(
                    tile[(32 * g + 8 * step + i) * kDim + v]))
                << (8 * i);
          w1 |= static_cast<uint32_t>(static_cast<uint8_t>(
                    tile[(32 * g + 8 * step + 4 + i) * kDim + v]))
                << (8 * i);
        }
        b[c][step] = codes_to_bf16x8(w0, w1);
      }
    }
  }
  if (t < kDim) {
    s_lds[t] = smoothing[pair * kDim + t];
    e_lds[t] = scales[pair * kDim + t] / kQuantizedMaximum;
  }

  // Producer role: thread t builds token row m = t / 16 of each block, keys
  // 8*kc..+7 (kc = t % 16), which is k-step kc % 4 of lane group kc / 4.
  const int m = t >> 4;
  const int kc = t & 15;
  const int dst_lane = m + 16 * (kc >> 2);
  const int dst_step = kc & 3;
  // Per-workgroup bases (uniform, scalar registers) plus per-lane 32-bit byte
  // offsets: the loads and stores take the scalar-base addressing form.
  const char* const q_seq =
      reinterpret_cast<const char*>(queries + (n * tokens * query_heads + qh) * kDim);
  const uint32_t q_row = query_heads * kDim * 2;  // bytes per token
  char* const o_seq = reinterpret_cast<char*>(out + (n * tokens * value_heads + h) * kDim);
  const uint32_t o_row = value_heads * kDim * 4;
  const bool odd = (col & 1) != 0;
  const int first = 32 * wave + (odd ? 15 + col : col);
  // Running lane offsets of the round's first block (query row m, output row
  // 4g, value `first`); the sub-block and row steps are uniform.  Offsets that
  // change every round keep the compiler from holding one per sub-block and
  // row in registers.
  uint32_t q_off = m * q_row + 16 * kc;
  uint32_t o_off = 4 * g * o_row + 4 * first;
  const uint32_t q_last = (tokens - 1) * q_row + 16 * kc;  // query row tokens - 1

  for (uint32_t block = 0; block < tokens; block += kSub * kBlockTokens) {
    __syncthreads();  // s_lds ready / previous blocks' operands consumed
    uint4 qv[kSub];
#pragma unroll
    for (int sub = 0; sub < kSub; ++sub) {
      uint32_t offset = q_off + kBlockTokens * sub * q_row;
      if constexpr (kTail) offset = min(offset, q_last);  // token clamped to tokens - 1
      qv[sub] = *reinterpret_cast<const uint4*>(q_seq + offset);
    }
#pragma unroll
    for (int sub = 0; sub < kSub; ++sub) {
      const float4 s0 = *reinterpret_cast<const float4*>(s_lds + 8 * kc);
      const float4 s1 = *reinterpret_cast<const float4*>(s_lds + 8 * kc + 4);
      const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
      uint32_t hi[4], lo[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const uint32_t word = word_of(qv[sub], p);
        const float w0 = sv[2 * p] * (query_scale * bf16_to_float(word & 0xFFFFu));
        const float w1 = sv[2 * p + 1] * (query_scale * bf16_to_float(word >> 16));
        split2_pair(w0, w1, hi[p], lo[p]);
      }
      a_lds[sub][0][dst_step][dst_lane] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
      a_lds[sub][1][dst_step][dst_lane] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    }
    __syncthreads();

#pragma unroll
    for (int sub = 0; sub < kSub; ++sub) {
      const uint32_t rows = block + kBlockTokens * sub;  // first token of the block
      if (kTail && rows >= tokens) break;
      f32x4 acc[2];
#pragma unroll
      for (int c = 0; c < 2; ++c) acc[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int step = 0; step < 4; ++step) {
#pragma unroll
        for (int part = 0; part < 2; ++part) {
          const bf16x8 a = __builtin_bit_cast(bf16x8, a_lds[sub][part][step][lane]);
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[c][step], acc[c],
                                                             0, 0, 0);
          }
        }
      }
      // Accumulator r of column tile c is token row 4g + r of the block, value
      // 32 wave + 16 c + col.  Adjacent lanes swap one value (DPP quad_perm
      // [1,0,3,2]) so that the even lane of a pair holds values col, col + 1 of
      // tile 0 and the odd lane values col - 1, col of tile 1: each store then
      // writes the wave's 32 values of a row as one whole 128-byte line.
      const float2 factor = *reinterpret_cast<const float2*>(&e_lds[first]);
      uint2 pairs[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float send = odd ? acc[0][r] : acc[1][r];
        const float got = __builtin_bit_cast(
            float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, send), 0xB1, 0xF,
                                               0xF, false));
        const float lo = odd ? got : acc[0][r];
        const float hi = odd ? acc[1][r] : got;
        pairs[r] = make_uint2(__float_as_uint(lo * factor.x), __float_as_uint(hi * factor.y));
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (!kTail || rows + 4 * g + r < tokens) {
          stream_store(reinterpret_cast<uint2*>(o_seq + o_off + (kBlockTokens * sub + r) * o_row),
                       pairs[r]);
        }
      }
    }
    q_off += kSub * kBlockTokens * q_row;
    o_off += kSub * kBlockTokens * o_row;
  }
}

bool projection_shape_ok(uint32_t value_heads, uint32_t query_heads) {
  return value_heads > 0 && query_heads > 0 && query_heads <= value_heads &&
         value_heads % query_heads == 0;
}

}  // namespace
}  // namespace gdn

// Decode projection: residual [batch][value_heads] tiles in `layout`, smoothing
// and scales [batch][value_heads][128], queries bf16 [batch][query_heads][128],
// outputs fp32 [batch][value_heads][128].
extern "C" int32_t
statecentric_gdn_state_codec_encoded_projection_decode_launch_v4(
    void* stream, const int8_t* residual, const float* smoothing,
    const float* scales, const uint16_t* queries, float* outputs,
    uint32_t batch, uint32_t value_heads, uint32_t query_heads,
    float query_scale, uint32_t layout) {
  if (residual == nullptr || smoothing == nullptr || scales == nullptr ||
      queries == nullptr || outputs == nullptr || batch == 0 ||
      !gdn::projection_shape_ok(value_heads, query_heads) ||
      (layout != gdn::kKeyValue && layout != gdn::kValueKey) ||
      !gdn::aligned16(residual, smoothing, scales, queries, outputs)) {
    return gdn::kStatusInvalidArgument;
  }
  const uint64_t tiles = static_cast<uint64_t>(batch) * value_heads;
  const uint64_t blocks = (tiles + 3) / 4;
  if (blocks > gdn::kMaxGrid) return gdn::kStatusInvalidArgument;
  const uint32_t group = value_heads / query_heads;
  const dim3 grid(static_cast<uint32_t>(blocks));
  const dim3 block(gdn::kThreads);
  if (layout == gdn::kValueKey) {
    return gdn::launch(gdn::decode_projection_kernel<gdn::kValueKey>, grid,
                       block, stream, residual, smoothing, scales, queries,
                       outputs, tiles, value_heads, group, query_heads,
                       query_scale);
  }
  return gdn::launch(gdn::decode_projection_kernel<gdn::kKeyValue>, grid, block,
                     stream, residual, smoothing, scales, queries, outputs,
                     tiles, value_heads, group, query_heads, query_scale);
}

// Chunked projection: residual [seqs][value_heads] tiles, queries bf16
// [seqs][tokens][query_heads][128], outputs fp32 [seqs][tokens][value_heads][128].
extern "C" int32_t
statecentric_gdn_state_codec_encoded_projection_chunked_launch_v4(
    void* stream, const int8_t* residual, const float* smoothing,
    const float* scales, const uint16_t* queries, float* outputs,
    uint32_t seqs, uint32_t tokens, uint32_t value_heads, uint32_t query_heads,
    float query_scale, uint32_t layout) {
  if (residual == nullptr || smoothing == nullptr || scales == nullptr ||
      queries == nullptr || outputs == nullptr || seqs == 0 || tokens == 0 ||
      !gdn::projection_shape_ok(value_heads, query_heads) ||
      (layout != gdn::kKeyValue && layout != gdn::kValueKey) ||
      !gdn::aligned16(residual, smoothing, scales, queries, outputs)) {
    return gdn::kStatusInvalidArgument;
  }
  const uint64_t pairs = static_cast<uint64_t>(seqs) * value_heads;
  if (pairs > gdn::kMaxGrid) return gdn::kStatusInvalidArgument;
  // One sequence's query and output rows are addressed with 32-bit byte
  // offsets (value_heads >= query_heads, fp32 outputs >= bf16 queries).
  if (static_cast<uint64_t>(tokens) * value_heads * gdn::kDim * sizeof(float) > 0xFFFFFFFFull) {
    return gdn::kStatusInvalidArgument;
  }
  const uint32_t group = value_heads / query_heads;
  const dim3 grid(static_cast<uint32_t>(pairs));
  const dim3 block(gdn::kThreads);
  // 32-token rounds when every round is full, else 16-token rounds with the
  // tail handled.
  const bool whole = tokens % 32 == 0;
  if (layout == gdn::kValueKey) {
    return whole ? gdn::launch(gdn::chunked_projection_kernel<gdn::kValueKey, 2, false>, grid,
                               block, stream, residual, smoothing, scales, queries, outputs,
                               tokens, value_heads, group, query_heads, query_scale)
                 : gdn::launch(gdn::chunked_projection_kernel<gdn::kValueKey, 1, true>, grid,
                               block, stream, residual, smoothing, scales, queries, outputs,
                               tokens, value_heads, group, query_heads, query_scale);
  }
  return whole ? gdn::launch(gdn::chunked_projection_kernel<gdn::kKeyValue, 2, false>, grid,
                             block, stream, residual, smoothing, scales, queries, outputs,
                             tokens, value_heads, group, query_heads, query_scale)
               : gdn::launch(gdn::chunked_projection_kernel<gdn::kKeyValue, 1, true>, grid,
                             block, stream, residual, smoothing, scales, queries, outputs,
                             tokens, value_heads, group, query_heads, query_scale);
}
