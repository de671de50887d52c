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
// tile on bf16 MFMA (v_mfma_f32_32x32x16_bf16).  Codes are exact in bf16; the
// fp32 operand w[t][k] = s[k] * x_t[k] is split into three bf16 parts
// w = hi + mid + lo (exact), staged in LDS in the MFMA operand order, so the
// products are exact and only fp32 accumulation rounds.  The scale[v] / 127
// factor is applied in the epilogue.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "codec_math.h"
#include "launch.h"

namespace gdn {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;

constexpr int kThreads = 256;

__device__ __forceinline__ float code_byte(uint32_t word, int byte) {
  return static_cast<float>(
      static_cast<int8_t>(static_cast<uint8_t>(word >> (8 * byte))));
}

__device__ __forceinline__ uint32_t word_of(const uint4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// ------------------------------------------------------------------ decode

// Adds partner halves so that, over the 3 lane bits selected by masks
// m2 > m1 > m0, 16 partials reduce to 2 per lane: the lane keeps entries
// 2 * idx + {0, 1} where idx = 4*bit(m2) + 2*bit(m1) + bit(m0).
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

template <uint32_t kLayout>
__global__ __launch_bounds__(kThreads) void decode_projection_kernel(
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
      row[j] = *reinterpret_cast<const uint4*>(c + (r8 + 8 * j) * kDim + 16 * kq);
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
    reduce16_over_8_lanes(acc, lane, 4, 2, 1);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int v = r8 + 8 * (2 * kq + e);
      o[v] = acc[e] / kQuantizedMaximum * scale[v];
    }
  } else {
    // [key][value] codes: lane owns values 16*vc..+15 of key rows kr + 8j.
    const int vc = lane & 7;
    const int kr = lane >> 3;
    uint4 row[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      row[j] = *reinterpret_cast<const uint4*>(c + (kr + 8 * j) * kDim + 16 * vc);
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
    reduce16_over_8_lanes(acc, lane, 32, 16, 8);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int v = 16 * vc + 2 * kr + e;
      o[v] = acc[e] / kQuantizedMaximum * scale[v];
    }
  }
}

// ----------------------------------------------------------------- chunked

// bf16 split of an fp32 value into three round-to-nearest-even parts whose
// sum is the value (each remainder is exact in fp32 and needs at most 8 more
// significant bits).
__device__ __forceinline__ void split3(float w, uint16_t& hi, uint16_t& mid,
                                       uint16_t& lo) {
  hi = float_to_bf16(w);
  const float r1 = w - bf16_to_float(hi);
  mid = float_to_bf16(r1);
  const float r2 = r1 - bf16_to_float(mid);
  lo = float_to_bf16(r2);
}

__device__ __forceinline__ uint32_t pack_bf16_of_codes(uint32_t word, int pair) {
  // bf16 of an int8 code is the upper half of its exact fp32 value.
  const uint32_t a = __float_as_uint(code_byte(word, 2 * pair));
  const uint32_t b = __float_as_uint(code_byte(word, 2 * pair + 1));
  return (a >> 16) | (b & 0xFFFF0000u);
}

// Logical key order of the MFMA operands: for k-step s (0..7) and lane half g
// (lane / 32), the 8 operand elements are keys 64g + 8s + i.  A (queries) and
// B (codes) use the same order, so the contraction covers every key once, and
// each lane's codes for all 8 steps are one contiguous 64-byte run.
template <uint32_t kLayout>
__global__ __launch_bounds__(kThreads) void chunked_projection_kernel(
    const int8_t* __restrict__ codes, const float* __restrict__ smoothing,
    const float* __restrict__ scales, const uint16_t* __restrict__ queries,
    float* __restrict__ out, uint32_t tokens, uint32_t value_heads,
    uint32_t group, uint32_t query_heads, float query_scale) {
  // A operand, [split][k-step][lane] x 8 bf16 (16 B): 24 KiB.
  __shared__ uint4 a_lds[3][8][64];
  __shared__ float s_lds[kDim];

  const uint64_t pair = blockIdx.x;  // sequence * value_heads + head
  const uint64_t n = pair / value_heads;
  const uint64_t h = pair % value_heads;
  const uint64_t qh = h / group;
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int g = lane >> 5;
  const int v = 32 * wave + (lane & 31);

  // B operand: codes(v, 64g + 8s + i) as bf16, s = 0..7.
  bf16x8 b[8];
  const int8_t* tile = codes + pair * kTile;
  if constexpr (kLayout == kValueKey) {
    const int8_t* run = tile + v * kDim + 64 * g;
#pragma unroll
    for (int part = 0; part < 4; ++part) {
      const uint4 word4 = *reinterpret_cast<const uint4*>(run + 16 * part);
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const uint32_t w0 = word_of(word4, 2 * half);
        const uint32_t w1 = word_of(word4, 2 * half + 1);
        uint4 packed;
        packed.x = pack_bf16_of_codes(w0, 0);
        packed.y = pack_bf16_of_codes(w0, 1);
        packed.z = pack_bf16_of_codes(w1, 0);
        packed.w = pack_bf16_of_codes(w1, 1);
        b[2 * part + half] = __builtin_bit_cast(bf16x8, packed);
      }
    }
  } else {
#pragma unroll
    for (int step = 0; step < 8; ++step) {
      uint32_t w0 = 0, w1 = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        w0 |= static_cast<uint32_t>(static_cast<uint8_t>(
                  tile[(64 * g + 8 * step + i) * kDim + v]))
              << (8 * i);
        w1 |= static_cast<uint32_t>(static_cast<uint8_t>(
                  tile[(64 * g + 8 * step + 4 + i) * kDim + v]))
              << (8 * i);
      }
      uint4 packed;
      packed.x = pack_bf16_of_codes(w0, 0);
      packed.y = pack_bf16_of_codes(w0, 1);
      packed.z = pack_bf16_of_codes(w1, 0);
      packed.w = pack_bf16_of_codes(w1, 1);
      b[step] = __builtin_bit_cast(bf16x8, packed);
    }
  }
  const float epilogue = scales[pair * kDim + v] / kQuantizedMaximum;
  if (t < kDim) s_lds[t] = smoothing[pair * kDim + t];

  // Producer role: thread t builds w for token row m = t / 8 of the block and
  // keys 16*kc..+15, which are k-steps 2*(kc%4) + {0,1} of lane half kc / 4.
  const int m = t >> 3;
  const int kc = t & 7;
  const int dst_lane = m + 32 * (kc >> 2);
  const int dst_step = 2 * (kc & 3);

  for (uint32_t block = 0; block < tokens; block += 32) {
    __syncthreads();  // s_lds ready / previous block's operands consumed
    const uint32_t token = block + m;
    uint32_t qw[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (token < tokens) {
      const uint16_t* qrow =
          queries + ((n * tokens + token) * query_heads + qh) * kDim + 16 * kc;
      const uint4 q0 = *reinterpret_cast<const uint4*>(qrow);
      const uint4 q1 = *reinterpret_cast<const uint4*>(qrow + 8);
      qw[0] = q0.x; qw[1] = q0.y; qw[2] = q0.z; qw[3] = q0.w;
      qw[4] = q1.x; qw[5] = q1.y; qw[6] = q1.z; qw[7] = q1.w;
    }
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      uint32_t hi[4], mid[4], lo[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        uint16_t h2[2], m2[2], l2[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int i = 8 * half + 2 * p + e;  // 0..15 within the chunk
          const uint16_t qbits = static_cast<uint16_t>(qw[i >> 1] >> (16 * (i & 1)));
          const float x = query_scale * bf16_to_float(qbits);
          const float w = s_lds[16 * kc + i] * x;
          split3(w, h2[e], m2[e], l2[e]);
        }
        hi[p] = h2[0] | (static_cast<uint32_t>(h2[1]) << 16);
        mid[p] = m2[0] | (static_cast<uint32_t>(m2[1]) << 16);
        lo[p] = l2[0] | (static_cast<uint32_t>(l2[1]) << 16);
      }
      a_lds[0][dst_step + half][dst_lane] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
      a_lds[1][dst_step + half][dst_lane] = make_uint4(mid[0], mid[1], mid[2], mid[3]);
      a_lds[2][dst_step + half][dst_lane] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    }
    __syncthreads();

    f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int step = 0; step < 8; ++step) {
#pragma unroll
      for (int split = 0; split < 3; ++split) {
        const bf16x8 a = __builtin_bit_cast(bf16x8, a_lds[split][step][lane]);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b[step], acc, 0, 0, 0);
      }
    }
    // Accumulator element r of lane holds row 8*(r/4) + 4*g + r%4, column v.
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const uint32_t row_token = block + 8 * (r >> 2) + 4 * g + (r & 3);
      if (row_token < tokens) {
        out[((n * tokens + row_token) * value_heads + h) * kDim + v] =
            acc[r] * epilogue;
      }
    }
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
      (layout != gdn::kKeyValue && layout != gdn::kValueKey)) {
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
      (layout != gdn::kKeyValue && layout != gdn::kValueKey)) {
    return gdn::kStatusInvalidArgument;
  }
  const uint64_t pairs = static_cast<uint64_t>(seqs) * value_heads;
  if (pairs > gdn::kMaxGrid) return gdn::kStatusInvalidArgument;
  const uint32_t group = value_heads / query_heads;
  const dim3 grid(static_cast<uint32_t>(pairs));
  const dim3 block(gdn::kThreads);
  if (layout == gdn::kValueKey) {
    return gdn::launch(gdn::chunked_projection_kernel<gdn::kValueKey>, grid,
                       block, stream, residual, smoothing, scales, queries,
                       outputs, tokens, value_heads, group, query_heads,
                       query_scale);
  }
  return gdn::launch(gdn::chunked_projection_kernel<gdn::kKeyValue>, grid, block,
                     stream, residual, smoothing, scales, queries, outputs,
                     tokens, value_heads, group, query_heads, query_scale);
}
