// Dense fp32 GDN step (kernel/gdn_state_codec_fp32_gdn_step.cpp:1-23): the
// reference's uncompressed baseline, a [S][key][value] fp32 state updated in
// place.  Per value column c:
//   projection = sum_r S[r][c] * read[r]           (rows in order)
//   correction = value[c] - projection
//   S'[r][c]   = decay * S[r][c] + key[r] * correction
//   out[c]     = sum_r S'[r][c] * query[r]          (rows in order)
// One thread per column keeps the reference's sequential row order, so the
// result is bit-identical to the CPU statement of that kernel; consecutive
// threads read consecutive columns, so every row access is one coalesced
// 512-byte line.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gdn_state_codec_window.h"
#include "launch.h"
#include "window_common.h"

namespace gdn {
namespace {

constexpr int kThreads = 256;
constexpr int kStatesPerBlock = kThreads / kDim;

__global__ __launch_bounds__(kThreads) void dense_step_kernel(
    float* __restrict__ state, const float* __restrict__ decay,
    const uint16_t* __restrict__ keys, const uint16_t* __restrict__ reads,
    const uint16_t* __restrict__ queries, const uint16_t* __restrict__ values,
    float* __restrict__ outputs, uint32_t states) {
  __shared__ float vectors[kStatesPerBlock][3][kDim];  // read, key, query
  const int local = threadIdx.x / kDim;
  const int column = threadIdx.x % kDim;
  const uint32_t s = blockIdx.x * kStatesPerBlock + local;
  const bool live = s < states;
  const uint64_t vb = static_cast<uint64_t>(s) * kDim;
  if (live) {
    vectors[local][0][column] = half_bits_to_float(reads[vb + column]);
    vectors[local][1][column] = half_bits_to_float(keys[vb + column]);
    vectors[local][2][column] = half_bits_to_float(queries[vb + column]);
  }
  __syncthreads();
  if (!live) return;
  float* S = state + static_cast<uint64_t>(s) * kTile;
  float projection = 0.0f;
  for (int r = 0; r < kDim; ++r) projection += S[r * kDim + column] * vectors[local][0][r];
  const float correction = half_bits_to_float(values[vb + column]) - projection;
  const float g = decay[s];
  float out = 0.0f;
  for (int r = 0; r < kDim; ++r) {
    const float next = g * S[r * kDim + column] + vectors[local][1][r] * correction;
    S[r * kDim + column] = next;
    out += next * vectors[local][2][r];
  }
  outputs[vb + column] = out;
}

}  // namespace
}  // namespace gdn

extern "C" int32_t statecentric_gdn_state_codec_fp32_gdn_step_launch_v1(
    void* stream, float* dense_state, const float* decay, const uint16_t* write_keys,
    const uint16_t* reads, const uint16_t* queries, const uint16_t* values, float* outputs,
    uint32_t states) {
  if (!dense_state || !decay || !write_keys || !reads || !queries || !values || !outputs ||
      states == 0 || states > gdn::kMaxWindowStates ||
      !gdn::aligned16(dense_state, decay, write_keys, reads, queries, values, outputs)) {
    return gdn::kStatusInvalidArgument;
  }
  const dim3 grid((states + gdn::kStatesPerBlock - 1) / gdn::kStatesPerBlock);
  return gdn::launch(gdn::dense_step_kernel, grid, dim3(gdn::kThreads), stream, dense_state,
                     decay, write_keys, reads, queries, values, outputs, states);
}
