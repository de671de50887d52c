// Self-check of the wavefront exchanges in lane_exchange.h (not part of the
// codec's C-ABI): one wavefront applies every helper to two input vectors and
// writes the results, which tests/test_lane_exchange_gpu.py compares with
// numpy.  It pins the permlane swaps' lane mapping and the extraction of both
// swap results, which this compiler once mis-lowered.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bf16_operands.h"
#include "lane_exchange.h"

namespace {

constexpr int kLanes = 64;
// Output layout, in blocks of 64 values:
//   0..5   fold<m>(x, y) for m = 32, 16, 8, 4, 2, 1
//   6..11  add_partner<m>(x) for the same masks
//   12     wave_sum_valu(x)
//   13     wave_max_valu(x)
//   14..16 integer fold<m>(bits(x), bits(y)) for m = 4, 2, 1
constexpr int kOutputs = 17 * kLanes;

template <int kMask>
__device__ void folds(const float* in, float* out, int lane, int block) {
  const float x = in[lane], y = in[kLanes + lane];
  out[block * kLanes + lane] = gdn::fold<kMask>(x, y, lane);
  out[(block + 6) * kLanes + lane] = gdn::add_partner<kMask>(x);
}

__global__ __launch_bounds__(kLanes) void lane_probe_kernel(const float* in, float* out) {
  const int lane = threadIdx.x;
  folds<32>(in, out, lane, 0);
  folds<16>(in, out, lane, 1);
  folds<8>(in, out, lane, 2);
  folds<4>(in, out, lane, 3);
  folds<2>(in, out, lane, 4);
  folds<1>(in, out, lane, 5);
  const float x = in[lane], y = in[kLanes + lane];
  out[12 * kLanes + lane] = gdn::wave_sum_valu(x);
  out[13 * kLanes + lane] = gdn::wave_max_valu(x);
  const int xi = __float_as_int(x), yi = __float_as_int(y);
  out[14 * kLanes + lane] = __int_as_float(gdn::fold<4>(xi, yi, lane));
  out[15 * kLanes + lane] = __int_as_float(gdn::fold<2>(xi, yi, lane));
  out[16 * kLanes + lane] = __int_as_float(gdn::fold<1>(xi, yi, lane));
}

}  // namespace

// in: 128 floats (x then y); out: 17 * 64 floats.  One wavefront.
extern "C" int32_t gdn_lane_probe(void* stream, const float* in, float* out) {
  if (in == nullptr || out == nullptr) return 1;
  hipLaunchKernelGGL(lane_probe_kernel, dim3(1), dim3(kLanes), 0,
                     static_cast<hipStream_t>(stream), in, out);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

extern "C" uint32_t gdn_lane_probe_outputs() { return kOutputs; }

namespace {

__global__ __launch_bounds__(256) void split_probe_kernel(const float* in, uint32_t* hi,
                                                          uint32_t* lo, uint32_t pairs) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= pairs) return;
  gdn::split2_pair(in[2 * i], in[2 * i + 1], hi[i], lo[i]);
}

}  // namespace

// Self-check of the chunked projection's bf16 split (bf16_operands.h): in
// holds 2 * pairs floats; hi and lo receive one packed bf16 pair per input
// pair (low element first).
extern "C" int32_t gdn_split_probe(void* stream, const float* in, uint32_t* hi, uint32_t* lo,
                                   uint32_t pairs) {
  if (in == nullptr || hi == nullptr || lo == nullptr || pairs == 0) return 1;
  hipLaunchKernelGGL(split_probe_kernel, dim3((pairs + 255u) / 256u), dim3(256), 0,
                     static_cast<hipStream_t>(stream), in, hi, lo, pairs);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}
