// Boundary encode with the rank-r compensator fit, the public capsule path's
// quantizer (GdnStateCodecCapsule::FromDenseBoundary, state_capsule.cpp:318-335,
// which calls QuantizeBoundary :129-226).
//
// For each [key][value] head the fit (:136-188) takes rank r = 0..r-1 in turn:
//   right[c] = sinf((r+1)(c+1)), normalized (if the norm fails, right[0] = 1);
//   32 times: left = R right, normalized; right = R^T left, normalized
//     (either normalization failing ends the loop);
//   singular value sv = sum over rows, then columns, of left[row] * R * right[col];
//   compensator_keys[row][r] = left[row] * sv, compensator_values[col][r] = right[col];
//   R -= left[row] * sv * right[col].
// Norms are the reference's Norm (:48-52): a sequential double sum of squares,
// a double square root, rounded to float; a vector normalizes when that norm
// exceeds FLT_EPSILON (:60-65).  Every sum here is sequential in the
// reference's order, in the precision it uses, so the result is bit-identical
// to the reference's CPU code.  The quant stage (:190-226) then runs on the
// fitted residual through the batched encode (codec.hip).
//
// One 128-thread workgroup per head.  The residual lives in LDS at a row
// stride of 129 floats, so a thread per row (left = R right) and a thread per
// column (right = R^T left) both read it without bank conflicts.  The norms
// and the singular value are single-thread chains, as the reference's order
// requires; the sums of the two products run one per thread.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <cfloat>
#include <cmath>

#include "gdn_state_codec_kernel.h"
#include "launch.h"

namespace gdn {
namespace {

constexpr int kFitThreads = 128;
constexpr int kRowStride = kDim + 1;
constexpr uint32_t kMaxFitRank = 4;
constexpr int kFitIterations = 32;  // state_capsule.cpp:147

// Per-head outcomes written to `status`.
constexpr int32_t kFitOk = 0;
constexpr int32_t kFitNonFiniteInput = 1;     // FromDenseBoundary's check (:329-331)
constexpr int32_t kFitNonFiniteSingular = 2;  // QuantizeBoundary's check (:167-169)

// The start vectors sinf((r+1)(c+1)), formed on the host with the same libm
// call the reference makes (std::sin of a float).
struct StartVectors {
  float value[kMaxFitRank][kDim];
};

struct FitArgs {
  const float* dense;     // [states][key][value]
  float* residual;        // [states][key][value]: the fitted residual
  float* comp_keys;       // [states][key][rank]
  float* comp_values;     // [states][value][rank]
  int32_t* status;        // [states]
  uint32_t rank;
};

struct FitShared {
  float r[kDim * kRowStride];
  float left[kDim];
  float right[kDim];
  float scalar;
  int flag;
};

// Normalize (:60-65) of v[0..127] with the reference's Norm: thread 0 forms
// the sequential double sum of squares (each square exact in double) and its
// double square root; every thread divides its own element.
__device__ bool normalize(FitShared& sh, float* v, int t) {
  if (t == 0) {
    double sum = 0.0;
    for (int i = 0; i < kDim; ++i) {
      const double x = static_cast<double>(v[i]);
      sum += x * x;
    }
    const float norm = static_cast<float>(sqrt(sum));
    sh.flag = norm > FLT_EPSILON ? 1 : 0;
    sh.scalar = norm;
  }
  __syncthreads();
  const bool ok = sh.flag != 0;
  if (ok) v[t] = v[t] / sh.scalar;
  __syncthreads();
  return ok;
}

__global__ __launch_bounds__(kFitThreads) void boundary_fit_kernel(FitArgs a, StartVectors start) {
  extern __shared__ __align__(16) unsigned char dynamic[];
  FitShared& sh = *reinterpret_cast<FitShared*>(dynamic);
  const int t = threadIdx.x;
  const uint64_t head = blockIdx.x;
  const float* const dense = a.dense + head * kTile;

  bool finite = true;
  for (int row = 0; row < kDim; ++row) {
    const float v = dense[row * kDim + t];
    finite = finite && isfinite(v);
    sh.r[row * kRowStride + t] = v;
  }
  if (__syncthreads_and(finite) == 0) {  // uniform: the reference rejects the head
    if (t == 0) a.status[head] = kFitNonFiniteInput;
    return;
  }

  for (uint32_t rank = 0; rank < a.rank; ++rank) {
    sh.right[t] = start.value[rank][t];
    __syncthreads();
    if (!normalize(sh, sh.right, t)) {
      if (t == 0) sh.right[0] = 1.0f;
      __syncthreads();
    }
    for (int iteration = 0; iteration < kFitIterations; ++iteration) {
      {  // left[row] = sum over columns of R[row][col] * right[col] (thread = row)
        const float* row = sh.r + t * kRowStride;
        float acc = 0.0f;
        for (int column = 0; column < kDim; ++column) acc += row[column] * sh.right[column];
        sh.left[t] = acc;
      }
      __syncthreads();
      if (!normalize(sh, sh.left, t)) break;
      {  // right[col] = sum over rows of R[row][col] * left[row] (thread = column)
        float acc = 0.0f;
        for (int row = 0; row < kDim; ++row) acc += sh.r[row * kRowStride + t] * sh.left[row];
        sh.right[t] = acc;
      }
      __syncthreads();
      if (!normalize(sh, sh.right, t)) break;
    }
    // Singular value: one sequential sum over rows, then columns (:160-166).
    if (t == 0) {
      float singular = 0.0f;
      for (int row = 0; row < kDim; ++row) {
        const float l = sh.left[row];
        const float* r = sh.r + row * kRowStride;
        for (int column = 0; column < kDim; ++column) singular += l * r[column] * sh.right[column];
      }
      sh.scalar = singular;
    }
    __syncthreads();
    const float singular = sh.scalar;
    if (!isfinite(singular)) {  // uniform
      if (t == 0) a.status[head] = kFitNonFiniteSingular;
      return;
    }
    const float key = sh.left[t] * singular;
    a.comp_keys[(head * kDim + t) * a.rank + rank] = key;
    a.comp_values[(head * kDim + t) * a.rank + rank] = sh.right[t];
    {  // R[row][col] -= left[row] * sv * right[col] (thread = row)
      float* row = sh.r + t * kRowStride;
      for (int column = 0; column < kDim; ++column) row[column] -= key * sh.right[column];
    }
    __syncthreads();
  }

  float* const out = a.residual + head * kTile;
  for (int row = 0; row < kDim; ++row) out[row * kDim + t] = sh.r[row * kRowStride + t];
  if (t == 0) a.status[head] = kFitOk;
}

const StartVectors& start_vectors() {
  static const StartVectors table = [] {
    StartVectors s{};
    for (uint32_t rank = 0; rank < kMaxFitRank; ++rank) {
      for (int column = 0; column < kDim; ++column) {
        // Read through a volatile so that the compiler calls the library's
        // sinf, as the reference does, instead of folding the constant.
        volatile float argument = static_cast<float>((rank + 1) * (column + 1));
        s.value[rank][column] = std::sin(static_cast<float>(argument));
      }
    }
    return s;
  }();
  return table;
}

}  // namespace
}  // namespace gdn

// FromDenseBoundary's quantizer for a batch of [key][value] heads.
extern "C" int32_t statecentric_gdn_state_codec_quantize_boundary_launch_v1(
    void* stream, const float* dense, float* residual, int8_t* quantized, float* smoothing,
    float* value_scales, float* compensator_keys, float* compensator_values, int32_t* status,
    uint64_t heads, uint32_t rank) {
  if (dense == nullptr || residual == nullptr || quantized == nullptr || smoothing == nullptr ||
      value_scales == nullptr || status == nullptr || heads == 0 || heads > gdn::kMaxGrid ||
      rank > gdn::kMaxFitRank ||
      (rank > 0 && (compensator_keys == nullptr || compensator_values == nullptr)) ||
      !gdn::aligned16(dense, residual, quantized, smoothing, value_scales, compensator_keys,
                      compensator_values, status)) {
    return gdn::kStatusInvalidArgument;
  }
  const gdn::FitArgs args{dense, residual, compensator_keys, compensator_values, status, rank};
  const hipError_t attribute = hipFuncSetAttribute(
      reinterpret_cast<const void*>(gdn::boundary_fit_kernel),
      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(sizeof(gdn::FitShared)));
  if (attribute != hipSuccess) return gdn::kStatusLaunchFailed;
  void* kernel_args[] = {const_cast<gdn::FitArgs*>(&args),
                         const_cast<gdn::StartVectors*>(&gdn::start_vectors())};
  if (hipLaunchKernel(reinterpret_cast<const void*>(gdn::boundary_fit_kernel),
                      dim3(static_cast<uint32_t>(heads)), dim3(gdn::kFitThreads), kernel_args,
                      sizeof(gdn::FitShared), static_cast<hipStream_t>(stream)) != hipSuccess) {
    return gdn::kStatusLaunchFailed;
  }
  return statecentric_gdn_state_codec_encode_launch_v4(stream, residual, quantized, smoothing,
                                                      value_scales, heads, gdn::kKeyValue);
}
