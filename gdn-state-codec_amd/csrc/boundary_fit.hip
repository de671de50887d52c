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
// column (right = R^T left) both read it without bank conflicts.  Each of
// those sums runs on its own thread with its 128 loads unrolled ahead of the
// chain.  Every thread evaluates each norm identically from LDS (no broadcast,
// one barrier fewer) and writes its normalized element to the vector's other
// buffer.  The singular value's 16,384 products are formed in parallel, one row
// per thread in registers, and summed in the reference's order by a relay:
// row r's thread adds its 128 products to the total of rows 0..r-1.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <cfloat>
#include <cmath>
#include <type_traits>

#include "gdn_state_codec_kernel.h"
#include "launch.h"
#include "window_common.h"

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
  float raw[kDim];     // a matrix-vector product before its normalization
  float left[kDim];
  float right[kDim];
  float total;         // the singular value's running sum
};

// f(std::integral_constant<int, i>) for i = 0 .. kCount - 1, expanded at
// compile time, so that register arrays indexed by i stay in VGPRs and the
// loads of a whole sum can be issued ahead of its dependent chain.
template <int kCount, int kIndex = 0, typename F>
__device__ __forceinline__ void unrolled(F&& f) {
  if constexpr (kIndex < kCount) {
    f(std::integral_constant<int, kIndex>{});
    unrolled<kCount, kIndex + 1>(f);
  }
}

// Normalize (:60-65) of raw[0..127] into out[]: the reference's Norm, a
// sequential double sum of squares (each square exact in double) and a
// double square root rounded to float, evaluated identically by every thread;
// each thread then writes its own element, divided when the norm exceeds
// FLT_EPSILON and copied unchanged otherwise (Normalize leaves the vector as
// it was).  The caller has made raw[] visible; the caller's next barrier
// publishes out[].
__device__ __forceinline__ bool normalize_into(const float* raw, float* out, int t) {
  double sum = 0.0;
  unrolled<kDim>([&](auto i) {
    const double x = static_cast<double>(raw[decltype(i)::value]);
    sum += x * x;
  });
  const float norm = static_cast<float>(sqrt(sum));
  const bool ok = norm > FLT_EPSILON;
  out[t] = ok ? raw[t] / norm : raw[t];
  return ok;
}

__global__ __launch_bounds__(kFitThreads) __attribute__((amdgpu_waves_per_eu(1, 2)))
void boundary_fit_kernel(FitArgs a, StartVectors start) {
  extern __shared__ __align__(16) unsigned char dynamic[];
  FitShared& sh = *reinterpret_cast<FitShared*>(dynamic);
  const int t = threadIdx.x;
  const uint64_t head = blockIdx.x;
  const float* const dense = a.dense + head * kTile;
  float* const my_row = sh.r + t * kRowStride;

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
    sh.raw[t] = start.value[rank][t];
    __syncthreads();
    if (!normalize_into(sh.raw, sh.right, t) && t == 0) sh.right[0] = 1.0f;
    __syncthreads();
    for (int iteration = 0; iteration < kFitIterations; ++iteration) {
      {  // left[row] = sum over columns of R[row][col] * right[col] (thread = row)
        float acc = 0.0f;
        unrolled<kDim>([&](auto c) {
          constexpr int column = decltype(c)::value;
          acc += my_row[column] * sh.right[column];
        });
        sh.raw[t] = acc;
      }
      __syncthreads();
      const bool left_ok = normalize_into(sh.raw, sh.left, t);
      __syncthreads();
      if (!left_ok) break;  // uniform: every thread formed the same norm
      {  // right[col] = sum over rows of R[row][col] * left[row] (thread = column)
        float acc = 0.0f;
        unrolled<kDim>([&](auto r) {
          constexpr int row = decltype(r)::value;
          acc += sh.r[row * kRowStride + t] * sh.left[row];
        });
        sh.raw[t] = acc;
      }
      __syncthreads();
      const bool right_ok = normalize_into(sh.raw, sh.right, t);
      __syncthreads();
      if (!right_ok) break;
    }
    // Singular value (:160-166): thread t forms row t's products
    // (left[t] * R[t][col]) * right[col]; the relay then adds them in the
    // reference's order, rows 0..127, columns 0..127 within each row.
    float product[kDim];
    {
      const float l = sh.left[t];
      unrolled<kDim>([&](auto c) {
        constexpr int column = decltype(c)::value;
        product[column] = l * my_row[column] * sh.right[column];
      });
    }
    for (int row = 0; row < kDim; ++row) {
      if (row == kDim / 2) __syncthreads();  // the relay passes from wavefront 0 to 1
      if (t == row) {
        float total = row == 0 ? 0.0f : sh.total;
        unrolled<kDim>([&](auto c) { total += product[decltype(c)::value]; });
        sh.total = total;
      }
      wave_lds_sync();  // lane row's total before lane row + 1 reads it
    }
    __syncthreads();
    const float singular = sh.total;
    if (!isfinite(singular)) {  // uniform
      if (t == 0) a.status[head] = kFitNonFiniteSingular;
      return;
    }
    const float key = sh.left[t] * singular;
    a.comp_keys[(head * kDim + t) * a.rank + rank] = key;
    a.comp_values[(head * kDim + t) * a.rank + rank] = sh.right[t];
    // R[row][col] -= left[row] * sv * right[col] (thread = row)
    unrolled<kDim>([&](auto c) {
      constexpr int column = decltype(c)::value;
      my_row[column] -= key * sh.right[column];
    });
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
