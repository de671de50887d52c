// The exact-SVD boundary initializer: the reference runtime's
// GdnStateCodecRuntime._encode_dense_boundary(dense, "exact_svd")
// (src/gdn_state_codec/runtime.py:335-389), which takes the rank-4 truncated
// SVD of each dense [key][value] head D with torch.linalg.svd,
//   compensator_keys[k][r] = U[k][r] * S[r],   compensator_values[v][r] = V[v][r]
// (r = 0..3 by decreasing singular value, stored as fp16), quantizes the fp32
// residual D - keys * values^T and stores the codes in [value][key] order.
//
// The SVD here is a one-sided Jacobi (Hestenes) iteration on the provider
// tile P = D^T ([value][key], as the runtime holds it): rotating pairs of P's
// rows until every pair is orthogonal turns row v into u_v * s_v, so the four
// rows of largest norm are the four left singular vectors times their singular
// values, i.e. the compensator keys, and the matching right singular vectors
// are D^T u = P w, normalized.  The decomposition is unique only up to the
// signs of each (u, v) pair and, for equal singular values, the basis of
// their subspace; the product keys * values^T, which is all the codec uses,
// is not.  The residual then goes through the batched quant-only encode
// (codec.hip) in the provider layout.
//
// One 512-thread workgroup per head.  The 128 rows live in LDS in double
// (stride 130, so every row starts 16-byte aligned; 130 KiB, one workgroup
// per CU).  A sweep visits every pair of rows once in 127 rounds of 64
// disjoint pairs (the round-robin tournament: in round r, row 127 meets row r
// and row (r + p) mod 127 meets (r - p) mod 127 for p = 1..63); eight lanes
// serve one pair, each holding 16 values of both rows.  The time is the
// rounds' dependent latency, not issue: two waves per SIMD and short sums
// (two accumulators per lane) hide part of it.  The rotation follows
// Rutishauser's formula for the smaller angle.  Everything up to the outputs
// is double: with fp32 rows the rounding of the rotations, amplified by the
// gap between the fourth and fifth singular values (1-5% on Gaussian heads),
// left the rank-4 product 1e-5..6e-5 of the largest singular value off; in
// double it is the fp32 rounding of the outputs.  Before the sweeps the head
// is scaled by a power of two so that its largest magnitude lies in [1/2, 1),
// and the scaling is undone exactly on the keys.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "gdn_state_codec_kernel.h"
#include "lane_exchange.h"
#include "launch.h"
#include "window_common.h"

namespace gdn {
namespace {

constexpr int kSvdThreads = 512;
constexpr int kLanesPerPair = 8;
constexpr int kSvdRowStride = kDim + 2;  // doubles
constexpr int kRounds = kDim - 1;          // rounds per sweep (128 rows, odd 127)
constexpr int kSpan = kDim / kLanesPerPair;  // values of a row per lane
constexpr int kMaxSweeps = 30;
constexpr int kSvdRank = 4;
// A pair is rotated when its cosine exceeds 2^-36; this converges in 10-13
// sweeps on the test heads.
constexpr double kCosineTolerance = 0x1p-36;
// Rows whose squared norm (after scaling) is below 2^-96 -- every value below
// 2^-48 of the head's largest -- are taken as converged: their share of any
// singular value is below the fp32 rounding of the outputs.
constexpr double kNegligibleSquare = 0x1p-96;

// Per-head outcomes written to `status`.
constexpr int32_t kSvdOk = 0;
constexpr int32_t kSvdNonFiniteInput = 1;
constexpr int32_t kSvdNotConverged = 2;  // a rotation still happened in the last sweep

struct SvdArgs {
  const float* provider;   // [heads][value][key]
  float* residual;         // [heads][value][key]
  uint16_t* keys;          // fp16 [heads][key][4]
  uint16_t* values;        // fp16 [heads][value][4]
  int32_t* status;         // [heads]
  int max_sweeps;          // 1..kMaxSweeps
};

struct SvdShared {
  double w[kDim * kSvdRowStride];  // the rows being orthogonalized
  double norm[kDim];              // their squared norms after the sweeps
  double y[kSvdRank][kDim];       // P w_r for the four selected rows
  double y_norm[kSvdRank];
  float right[kDim][kSvdRank];
  float wave_max[kSvdThreads / 64];
  int top[kSvdRank];
};

// x * 2^-exponent in double (exact for every fp32 x).
__device__ __forceinline__ double scaled(float x, int exponent) {
  return ldexp(static_cast<double>(x), -exponent);
}

__global__ __launch_bounds__(kSvdThreads) void exact_svd_kernel(SvdArgs a) {
  extern __shared__ __align__(16) unsigned char dynamic[];
  SvdShared& sh = *reinterpret_cast<SvdShared*>(dynamic);
  const int t = threadIdx.x;
  const uint64_t head = blockIdx.x;
  const float* const p = a.provider + head * kTile;

  // ---- load, finiteness, largest magnitude --------------------------------
  constexpr int kLoads = kTile / 4 / kSvdThreads;  // 8 float4 per thread
  float4 v[kLoads];
#pragma unroll
  for (int i = 0; i < kLoads; ++i) v[i] = reinterpret_cast<const float4*>(p)[i * kSvdThreads + t];
  bool finite = true;
  float largest = 0.0f;
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    finite = finite && isfinite(v[i].x) && isfinite(v[i].y) && isfinite(v[i].z) &&
             isfinite(v[i].w);
    largest = fmaxf(largest, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)),
                                   fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
  }
  if (__syncthreads_and(finite) == 0) {  // uniform
    if (t == 0) a.status[head] = kSvdNonFiniteInput;
    return;
  }
  largest = wave_max(largest);
  if ((t & 63) == 0) sh.wave_max[t >> 6] = largest;
  __syncthreads();
  largest = sh.wave_max[0];
#pragma unroll
  for (int w = 1; w < kSvdThreads / 64; ++w) largest = fmaxf(largest, sh.wave_max[w]);
  int exponent = 0;  // largest = f * 2^exponent, f in [1/2, 1)
  frexpf(largest, &exponent);
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    const int f = i * kSvdThreads + t;  // float4 index: row f / 32, column 4 (f % 32)
    double* const to = sh.w + (f >> 5) * kSvdRowStride + 4 * (f & 31);
    *reinterpret_cast<double2*>(to) = make_double2(scaled(v[i].x, exponent),
                                                   scaled(v[i].y, exponent));
    *reinterpret_cast<double2*>(to + 2) = make_double2(scaled(v[i].z, exponent),
                                                       scaled(v[i].w, exponent));
  }
  __syncthreads();

  // ---- Jacobi sweeps ------------------------------------------------------
  const int pair = t / kLanesPerPair;
  const int lane = t % kLanesPerPair;
  bool converged = false;
  for (int sweep = 0; sweep < a.max_sweeps; ++sweep) {
    bool rotated = false;
    for (int round = 0; round < kRounds; ++round) {
      int first = kDim - 1, second = round;
      if (pair != 0) {
        first = round + pair;
        if (first >= kRounds) first -= kRounds;
        second = round - pair;
        if (second < 0) second += kRounds;
      }
      double* const row_a = sh.w + first * kSvdRowStride;
      double* const row_b = sh.w + second * kSvdRowStride;
      double x[kSpan], y[kSpan];
#pragma unroll
      for (int e = 0; e < kSpan / 2; ++e) {  // double2 chunks lane, lane + 8, ...
        const double2 xa = *reinterpret_cast<const double2*>(row_a + 2 * (lane + 8 * e));
        const double2 yb = *reinterpret_cast<const double2*>(row_b + 2 * (lane + 8 * e));
        x[2 * e] = xa.x, x[2 * e + 1] = xa.y;
        y[2 * e] = yb.x, y[2 * e + 1] = yb.y;
      }
      double a2[2] = {0.0, 0.0}, b2[2] = {0.0, 0.0}, g2[2] = {0.0, 0.0};
#pragma unroll
      for (int i = 0; i < kSpan; ++i) {
        a2[i & 1] = fma(x[i], x[i], a2[i & 1]);
        b2[i & 1] = fma(y[i], y[i], b2[i & 1]);
        g2[i & 1] = fma(x[i], y[i], g2[i & 1]);
      }
      double alpha = a2[0] + a2[1], beta = b2[0] + b2[1], gamma = g2[0] + g2[1];
      // The pair's eight lanes add their partial sums in the same commuted
      // order, so all eight hold identical totals and take the same branch.
      alpha += dpp_xor<1>(alpha), beta += dpp_xor<1>(beta), gamma += dpp_xor<1>(gamma);
      alpha += dpp_xor<2>(alpha), beta += dpp_xor<2>(beta), gamma += dpp_xor<2>(gamma);
      alpha += dpp_xor<4>(alpha), beta += dpp_xor<4>(beta), gamma += dpp_xor<4>(gamma);
      const bool active = alpha > kNegligibleSquare && beta > kNegligibleSquare &&
                          gamma * gamma > kCosineTolerance * kCosineTolerance * alpha * beta;
      if (active) {
        // Rotate (x, y) -> (c x - s y, s x + c y) by the angle of magnitude
        // at most pi/4 that makes the rows orthogonal: t = s/c solves
        // t^2 + 2 zeta t - 1 = 0 with zeta = (beta - alpha) / (2 gamma), and
        // the smaller root sign(zeta) / (|zeta| + sqrt(1 + zeta^2)), times
        // |2 gamma| above and below, is 2 gamma sign(d) / (|d| + sqrt(d^2 +
        // 4 gamma^2)) with d = beta - alpha: one dependent division fewer.
        // After the head's scaling alpha, beta <= 128 and gamma^2 > 2^-264, so
        // neither square overflows or underflows.
        const double d = beta - alpha;
        const double two_gamma = 2.0 * gamma;
        // sign(zeta) |2 gamma| = 2 gamma sign(d), with sign(+0) = +1 (for
        // d = 0, zeta = +0 / (2 gamma) carries the sign of gamma).
        const double tangent = (d < 0.0 ? -two_gamma : two_gamma) /
                               (fabs(d) + sqrt(fma(d, d, two_gamma * two_gamma)));
        const double c = 1.0 / sqrt(fma(tangent, tangent, 1.0));
        const double s = c * tangent;
#pragma unroll
        for (int i = 0; i < kSpan; ++i) {
          const double xi = x[i], yi = y[i];
          x[i] = fma(c, xi, -(s * yi));
          y[i] = fma(s, xi, c * yi);
        }
#pragma unroll
        for (int e = 0; e < kSpan / 2; ++e) {
          *reinterpret_cast<double2*>(row_a + 2 * (lane + 8 * e)) =
              make_double2(x[2 * e], x[2 * e + 1]);
          *reinterpret_cast<double2*>(row_b + 2 * (lane + 8 * e)) =
              make_double2(y[2 * e], y[2 * e + 1]);
        }
        rotated = true;
      }
      __syncthreads();
    }
    if (__syncthreads_or(rotated) == 0) {  // uniform
      converged = true;
      break;
    }
  }

  // ---- the four rows of largest norm --------------------------------------
  if (t < kDim) {
    const double* const row = sh.w + t * kSvdRowStride;
    double sum = 0.0;
    for (int k = 0; k < kDim; ++k) sum = fma(row[k], row[k], sum);
    sh.norm[t] = sum;
  }
  __syncthreads();
  if (t == 0) {
    // Decreasing norm; equal norms in increasing row order.
    uint64_t taken[2] = {0, 0};
    for (int r = 0; r < kSvdRank; ++r) {
      int best = 0;
      double best_norm = -1.0;
      for (int row = 0; row < kDim; ++row) {
        const bool used = (taken[row >> 6] >> (row & 63)) & 1u;
        if (!used && sh.norm[row] > best_norm) best_norm = sh.norm[row], best = row;
      }
      taken[best >> 6] |= uint64_t{1} << (best & 63);
      sh.top[r] = best;
    }
  }
  __syncthreads();
  int top[kSvdRank];
#pragma unroll
  for (int r = 0; r < kSvdRank; ++r) top[r] = sh.top[r];

  // ---- right vectors: y_r = P w_r (scaled P), four lanes per row ----------
  static_assert(kSvdThreads == 4 * kDim, "four lanes per row");
  {
    const int row = t >> 2;
    const int part = t & 3;  // keys 32 part .. 32 part + 31
    const float4* const source = reinterpret_cast<const float4*>(p + row * kDim + 32 * part);
    double acc[kSvdRank] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll 4
    for (int j = 0; j < 8; ++j) {
      const float4 q = source[j];
      const double qs[4] = {scaled(q.x, exponent), scaled(q.y, exponent),
                            scaled(q.z, exponent), scaled(q.w, exponent)};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int k = 32 * part + 4 * j + c;
#pragma unroll
        for (int r = 0; r < kSvdRank; ++r) {
          acc[r] = fma(qs[c], sh.w[top[r] * kSvdRowStride + k], acc[r]);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < kSvdRank; ++r) {
      acc[r] += dpp_xor<1>(acc[r]);
      acc[r] += dpp_xor<2>(acc[r]);
      if (part == 0) sh.y[r][row] = acc[r];
    }
  }
  __syncthreads();
  if (t < kSvdRank) {
    double sum = 0.0;
    for (int row = 0; row < kDim; ++row) sum = fma(sh.y[t][row], sh.y[t][row], sum);
    sh.y_norm[t] = sqrt(sum);
  }
  __syncthreads();
  if (t < kDim) {
    uint32_t bits[kSvdRank];
#pragma unroll
    for (int r = 0; r < kSvdRank; ++r) {
      // A zero product (a head of rank below r + 1 whose row r is zero)
      // leaves a zero vector; its key is zero as well.
      const double n = sh.y_norm[r];
      const float right = n > 0.0 ? static_cast<float>(sh.y[r][t] / n) : 0.0f;
      sh.right[t][r] = right;
      bits[r] = float_to_half_bits(right);
    }
    *reinterpret_cast<uint2*>(a.values + (head * kDim + t) * kSvdRank) =
        make_uint2(bits[0] | (bits[1] << 16), bits[2] | (bits[3] << 16));
  }

  // ---- keys and residual ----------------------------------------------------
  const int key = t & (kDim - 1);
  float left[kSvdRank];
#pragma unroll
  for (int r = 0; r < kSvdRank; ++r) {
    left[r] = static_cast<float>(ldexp(sh.w[top[r] * kSvdRowStride + key], exponent));
  }
  if (t < kDim) {
    uint32_t bits[kSvdRank];
#pragma unroll
    for (int r = 0; r < kSvdRank; ++r) bits[r] = float_to_half_bits(left[r]);
    *reinterpret_cast<uint2*>(a.keys + (head * kDim + key) * kSvdRank) =
        make_uint2(bits[0] | (bits[1] << 16), bits[2] | (bits[3] << 16));
  }
  __syncthreads();  // sh.right
  float* const out = a.residual + head * kTile;
  for (int row = t >> 7; row < kDim; row += kSvdThreads / kDim) {
    float fit = left[0] * sh.right[row][0];
#pragma unroll
    for (int r = 1; r < kSvdRank; ++r) fit = fmaf(left[r], sh.right[row][r], fit);
    out[row * kDim + key] = p[row * kDim + key] - fit;
  }
  // An unconverged head still gets the fit of its last sweep, flagged.
  if (t == 0) a.status[head] = converged ? kSvdOk : kSvdNotConverged;
}

}  // namespace
}  // namespace gdn

namespace gdn {
namespace {

int32_t launch_exact_svd(void* stream, const float* provider, float* residual,
                         int8_t* quantized, float* smoothing, float* value_scales,
                         uint16_t* compensator_keys, uint16_t* compensator_values,
                         int32_t* status, uint64_t heads, uint32_t max_sweeps) {
  if (provider == nullptr || residual == nullptr || quantized == nullptr ||
      smoothing == nullptr || value_scales == nullptr || compensator_keys == nullptr ||
      compensator_values == nullptr || status == nullptr || heads == 0 || heads > kMaxGrid ||
      max_sweeps == 0 || max_sweeps > static_cast<uint32_t>(kMaxSweeps) ||
      !aligned16(provider, residual, quantized, smoothing, value_scales, compensator_keys,
                 compensator_values, status)) {
    return kStatusInvalidArgument;
  }
  const SvdArgs args{provider, residual, compensator_keys, compensator_values, status,
                     static_cast<int>(max_sweeps)};
  const hipError_t attribute = hipFuncSetAttribute(
      reinterpret_cast<const void*>(exact_svd_kernel),
      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(sizeof(SvdShared)));
  if (attribute != hipSuccess) return kStatusLaunchFailed;
  void* kernel_args[] = {const_cast<SvdArgs*>(&args)};
  if (hipLaunchKernel(reinterpret_cast<const void*>(exact_svd_kernel),
                      dim3(static_cast<uint32_t>(heads)), dim3(kSvdThreads), kernel_args,
                      sizeof(SvdShared), static_cast<hipStream_t>(stream)) != hipSuccess) {
    return kStatusLaunchFailed;
  }
  return statecentric_gdn_state_codec_encode_launch_v4(stream, residual, quantized, smoothing,
                                                      value_scales, heads, kValueKey);
}

}  // namespace
}  // namespace gdn

// The exact-SVD initializer for a batch of provider heads.
extern "C" int32_t statecentric_gdn_state_codec_exact_svd_boundary_launch_v1(
    void* stream, const float* provider, float* residual, int8_t* quantized, float* smoothing,
    float* value_scales, uint16_t* compensator_keys, uint16_t* compensator_values,
    int32_t* status, uint64_t heads) {
  return gdn::launch_exact_svd(stream, provider, residual, quantized, smoothing, value_scales,
                               compensator_keys, compensator_values, status, heads,
                               gdn::kMaxSweeps);
}

// The same with a caller-chosen sweep limit.
extern "C" int32_t statecentric_gdn_state_codec_exact_svd_boundary_sweeps_launch_v1(
    void* stream, const float* provider, float* residual, int8_t* quantized, float* smoothing,
    float* value_scales, uint16_t* compensator_keys, uint16_t* compensator_values,
    int32_t* status, uint64_t heads, uint32_t max_sweeps) {
  return gdn::launch_exact_svd(stream, provider, residual, quantized, smoothing, value_scales,
                               compensator_keys, compensator_values, status, heads, max_sweeps);
}
