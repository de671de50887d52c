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
// One 128-thread workgroup per head; thread t holds residual row t in 128
// VGPRs.  Row sums (left = R right, the singular value's products, the update)
// read the thread's own registers.  Column sums (right = R^T left) need the
// transpose: the rows are staged through LDS 64 at a time, column-major (a
// 34 KiB buffer, so four heads fit in a CU's LDS where the whole 66 KiB
// residual allowed two), and thread t sums column t in row order.  Each norm's terms are the exact
// double squares of the vector's elements, which their owners publish in LDS
// beside the vector; every thread then runs the reference's sequential sum over
// them.  The singular value's 16,384 products are formed by the row owners,
// staged 64 rows at a time, and summed in the reference's order by one lane.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <cfloat>
#include <cmath>
#include <type_traits>

#include "gdn_state_codec_kernel.h"
#include "launch.h"
#include "pipelined_sum.h"
#include "window_common.h"

namespace gdn {
namespace {

constexpr int kFitThreads = 128;
constexpr int kChunkRows = 64;               // rows staged in LDS at a time
constexpr int kChunkStride = kDim + 4;       // products: row starts 4 banks apart
constexpr int kColumnStride = kChunkRows + 4;  // staged rows, column-major
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
  // 64 staged rows, column-major (column c at c * kColumnStride), or 64 rows of
  // the singular value's products, row-major (row i at i * kChunkStride).
  float chunk[kDim * kColumnStride];
  double square[kDim];  // (double)v[i] * v[i] of the vector being normalized
  float left[kDim];
  float right[kDim];
  float total;          // the singular value's running sum
};
static_assert(workgroups_by_lds(sizeof(FitShared)) >= 4, "four heads per CU");

struct Float16 {
  float v[16];
};
struct Double8 {
  double v[8];
};

// Thread t's element v of a vector about to be normalized: its exact double
// square for the norm.  The caller's next barrier publishes it.
__device__ __forceinline__ void publish_square(FitShared& sh, int t, float v) {
  sh.square[t] = static_cast<double>(v) * static_cast<double>(v);
}

// Normalize (:60-65) of the published vector into out[]: the reference's Norm,
// a sequential double sum of the squares and a double square root rounded to
// float, evaluated identically by every thread; thread t then writes its own
// element v, divided when the norm exceeds FLT_EPSILON and unchanged otherwise
// (Normalize leaves the vector as it was).  The caller's next barrier
// publishes out[].
__device__ __forceinline__ bool normalize_into(const FitShared& sh, float* out, int t,
                                               float v, float* normalized) {
  double sum = 0.0;
  pipelined<kDim / 8, Double8>(
      [&](auto g, Double8& r) {
        unrolled<8>([&](auto i) { r.v[i] = sh.square[8 * decltype(g)::value + i]; });
      },
      [&](auto, const Double8& r) { unrolled<8>([&](auto i) { sum += r.v[i]; }); });
  const float norm = static_cast<float>(sqrt(sum));
  const bool ok = norm > FLT_EPSILON;
  *normalized = ok ? v / norm : v;
  out[t] = *normalized;
  return ok;
}

// The singular value's sequential sum over the staged products of 64 rows
// (row-major, the reference's order), by one lane, continuing from `total`.
// Segments of 16 products are read one ahead of the adds.
__device__ __forceinline__ float relay(const float* chunk, float total) {
  constexpr int kSegment = 16;
  constexpr int kPerRow = kDim / kSegment;
  constexpr int kSegments = kChunkRows * kPerRow;
  const auto load = [&](float (&seg)[kSegment], int s) {
    const float* src = chunk + (s / kPerRow) * kChunkStride + kSegment * (s % kPerRow);
    unrolled<kSegment / 4>([&](auto q) {
      constexpr int c = 4 * decltype(q)::value;
      const float4 v = *reinterpret_cast<const float4*>(src + c);
      seg[c] = v.x;
      seg[c + 1] = v.y;
      seg[c + 2] = v.z;
      seg[c + 3] = v.w;
    });
  };
  float a[kSegment], b[kSegment];
  load(a, 0);
  for (int s = 0; s < kSegments; s += 2) {
    load(b, s + 1);
    unrolled<kSegment>([&](auto c) { total += a[decltype(c)::value]; });
    if (s + 2 < kSegments) load(a, s + 2);
    unrolled<kSegment>([&](auto c) { total += b[decltype(c)::value]; });
  }
  return total;
}

__global__ __launch_bounds__(kFitThreads) __attribute__((amdgpu_waves_per_eu(2)))
void boundary_fit_kernel(FitArgs a, StartVectors start) {
  extern __shared__ __align__(16) unsigned char dynamic[];
  FitShared& sh = *reinterpret_cast<FitShared*>(dynamic);
  const int t = threadIdx.x;
  const uint64_t head = blockIdx.x;

  float row[kDim];
  bool finite = true;
  {
    const float4* src = reinterpret_cast<const float4*>(a.dense + head * kTile) + t * (kDim / 4);
    unrolled<kDim / 4>([&](auto q) {
      constexpr int c = 4 * decltype(q)::value;
      const float4 v = src[c / 4];
      row[c] = v.x;
      row[c + 1] = v.y;
      row[c + 2] = v.z;
      row[c + 3] = v.w;
      finite = finite && isfinite(v.x) && isfinite(v.y) && isfinite(v.z) && isfinite(v.w);
    });
  }
  if (__syncthreads_and(finite) == 0) {  // uniform: the reference rejects the head
    if (t == 0) a.status[head] = kFitNonFiniteInput;
    return;
  }

  for (uint32_t rank = 0; rank < a.rank; ++rank) {
    float my_left = 0.0f;
    float my_right;
    publish_square(sh, t, start.value[rank][t]);
    __syncthreads();
    if (!normalize_into(sh, sh.right, t, start.value[rank][t], &my_right) && t == 0) {
      sh.right[0] = 1.0f;
      my_right = 1.0f;
    }
    __syncthreads();
    for (int iteration = 0; iteration < kFitIterations; ++iteration) {
      {  // left[row] = sum over columns of R[row][col] * right[col] (thread = row)
        float acc = 0.0f;
        pipelined<kDim / 16, Float16>(
            [&](auto g, Float16& r) {
              unrolled<16>([&](auto i) { r.v[i] = sh.right[16 * decltype(g)::value + i]; });
            },
            [&](auto g, const Float16& r) {
              unrolled<16>([&](auto i) {
                acc += row[16 * decltype(g)::value + decltype(i)::value] * r.v[i];
              });
            });
        publish_square(sh, t, acc);
        __syncthreads();
        const bool left_ok = normalize_into(sh, sh.left, t, acc, &my_left);
        __syncthreads();
        if (!left_ok) break;  // uniform: every thread formed the same norm
      }
      {  // right[col] = sum over rows of R[row][col] * left[row] (thread = column),
         // the rows staged through LDS 64 at a time
        float acc = 0.0f;
        unrolled<kDim / kChunkRows>([&](auto h) {
          constexpr int first = decltype(h)::value * kChunkRows;
          if (h > 0) __syncthreads();  // every thread done with the previous rows
          if (t / kChunkRows == decltype(h)::value) {
            // Column-major, one 4-byte write per value from a single base
            // address (volatile, so none are merged): contiguous writes are
            // merged into 16-byte ones, which need the row in aligned register
            // quads, and paired 4-byte writes need a base address per few
            // columns, which the compiler keeps live through the whole loop.
            typedef __attribute__((address_space(3))) float LdsFloat;
            volatile LdsFloat* dst =
                (volatile LdsFloat*)(sh.chunk + t % kChunkRows);
            unrolled<kDim>([&](auto c) {
              dst[decltype(c)::value * kColumnStride] = row[decltype(c)::value];
            });
          }
          __syncthreads();
          struct Pair8 {
            float r[8];
            float l[8];
          };
          const float* column = sh.chunk + t * kColumnStride;
          pipelined<kChunkRows / 8, Pair8>(
              [&](auto g, Pair8& p) {
                unrolled<8>([&](auto i) {
                  constexpr int r = 8 * decltype(g)::value + decltype(i)::value;
                  p.r[i] = column[r];
                  p.l[i] = sh.left[first + r];
                });
              },
              [&](auto, const Pair8& p) {
                unrolled<8>([&](auto i) { acc += p.r[i] * p.l[i]; });
              });
        });
        publish_square(sh, t, acc);
        __syncthreads();
        const bool right_ok = normalize_into(sh, sh.right, t, acc, &my_right);
        __syncthreads();
        if (!right_ok) break;
      }
    }
    // Singular value (:160-166): row t's products (left[t] * R[t][col]) *
    // right[col], staged 64 rows at a time and summed by one lane in the
    // reference's order, rows 0..127, columns 0..127 within each row.
    unrolled<kDim / kChunkRows>([&](auto h) {
      constexpr int half = decltype(h)::value;
      if (t / kChunkRows == half) {
        float* dst = sh.chunk + (t % kChunkRows) * kChunkStride;
        pipelined<kDim / 16, Float16>(
            [&](auto g, Float16& r) {
              unrolled<16>([&](auto i) { r.v[i] = sh.right[16 * decltype(g)::value + i]; });
            },
            [&](auto g, const Float16& r) {
              unrolled<4>([&](auto q) {
                constexpr int c = 16 * decltype(g)::value + 4 * decltype(q)::value;
                constexpr int i = 4 * decltype(q)::value;
                *reinterpret_cast<float4*>(dst + c) = make_float4(
                    my_left * row[c] * r.v[i], my_left * row[c + 1] * r.v[i + 1],
                    my_left * row[c + 2] * r.v[i + 2], my_left * row[c + 3] * r.v[i + 3]);
              });
            });
      }
      __syncthreads();
      if (t == half * kChunkRows) sh.total = relay(sh.chunk, half == 0 ? 0.0f : sh.total);
      __syncthreads();
    });
    const float singular = sh.total;
    if (!isfinite(singular)) {  // uniform
      if (t == 0) a.status[head] = kFitNonFiniteSingular;
      return;
    }
    const float key = my_left * singular;
    // Uniform per-head bases and 32-bit lane offsets (no 64-bit lane addresses
    // held through the loop).
    const uint32_t slot = static_cast<uint32_t>(t) * a.rank + rank;
    (a.comp_keys + head * kDim * a.rank)[slot] = key;
    (a.comp_values + head * kDim * a.rank)[slot] = my_right;
    // R[row][col] -= left[row] * sv * right[col] (thread = row)
    pipelined<kDim / 16, Float16>(
        [&](auto g, Float16& r) {
          unrolled<16>([&](auto i) { r.v[i] = sh.right[16 * decltype(g)::value + i]; });
        },
        [&](auto g, const Float16& r) {
          unrolled<16>([&](auto i) {
            row[16 * decltype(g)::value + decltype(i)::value] -= key * r.v[i];
          });
        });
    __syncthreads();  // right[] and the chunk are rewritten by the next rank
  }

  float4* out = reinterpret_cast<float4*>(a.residual + head * kTile) + t * (kDim / 4);
  unrolled<kDim / 4>([&](auto q) {
    constexpr int c = 4 * decltype(q)::value;
    out[c / 4] = make_float4(row[c], row[c + 1], row[c + 2], row[c + 3]);
  });
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
  const void* const kernel = reinterpret_cast<const void*>(gdn::boundary_fit_kernel);
  const hipError_t attribute = hipFuncSetAttribute(
      kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
      static_cast<int>(sizeof(gdn::FitShared)));
  if (attribute != hipSuccess) return gdn::kStatusLaunchFailed;
  void* kernel_args[] = {const_cast<gdn::FitArgs*>(&args),
                         const_cast<gdn::StartVectors*>(&gdn::start_vectors())};
  if (hipLaunchKernel(kernel,
                      dim3(static_cast<uint32_t>(heads)), dim3(gdn::kFitThreads), kernel_args,
                      sizeof(gdn::FitShared), static_cast<hipStream_t>(stream)) != hipSuccess) {
    return gdn::kStatusLaunchFailed;
  }
  return statecentric_gdn_state_codec_encode_launch_v4(stream, residual, quantized, smoothing,
                                                      value_scales, heads, gdn::kKeyValue);
}
