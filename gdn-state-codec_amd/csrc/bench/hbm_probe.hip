// HBM bandwidth probes used by bench.py (not part of the codec's C-ABI).
//
// Streaming kernels with the codec's access granularity (16-byte
// vector loads/stores, 256-thread workgroups, one contiguous 4 KiB chunk per
// workgroup iteration): copy, read-only and write-only, each with plain and
// with nontemporal accesses (the hint the codec kernels use).  They give the
// bandwidth this GPU actually sustains, and the plain copy kernel is the
// known-size reference that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings.
// Each probe also runs in the XCD-contiguous order of the codec kernels
// (xcd_contiguous_item in launch.h: XCD x streams the x-th eighth of the
// buffer) beside the dispatcher's interleaved order.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "launch.h"
#include "stream_memory.h"

namespace {

template <bool kNontemporal>
__device__ __forceinline__ uint4 load16(const uint4* p) {
  if constexpr (kNontemporal) return gdn::stream_load(p);
  return *p;
}

template <bool kNontemporal>
__device__ __forceinline__ void store16(uint4* p, uint4 v) {
  if constexpr (kNontemporal) {
    gdn::stream_store(reinterpret_cast<float4*>(p),
                      make_float4(__uint_as_float(v.x), __uint_as_float(v.y),
                                  __uint_as_float(v.z), __uint_as_float(v.w)));
  } else {
    *p = v;
  }
}

constexpr int kThreads = 256;
constexpr int kUnroll = 4;  // 16-byte accesses in flight per thread

template <bool kNontemporal, bool kXcd>
__global__ __launch_bounds__(kThreads) void copy_kernel(const uint4* __restrict__ src,
                                                        uint4* __restrict__ dst,
                                                        uint64_t vectors) {
  // Interleaved: the grid strides over the whole buffer.  XCD-contiguous:
  // workgroup b (XCD b % 8) strides over the (b % 8)-th eighth with the
  // workgroups of its XCD (the grid and the vector count are multiples of 8).
  const uint64_t groups = kXcd ? gridDim.x / 8 : gridDim.x;
  const uint64_t member = kXcd ? blockIdx.x / 8 : blockIdx.x;
  const uint64_t begin = kXcd ? (blockIdx.x % 8) * (vectors / 8) : 0;
  const uint64_t end = kXcd ? begin + vectors / 8 : vectors;
  const uint64_t stride = groups * kThreads * kUnroll;
  for (uint64_t base = begin + member * kThreads * kUnroll + threadIdx.x; base < end;
       base += stride) {
    uint4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint64_t i = base + static_cast<uint64_t>(u) * kThreads;
      if (i < end) v[u] = load16<kNontemporal>(src + i);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint64_t i = base + static_cast<uint64_t>(u) * kThreads;
      if (i < end) store16<kNontemporal>(dst + i, v[u]);
    }
  }
}

template <bool kNontemporal, bool kXcd>
__global__ __launch_bounds__(kThreads) void read_kernel(const uint4* __restrict__ src,
                                                        uint32_t* __restrict__ sink,
                                                        uint64_t vectors) {
  // Interleaved: the grid strides over the whole buffer.  XCD-contiguous:
  // workgroup b (XCD b % 8) strides over the (b % 8)-th eighth with the
  // workgroups of its XCD (the grid and the vector count are multiples of 8).
  const uint64_t groups = kXcd ? gridDim.x / 8 : gridDim.x;
  const uint64_t member = kXcd ? blockIdx.x / 8 : blockIdx.x;
  const uint64_t begin = kXcd ? (blockIdx.x % 8) * (vectors / 8) : 0;
  const uint64_t end = kXcd ? begin + vectors / 8 : vectors;
  const uint64_t stride = groups * kThreads * kUnroll;
  uint32_t acc = 0;
  for (uint64_t base = begin + member * kThreads * kUnroll + threadIdx.x; base < end;
       base += stride) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint64_t i = base + static_cast<uint64_t>(u) * kThreads;
      if (i < end) {
        const uint4 v = load16<kNontemporal>(src + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
      }
    }
  }
  // One word per thread keeps the loads live; the sink holds gridDim*256 words.
  sink[static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x] = acc;
}

template <bool kNontemporal, bool kXcd>
__global__ __launch_bounds__(kThreads) void write_kernel(uint4* __restrict__ dst,
                                                         uint64_t vectors,
                                                         uint32_t value) {
  // Interleaved: the grid strides over the whole buffer.  XCD-contiguous:
  // workgroup b (XCD b % 8) strides over the (b % 8)-th eighth with the
  // workgroups of its XCD (the grid and the vector count are multiples of 8).
  const uint64_t groups = kXcd ? gridDim.x / 8 : gridDim.x;
  const uint64_t member = kXcd ? blockIdx.x / 8 : blockIdx.x;
  const uint64_t begin = kXcd ? (blockIdx.x % 8) * (vectors / 8) : 0;
  const uint64_t end = kXcd ? begin + vectors / 8 : vectors;
  const uint64_t stride = groups * kThreads * kUnroll;
  const uint4 v = make_uint4(value, value, value, value);
  for (uint64_t base = begin + member * kThreads * kUnroll + threadIdx.x; base < end;
       base += stride) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint64_t i = base + static_cast<uint64_t>(u) * kThreads;
      if (i < end) store16<kNontemporal>(dst + i, v);
    }
  }
}

// Tile-shaped mixed streams with the codec's exact access pattern, one
// 256-thread workgroup per 128 x 128 tile: thread t touches rows
// 8j + t / 32 (j = 0..15), four consecutive columns 4 (t % 32)..+3 of each.
//   expand   (1:4 read:write, the dequantize's mix): 16 KiB of bytes in, each
//            byte widened to an fp32 value, 64 KiB out; a 4-byte load and a
//            16-byte store per row.
//   halve    (2:1, the bf16 pool encode's mix): 32 KiB of bf16 in, each
//            value's low byte kept, 16 KiB out; an 8-byte load and a 4-byte
//            store per row.
//   contract (4:1, the quantize's mix): 64 KiB of fp32 in, each value's low
//            byte kept, 16 KiB out; a 16-byte load and a 4-byte store per row.
// Loads are all issued before the stores, as in the codec kernels.
constexpr int kTileDim = 128;
constexpr int kRowsPerThread = 16;

template <bool kNontemporal, bool kXcd>
__global__ __launch_bounds__(kThreads) void expand_kernel(const uint32_t* __restrict__ src,
                                                          float4* __restrict__ dst) {
  const uint64_t tile = kXcd ? gdn::xcd_contiguous_item(blockIdx.x, gridDim.x) : blockIdx.x;
  const int row0 = threadIdx.x >> 5;
  const int quad = threadIdx.x & 31;
  const uint32_t* in = src + tile * (kTileDim * kTileDim / 4);
  float4* out = dst + tile * (kTileDim * kTileDim / 4);
  uint32_t w[kRowsPerThread];
#pragma unroll
  for (int j = 0; j < kRowsPerThread; ++j) {
    const uint32_t* p = in + (8 * j + row0) * (kTileDim / 4) + quad;
    w[j] = kNontemporal ? __builtin_nontemporal_load(p) : *p;
  }
#pragma unroll
  for (int j = 0; j < kRowsPerThread; ++j) {
    const float4 v = make_float4(static_cast<float>(w[j] & 0xFFu),
                                 static_cast<float>((w[j] >> 8) & 0xFFu),
                                 static_cast<float>((w[j] >> 16) & 0xFFu),
                                 static_cast<float>(w[j] >> 24));
    float4* q = out + (8 * j + row0) * (kTileDim / 4) + quad;
    if (kNontemporal) {
      gdn::stream_store(q, v);
    } else {
      *q = v;
    }
  }
}

template <bool kNontemporal, bool kXcd>
__global__ __launch_bounds__(kThreads) void contract_kernel(const uint4* __restrict__ src,
                                                            uint32_t* __restrict__ dst) {
  const uint64_t tile = kXcd ? gdn::xcd_contiguous_item(blockIdx.x, gridDim.x) : blockIdx.x;
  const int row0 = threadIdx.x >> 5;
  const int quad = threadIdx.x & 31;
  const uint4* in = src + tile * (kTileDim * kTileDim / 4);
  uint32_t* out = dst + tile * (kTileDim * kTileDim / 4);
  uint4 v[kRowsPerThread];
#pragma unroll
  for (int j = 0; j < kRowsPerThread; ++j) {
    v[j] = load16<kNontemporal>(in + (8 * j + row0) * (kTileDim / 4) + quad);
  }
#pragma unroll
  for (int j = 0; j < kRowsPerThread; ++j) {
    const uint32_t packed = (v[j].x & 0xFFu) | ((v[j].y & 0xFFu) << 8) |
                            ((v[j].z & 0xFFu) << 16) | (v[j].w << 24);
    uint32_t* q = out + (8 * j + row0) * (kTileDim / 4) + quad;
    if (kNontemporal) {
      __builtin_nontemporal_store(packed, q);
    } else {
      *q = packed;
    }
  }
}

template <bool kNontemporal, bool kXcd>
__global__ __launch_bounds__(kThreads) void halve_kernel(const uint2* __restrict__ src,
                                                         uint32_t* __restrict__ dst) {
  const uint64_t tile = kXcd ? gdn::xcd_contiguous_item(blockIdx.x, gridDim.x) : blockIdx.x;
  const int row0 = threadIdx.x >> 5;
  const int quad = threadIdx.x & 31;
  const uint2* in = src + tile * (kTileDim * kTileDim / 4);
  uint32_t* out = dst + tile * (kTileDim * kTileDim / 4);
  uint2 v[kRowsPerThread];
#pragma unroll
  for (int j = 0; j < kRowsPerThread; ++j) {
    const uint2* p = in + (8 * j + row0) * (kTileDim / 4) + quad;
    if constexpr (kNontemporal) {
      v[j] = gdn::stream_load(p);
    } else {
      v[j] = *p;
    }
  }
#pragma unroll
  for (int j = 0; j < kRowsPerThread; ++j) {
    const uint32_t packed = (v[j].x & 0xFFu) | (((v[j].x >> 16) & 0xFFu) << 8) |
                            ((v[j].y & 0xFFu) << 16) | ((v[j].y >> 16) << 24);
    uint32_t* q = out + (8 * j + row0) * (kTileDim / 4) + quad;
    if (kNontemporal) {
      __builtin_nontemporal_store(packed, q);
    } else {
      *q = packed;
    }
  }
}

// VALU issue ceiling: every thread runs `rounds` rounds of 16 independent
// operations (mode 0: fp32 fma, v_fma_f32; mode 1: u32 xor-add, v_xad_u32;
// mode 2: fp64 add, v_add_f64), so each wavefront issues 16 * rounds VALU
// instructions besides a few of loop control, with no memory traffic.
constexpr int kValuChains = 16;

template <int kMode>
__global__ __launch_bounds__(kThreads) void valu_kernel(uint32_t* __restrict__ sink,
                                                        uint32_t rounds, float x, float y) {
  if constexpr (kMode == 0) {
    float a[kValuChains];
#pragma unroll
    for (int i = 0; i < kValuChains; ++i) a[i] = static_cast<float>(threadIdx.x + i);
    for (uint32_t r = 0; r < rounds; ++r) {
#pragma unroll
      for (int i = 0; i < kValuChains; ++i) a[i] = fmaf(a[i], x, y);
    }
    float total = 0.0f;
#pragma unroll
    for (int i = 0; i < kValuChains; ++i) total += a[i];
    sink[blockIdx.x * kThreads + threadIdx.x] = __float_as_uint(total);
  } else if constexpr (kMode == 1) {
    uint32_t a[kValuChains];
    const uint32_t step = __float_as_uint(x);
#pragma unroll
    for (int i = 0; i < kValuChains; ++i) a[i] = threadIdx.x + i;
    for (uint32_t r = 0; r < rounds; ++r) {
#pragma unroll
      for (int i = 0; i < kValuChains; ++i) a[i] = (a[i] ^ step) + static_cast<uint32_t>(i);
    }
    uint32_t total = 0;
#pragma unroll
    for (int i = 0; i < kValuChains; ++i) total ^= a[i];
    sink[blockIdx.x * kThreads + threadIdx.x] = total;
  } else {
    double a[kValuChains];
#pragma unroll
    for (int i = 0; i < kValuChains; ++i) a[i] = static_cast<double>(threadIdx.x + i);
    const double step = static_cast<double>(x);
    for (uint32_t r = 0; r < rounds; ++r) {
#pragma unroll
      for (int i = 0; i < kValuChains; ++i) a[i] = a[i] + step;
    }
    double total = 0.0;
#pragma unroll
    for (int i = 0; i < kValuChains; ++i) total += a[i];
    sink[blockIdx.x * kThreads + threadIdx.x] = static_cast<uint32_t>(total);
  }
}

}  // namespace

// Grid size used by every probe: enough workgroups to fill 256 CUs many
// times over; the sink for the read probe must hold kProbeGrid * 256 words.
extern "C" uint32_t gdn_hbm_probe_grid() { return 256u * 64u; }

// mode bit 0: nontemporal accesses; bit 1: XCD-contiguous order.
extern "C" int32_t gdn_hbm_probe_copy(void* stream, const void* src, void* dst,
                                      uint64_t bytes, uint32_t mode) {
  if (src == nullptr || dst == nullptr || bytes % 128 != 0 || mode > 3) return 1;
  const auto kernel = mode == 0 ? copy_kernel<false, false> : mode == 1 ? copy_kernel<true, false> : mode == 2 ? copy_kernel<false, true> : copy_kernel<true, true>;
  hipLaunchKernelGGL(kernel, dim3(gdn_hbm_probe_grid()), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream),
                     static_cast<const uint4*>(src), static_cast<uint4*>(dst),
                     bytes / 16);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

extern "C" int32_t gdn_hbm_probe_read(void* stream, const void* src, void* sink,
                                      uint64_t bytes, uint32_t mode) {
  if (src == nullptr || sink == nullptr || bytes % 128 != 0 || mode > 3) return 1;
  const auto kernel = mode == 0 ? read_kernel<false, false> : mode == 1 ? read_kernel<true, false> : mode == 2 ? read_kernel<false, true> : read_kernel<true, true>;
  hipLaunchKernelGGL(kernel, dim3(gdn_hbm_probe_grid()), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream),
                     static_cast<const uint4*>(src), static_cast<uint32_t*>(sink),
                     bytes / 16);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

extern "C" int32_t gdn_hbm_probe_write(void* stream, void* dst, uint64_t bytes,
                                       uint32_t mode) {
  if (dst == nullptr || bytes % 128 != 0 || mode > 3) return 1;
  const auto kernel = mode == 0 ? write_kernel<false, false> : mode == 1 ? write_kernel<true, false> : mode == 2 ? write_kernel<false, true> : write_kernel<true, true>;
  hipLaunchKernelGGL(kernel, dim3(gdn_hbm_probe_grid()), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<uint4*>(dst),
                     bytes / 16, 0x3F800000u);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

// 1:4 stream: `tiles` 16 KiB tiles of bytes at src widened into `tiles`
// 64 KiB tiles of fp32 at dst (one workgroup per tile).
extern "C" int32_t gdn_hbm_probe_expand(void* stream, const void* src, void* dst,
                                        uint64_t tiles, uint32_t mode) {
  if (src == nullptr || dst == nullptr || tiles == 0 || tiles > 0x7FFFFFFFull || mode > 3) {
    return 1;
  }
  const auto kernel = mode == 0 ? expand_kernel<false, false> : mode == 1 ? expand_kernel<true, false> : mode == 2 ? expand_kernel<false, true> : expand_kernel<true, true>;
  hipLaunchKernelGGL(kernel, dim3(static_cast<uint32_t>(tiles)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint32_t*>(src),
                     static_cast<float4*>(dst));
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

// 4:1 stream: `tiles` 64 KiB tiles at src narrowed into `tiles` 16 KiB tiles
// at dst (one workgroup per tile).
extern "C" int32_t gdn_hbm_probe_contract(void* stream, const void* src, void* dst,
                                          uint64_t tiles, uint32_t mode) {
  if (src == nullptr || dst == nullptr || tiles == 0 || tiles > 0x7FFFFFFFull || mode > 3) {
    return 1;
  }
  const auto kernel = mode == 0 ? contract_kernel<false, false> : mode == 1 ? contract_kernel<true, false> : mode == 2 ? contract_kernel<false, true> : contract_kernel<true, true>;
  hipLaunchKernelGGL(kernel, dim3(static_cast<uint32_t>(tiles)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint4*>(src),
                     static_cast<uint32_t*>(dst));
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

// 2:1 stream: `tiles` 32 KiB tiles of bf16 at src narrowed into `tiles` 16 KiB
// tiles at dst (one workgroup per tile).
extern "C" int32_t gdn_hbm_probe_halve(void* stream, const void* src, void* dst,
                                       uint64_t tiles, uint32_t mode) {
  if (src == nullptr || dst == nullptr || tiles == 0 || tiles > 0x7FFFFFFFull || mode > 3) {
    return 1;
  }
  const auto kernel = mode == 0 ? halve_kernel<false, false> : mode == 1 ? halve_kernel<true, false> : mode == 2 ? halve_kernel<false, true> : halve_kernel<true, true>;
  hipLaunchKernelGGL(kernel, dim3(static_cast<uint32_t>(tiles)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint2*>(src),
                     static_cast<uint32_t*>(dst));
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

// VALU probe: `blocks` workgroups of 256 threads, each thread 16 * rounds
// operations of the kind `mode` selects; sink holds blocks * 256 words.
extern "C" int32_t gdn_valu_probe(void* stream, void* sink, uint32_t blocks, uint32_t rounds,
                                  uint32_t mode) {
  if (sink == nullptr || blocks == 0 || rounds == 0 || mode > 2) return 1;
  const auto kernel = mode == 0 ? valu_kernel<0> : mode == 1 ? valu_kernel<1> : valu_kernel<2>;
  hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<uint32_t*>(sink), rounds, 1.0000001f, 0.5f);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}
