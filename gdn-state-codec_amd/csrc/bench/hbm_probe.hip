// HBM bandwidth probes used by bench.py (not part of the codec's C-ABI).
//
// Three streaming kernels with the codec's access granularity (16-byte
// vector loads/stores, 256-thread workgroups, one contiguous 4 KiB chunk per
// workgroup iteration): copy, read-only and write-only.  They give the
// bandwidth this GPU actually sustains, and the copy kernel is the known-size
// reference that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;  // 16-byte accesses in flight per thread

__global__ __launch_bounds__(kThreads) void copy_kernel(const uint4* __restrict__ src,
                                                        uint4* __restrict__ dst,
                                                        uint64_t vectors) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads * kUnroll;
  for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * kThreads * kUnroll +
                       threadIdx.x;
       base < vectors; base += stride) {
    uint4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint64_t i = base + static_cast<uint64_t>(u) * kThreads;
      if (i < vectors) v[u] = src[i];
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint64_t i = base + static_cast<uint64_t>(u) * kThreads;
      if (i < vectors) dst[i] = v[u];
    }
  }
}

__global__ __launch_bounds__(kThreads) void read_kernel(const uint4* __restrict__ src,
                                                        uint32_t* __restrict__ sink,
                                                        uint64_t vectors) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads * kUnroll;
  uint32_t acc = 0;
  for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * kThreads * kUnroll +
                       threadIdx.x;
       base < vectors; base += stride) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint64_t i = base + static_cast<uint64_t>(u) * kThreads;
      if (i < vectors) {
        const uint4 v = src[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
      }
    }
  }
  // One word per thread keeps the loads live; the sink holds gridDim*256 words.
  sink[static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x] = acc;
}

__global__ __launch_bounds__(kThreads) void write_kernel(uint4* __restrict__ dst,
                                                         uint64_t vectors,
                                                         uint32_t value) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads * kUnroll;
  const uint4 v = make_uint4(value, value, value, value);
  for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * kThreads * kUnroll +
                       threadIdx.x;
       base < vectors; base += stride) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint64_t i = base + static_cast<uint64_t>(u) * kThreads;
      if (i < vectors) dst[i] = v;
    }
  }
}

}  // namespace

// Grid size used by every probe: enough workgroups to fill 256 CUs many
// times over; the sink for the read probe must hold kProbeGrid * 256 words.
extern "C" uint32_t gdn_hbm_probe_grid() { return 256u * 64u; }

extern "C" int32_t gdn_hbm_probe_copy(void* stream, const void* src, void* dst,
                                      uint64_t bytes) {
  if (src == nullptr || dst == nullptr || bytes % 16 != 0) return 1;
  hipLaunchKernelGGL(copy_kernel, dim3(gdn_hbm_probe_grid()), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream),
                     static_cast<const uint4*>(src), static_cast<uint4*>(dst),
                     bytes / 16);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

extern "C" int32_t gdn_hbm_probe_read(void* stream, const void* src, void* sink,
                                      uint64_t bytes) {
  if (src == nullptr || sink == nullptr || bytes % 16 != 0) return 1;
  hipLaunchKernelGGL(read_kernel, dim3(gdn_hbm_probe_grid()), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream),
                     static_cast<const uint4*>(src), static_cast<uint32_t*>(sink),
                     bytes / 16);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

extern "C" int32_t gdn_hbm_probe_write(void* stream, void* dst, uint64_t bytes) {
  if (dst == nullptr || bytes % 16 != 0) return 1;
  hipLaunchKernelGGL(write_kernel, dim3(gdn_hbm_probe_grid()), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<uint4*>(dst),
                     bytes / 16, 0x3F800000u);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}
