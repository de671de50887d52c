// Workgroup residency against LDS size, used by bench.py (not part of the
// codec's C-ABI).
//
// Each workgroup (64 or 128 threads) holds `lds_bytes` of dynamic LDS (it
// writes and reads a word per thread so the allocation is live) and waits until
// `ticks` of the 100 MHz real-time counter have passed since it started.
// Launched with `blocks` = k x (compute units), the kernel takes about one
// wait when k workgroups fit on a CU together and about two when fewer do,
// so a sweep of lds_bytes shows the sizes at which residency steps down:
// the LDS allocation granularity, which decides how many workgroups of a
// kernel with a given LDS footprint share a CU.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kProbeThreads = 128;
constexpr uint32_t kMinLdsBytes = kProbeThreads * 4;
constexpr uint32_t kMaxLdsBytes = 160 * 1024;
constexpr uint32_t kMaxBlocks = 1u << 20;
constexpr uint64_t kMaxTicks = 10000000;  // 0.1 s

__global__ __launch_bounds__(kProbeThreads) void lds_residency_kernel(uint32_t* sink,
                                                                      uint64_t ticks) {
  const uint32_t threads = blockDim.x;
  extern __shared__ uint32_t lds[];
  const uint64_t start = __builtin_amdgcn_s_memrealtime();
  lds[threadIdx.x] = threadIdx.x;
  __syncthreads();
  uint64_t now = start;
  while (now - start < ticks) {
    __builtin_amdgcn_s_sleep(1);
    now = __builtin_amdgcn_s_memrealtime();
  }
  if (threadIdx.x == 0) {
    sink[blockIdx.x] = lds[(threadIdx.x + 1) % threads] + static_cast<uint32_t>(now - start);
  }
}

}  // namespace

// Returns 0, 1 for arguments outside the probe's limits (sink null, blocks 0
// or above 2^20, threads not 64 or 128, lds_bytes outside [512, 160 KiB],
// ticks 0 or above 10^7) and 5 when HIP refuses the launch.  `sink` holds
// `blocks` words.
extern "C" int32_t gdn_lds_residency_probe(void* stream, uint32_t* sink, uint32_t blocks,
                                           uint32_t threads, uint32_t lds_bytes,
                                           uint64_t ticks) {
  if (sink == nullptr || blocks == 0 || blocks > kMaxBlocks ||
      (threads != 64 && threads != kProbeThreads) || lds_bytes < kMinLdsBytes ||
      lds_bytes > kMaxLdsBytes || ticks == 0 || ticks > kMaxTicks) {
    return 1;
  }
  const void* kernel = reinterpret_cast<const void*>(lds_residency_kernel);
  if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                          static_cast<int>(lds_bytes)) != hipSuccess) {
    return 5;
  }
  void* args[] = {&sink, &ticks};
  if (hipLaunchKernel(kernel, dim3(blocks), dim3(threads), args, lds_bytes,
                      static_cast<hipStream_t>(stream)) != hipSuccess) {
    return 5;
  }
  return 0;
}
