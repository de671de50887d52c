// Kernel-launch plumbing shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <tuple>

#include "work_order.h"

namespace gdn {

// Status codes of every extern "C" entry point.  0 and 1 are the reference's
// (gdn_state_codec_quantize.cpp:207-211: 1 = null pointer or out-of-range
// count); 5 reports a HIP launch failure, which the reference's AscendC
// launches cannot observe.
constexpr int32_t kStatusOk = 0;
constexpr int32_t kStatusInvalidArgument = 1;
constexpr int32_t kStatusLaunchFailed = 5;

// Tile geometry: one Qwen3.5 GDN head is a 128 x 128 fp32 matrix.
constexpr int kDim = 128;
constexpr int kTile = kDim * kDim;

// Tile layouts.  kKeyValue is the codec/capsule layout [key][value]
// (gdn_state_codec_qwen38_gdn_adapter.h:10-11); kValueKey is the Qwen provider
// layout [value][key] (runtime.py:378, 407-408).
constexpr uint32_t kKeyValue = 0;
constexpr uint32_t kValueKey = 1;

// Pool element types.
constexpr uint32_t kDtypeF32 = 0;
constexpr uint32_t kDtypeBF16 = 1;

// Largest grid the launchers issue along x (hardware limit 2^31 - 1).
constexpr uint64_t kMaxGrid = 0x7FFFFFFFull;

// A CU has 163,840 bytes of LDS, and gfx950 allocates a workgroup's LDS in
// 1,280-byte granules (measured: csrc/bench/lds_probe.hip), so k workgroups
// share a CU only while k x ceil(bytes / 1280) x 1280 <= 163,840.  One byte
// past a multiple of 1,280 costs a whole granule.
constexpr uint32_t kLdsPerCu = 163840;
constexpr uint32_t kLdsGranule = 1280;
constexpr uint32_t workgroups_by_lds(uint64_t bytes) {
  return kLdsPerCu / static_cast<uint32_t>((bytes + kLdsGranule - 1) / kLdsGranule * kLdsGranule);
}

// Every device pointer an entry point takes must be 16-byte aligned.  The
// kernels move codes and fp32 tiles as 16-byte vectors and narrower words at
// offsets that are multiples of their own width, so a 16-byte aligned base
// keeps every access aligned.  Allocations (hipMalloc, torch) are 256-byte
// aligned; a view that starts at an arbitrary element offset may not be, and
// the entry points reject it with status 1 before any launch.  Null pointers
// pass this test (they are rejected separately where they are not allowed).
template <typename... Pointers>
inline bool aligned16(const Pointers*... pointers) {
  return ((reinterpret_cast<uintptr_t>(pointers) % 16u == 0u) && ...);
}

// Launches `kernel` on `stream` through hipLaunchKernel so the launch status
// comes back to the caller instead of staying in the thread's last-error slot.
// Arguments are converted to the kernel's parameter types first.
template <typename... KernelArgs, typename... Args>
int32_t launch(void (*kernel)(KernelArgs...), dim3 grid, dim3 block,
               void* stream, Args... args) {
  static_assert(sizeof...(KernelArgs) == sizeof...(Args), "argument count");
  std::tuple<KernelArgs...> values(static_cast<KernelArgs>(args)...);
  void* pointers[sizeof...(KernelArgs)];
  std::apply(
      [&pointers](auto&... value) {
        int index = 0;
        ((pointers[index++] = static_cast<void*>(&value)), ...);
      },
      values);
  const hipError_t status =
      hipLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block,
                      pointers, 0, static_cast<hipStream_t>(stream));
  return status == hipSuccess ? kStatusOk : kStatusLaunchFailed;
}

}  // namespace gdn
