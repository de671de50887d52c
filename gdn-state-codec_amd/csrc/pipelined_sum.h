// Compile-time loop expansion and a software-pipelined form for the dependent
// chains of the fit kernels (sequential sums whose operands come from LDS).
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

namespace gdn {

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

// A dependent chain over kGroups groups of operands read from LDS: load(g,
// regs) fills a group's registers, use(g, regs) consumes them in order.  Group
// g + 1 is loaded before group g is used, so its latency overlaps the chain,
// and a scheduling barrier after each group keeps the compiler from loading
// further ahead (only two groups of operands are live at a time).
template <int kGroups, typename Regs, typename Load, typename Use>
__device__ __forceinline__ void pipelined(Load&& load, Use&& use) {
  Regs buffer[2];
  load(std::integral_constant<int, 0>{}, buffer[0]);
  unrolled<kGroups>([&](auto g) {
    constexpr int group = decltype(g)::value;
    if constexpr (group + 1 < kGroups) {
      load(std::integral_constant<int, group + 1>{}, buffer[(group + 1) & 1]);
    }
    use(g, buffer[group & 1]);
    __builtin_amdgcn_sched_barrier(0);
  });
}

}  // namespace gdn
