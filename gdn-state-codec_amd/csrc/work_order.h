// Workgroup -> work item order of the streaming kernels, written so the same
// code compiles for the host (tests/codec_math_check.cpp checks that it is a
// bijection for every grid size it sweeps).
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define GDN_ORDER_HD __host__ __device__ __forceinline__
#else
#define GDN_ORDER_HD inline
#endif

namespace gdn {

// Work item of workgroup `block` of `blocks`.  The dispatcher hands workgroup b
// to XCD b % 8, so the identity order has the 8 XCDs working on neighbouring
// tiles at every moment.  This order gives XCD x the contiguous items
// x * q .. x * q + q - 1 (q = blocks / 8, in order), and the last blocks % 8
// items to the workgroups past 8 q.  Measured on the config-2 dequantize
// (bit-identical output): 3.26 ms against 3.70 ms in identity order on one box,
// 3.64-3.66 against 3.69-3.71 ms on four others; the gain depends on the box.
GDN_ORDER_HD uint64_t xcd_contiguous_item(uint64_t block, uint64_t blocks) {
  const uint64_t per_xcd = blocks >> 3;
  if (block >= per_xcd << 3) return block;
  return (block & 7u) * per_xcd + (block >> 3);
}

}  // namespace gdn
