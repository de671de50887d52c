// Internal entry shared by the decode runtime (decode_runtime.cpp) and the
// decode-pair kernels (decode_pair.hip).
#pragma once

#include <stdint.h>

namespace gdn {

// prepare_decode_pair_bf16 + int8 projection + finish_decode_pair_bf16 as one
// kernel; arguments as statecentric_gdn_state_codec_decode_runtime_step_v1,
// already admitted by the caller.
int32_t launch_fused_decode_pair_bf16(
    void* stream, const int8_t* residual, const float* smoothing, const float* scales,
    const uint16_t* comp_keys, const uint16_t* comp_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    const float* decay, const uint16_t* beta, const uint16_t* keys,
    const uint16_t* queries, const uint16_t* values, uint16_t* outputs, uint32_t states);

}  // namespace gdn
