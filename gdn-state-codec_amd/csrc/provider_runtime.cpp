// Host-side fusion of the provider initializer
// (reference: host/gdn_state_codec_provider_runtime.cpp:3-15, which runs the
// smoothing launch and then the quantize launch on the caller's stream).
// Here both stages are one kernel that reads each tile from HBM once; the
// admission checks are the reference's v2 checks, so a call the reference
// rejects is rejected with the same status.
#include <stdint.h>

#include "gdn_state_codec_kernel.h"

extern "C" int32_t statecentric_gdn_state_codec_provider_initialize_launch_v3(
    void* stream, const float* provider_state, float* smoothing,
    int8_t* quantized, float* value_scales, uint32_t states) {
  if (provider_state == nullptr || smoothing == nullptr ||
      quantized == nullptr || value_scales == nullptr || states == 0 ||
      states > 64) {
    return 1;
  }
  return statecentric_gdn_state_codec_encode_launch_v4(
      stream, provider_state, quantized, smoothing, value_scales, states,
      GDN_STATE_CODEC_LAYOUT_VALUE_KEY);
}
