// Decode runtime handles (host/gdn_state_codec_decode_runtime.cpp:72-148).
//
// The reference keeps one process-wide runtime for a fixed state count: it owns
// the Cube GEMM's scratch (quantized vectors, int32 projections, dynamic scales,
// tiling) and its step runs prepare -> int8 GEMM -> finish.  Here the step is a
// single fused kernel whose intermediates live in LDS, so the handle owns no
// device memory; it keeps the reference's lifecycle (singleton per process,
// reference-counted, bound to one state count, foreign handles rejected)
// because callers rely on it.
#include <stdint.h>

#include <mutex>

#include "decode_pair.h"
#include "gdn_state_codec_window.h"
#include "launch.h"
#include "window_common.h"

namespace {

struct DecodeRuntime {
  uint32_t states = 0;
  uint32_t references = 0;
};

std::mutex runtime_mutex;
DecodeRuntime* shared_runtime = nullptr;

}  // namespace

extern "C" void* statecentric_gdn_state_codec_decode_runtime_create_v1(uint32_t states) {
  if (states == 0 || states > gdn::kMaxWindowStates) return nullptr;
  std::lock_guard<std::mutex> lock(runtime_mutex);
  if (shared_runtime != nullptr) {
    if (shared_runtime->states != states) return nullptr;
    ++shared_runtime->references;
    return shared_runtime;
  }
  shared_runtime = new DecodeRuntime{states, 1};
  return shared_runtime;
}

extern "C" void statecentric_gdn_state_codec_decode_runtime_destroy_v1(void* opaque) {
  std::lock_guard<std::mutex> lock(runtime_mutex);
  auto* runtime = static_cast<DecodeRuntime*>(opaque);
  if (runtime == nullptr || runtime != shared_runtime) return;
  if (--runtime->references != 0) return;
  shared_runtime = nullptr;
  delete runtime;
}

extern "C" int32_t statecentric_gdn_state_codec_decode_runtime_step_v1(
    void* opaque, void* stream, const int8_t* residual, const float* smoothing,
    const float* scales, const uint16_t* compensator_keys,
    const uint16_t* compensator_values, float* record_decay, uint16_t* record_keys,
    uint16_t* record_corrections, uint32_t* positions, const float* decay,
    const uint16_t* beta, const uint16_t* keys, const uint16_t* queries,
    const uint16_t* values, uint16_t* outputs, uint32_t states) {
  {
    std::lock_guard<std::mutex> lock(runtime_mutex);
    auto* runtime = static_cast<DecodeRuntime*>(opaque);
    if (runtime == nullptr || runtime != shared_runtime || states != runtime->states ||
        !gdn::aligned16(residual, smoothing, scales, compensator_keys, compensator_values,
                        record_decay, record_keys, record_corrections, positions, decay, beta,
                        keys, queries, values, outputs)) {
      return 1;
    }
  }
  // The reference reports the failing stage: 2 = prepare, 3 = projection,
  // 4 = finish (decode_runtime.cpp:132-147).  The fused kernel checks the
  // prepare stage's arguments, then the finish stage's.
  if (!keys || !queries || !decay || !smoothing || states % 2 != 0) return 2;
  if (!residual) return 3;
  if (!scales || !compensator_keys || !compensator_values || !record_decay ||
      !record_keys || !record_corrections || !positions || !beta || !values || !outputs) {
    return 4;
  }
  const int32_t status = gdn::launch_fused_decode_pair_bf16(
      stream, residual, smoothing, scales, compensator_keys, compensator_values,
      record_decay, record_keys, record_corrections, positions, decay, beta, keys,
      queries, values, outputs, states);
  return status == gdn::kStatusOk ? 0 : 4;
}
