// Test infrastructure only: a C-ABI harness around the reference's portable C++
// CPU path, compiled from the reference sources where they lie (never copied).
// It is built by oracle/Makefile into oracle/_ref/ and used only by
// tests/golden/make_golden.py, the oracle-vs-reference tests and bench.py's
// cpu_baseline leg.  The product path never loads it.
//
// The quant-only stage of the codec is the anonymous-namespace function
// QuantizeBoundary (native/src/gdn_state_codec_state_capsule.cpp:129-227); it is
// reachable only from inside that translation unit, so this harness includes
// the .cpp (by include path, -I $(REF)/native/src) instead of linking it.
#include "gdn_state_codec_state_capsule.cpp"

#include <cstdint>
#include <cstring>
#include <algorithm>
#include <exception>
#include <string>
#include <string_view>
#include <vector>

#include "statecentric/gdn_state_codec_qwen38_gdn_adapter.h"

namespace {

statecentric::GdnStateCodecIdentity MakeIdentity(std::uint32_t keys,
                                                 std::uint32_t values) {
  return {std::string(64, 'a'), 1, 1, keys, values};
}

statecentric::GdnStateCodecParameters MakeParameters(std::uint32_t rank) {
  statecentric::GdnStateCodecParameters parameters;
  parameters.compensator_rank = rank;
  return parameters;
}

// Copies encoded capsule bytes out; 1 when `capacity` is too small.
int CopyBytes(const std::vector<std::uint8_t>& bytes, std::uint8_t* out,
              std::uint64_t capacity, std::uint64_t* size) {
  *size = bytes.size();
  if (bytes.size() > capacity) return 1;
  std::memcpy(out, bytes.data(), bytes.size());
  return 0;
}

// The exception text, NUL-terminated and cut to `capacity` bytes.
void CopyMessage(const char* text, char* message, std::uint64_t capacity) {
  if (message == nullptr || capacity == 0) return;
  const std::size_t length = std::min<std::size_t>(std::strlen(text), capacity - 1);
  std::memcpy(message, text, length);
  message[length] = '\0';
}

}  // namespace

extern "C" {

// QuantizeBoundary with compensator_rank = rank (0 = the quant-only
// initializer: the residual is the dense state itself).  Layout [K][V].
int gdnref_quantize_boundary(const float* dense, std::uint32_t keys,
                             std::uint32_t values, std::uint32_t rank,
                             std::int8_t* residual, float* smoothing,
                             float* value_scales, float* compensator_keys,
                             float* compensator_values) {
  try {
    const auto identity = MakeIdentity(keys, values);
    const auto parameters = MakeParameters(rank);
    const auto boundary = statecentric::QuantizeBoundary(
        std::span<const float>(dense, std::size_t{keys} * values), identity,
        parameters);
    std::memcpy(residual, boundary->residual.data(), boundary->residual.size());
    std::memcpy(smoothing, boundary->smoothing.data(), keys * sizeof(float));
    std::memcpy(value_scales, boundary->value_scales.data(),
                values * sizeof(float));
    if (rank > 0) {
      std::memcpy(compensator_keys, boundary->compensator_keys.data(),
                  std::size_t{keys} * rank * sizeof(float));
      std::memcpy(compensator_values, boundary->compensator_values.data(),
                  std::size_t{values} * rank * sizeof(float));
    }
    return 0;
  } catch (const std::exception&) {
    return 1;
  }
}

// DequantizeBoundary (state_capsule.cpp:229-251).  Compensators may be null
// when rank == 0.
int gdnref_dequantize_boundary(const std::int8_t* residual,
                               const float* smoothing,
                               const float* value_scales,
                               const float* compensator_keys,
                               const float* compensator_values,
                               std::uint32_t keys, std::uint32_t values,
                               std::uint32_t rank, float* dense) {
  try {
    const auto identity = MakeIdentity(keys, values);
    const auto parameters = MakeParameters(rank);
    statecentric::GdnStateCodecCapsule::Boundary boundary;
    boundary.residual.assign(residual, residual + std::size_t{keys} * values);
    boundary.smoothing.assign(smoothing, smoothing + keys);
    boundary.value_scales.assign(value_scales, value_scales + values);
    if (rank > 0) {
      boundary.compensator_keys.assign(
          compensator_keys, compensator_keys + std::size_t{keys} * rank);
      boundary.compensator_values.assign(
          compensator_values, compensator_values + std::size_t{values} * rank);
    }
    const auto out = statecentric::DequantizeBoundary(boundary, identity,
                                                      parameters);
    std::memcpy(dense, out.data(), out.size() * sizeof(float));
    return 0;
  } catch (const std::exception&) {
    return 1;
  }
}

// ReadWindowState with an empty record window (state_capsule.cpp:253-306):
// the boundary readout S^T x of the encoded state.
int gdnref_read_boundary(const std::int8_t* residual, const float* smoothing,
                         const float* value_scales,
                         const float* compensator_keys,
                         const float* compensator_values, std::uint32_t keys,
                         std::uint32_t values, std::uint32_t rank,
                         const float* read, float* output) {
  try {
    const auto identity = MakeIdentity(keys, values);
    const auto parameters = MakeParameters(rank);
    statecentric::GdnStateCodecCapsule::Boundary boundary;
    boundary.residual.assign(residual, residual + std::size_t{keys} * values);
    boundary.smoothing.assign(smoothing, smoothing + keys);
    boundary.value_scales.assign(value_scales, value_scales + values);
    if (rank > 0) {
      boundary.compensator_keys.assign(
          compensator_keys, compensator_keys + std::size_t{keys} * rank);
      boundary.compensator_values.assign(
          compensator_values, compensator_values + std::size_t{values} * rank);
    }
    const std::vector<statecentric::GdnStateCodecCapsule::UpdateRecord> none;
    const auto out = statecentric::ReadWindowState(
        boundary, none, std::span<const float>(read, keys), identity,
        parameters);
    std::memcpy(output, out.data(), out.size() * sizeof(float));
    return 0;
  } catch (const std::exception&) {
    return 1;
  }
}

// Qwen provider [value][key] -> codec [key][value]
// (gdn_state_codec_qwen38_gdn_adapter.cpp:21-38) and back (:40-57).
int gdnref_provider_to_codec(const float* provider, std::uint32_t keys,
                             std::uint32_t values, float* codec) {
  try {
    const auto out = statecentric::Qwen38ProviderStateToGdnStateCodec(
        std::span<const float>(provider, std::size_t{keys} * values), keys,
        values);
    std::memcpy(codec, out.data(), out.size() * sizeof(float));
    return 0;
  } catch (const std::exception&) {
    return 1;
  }
}

int gdnref_codec_to_provider(const float* codec, std::uint32_t keys,
                             std::uint32_t values, float* provider) {
  try {
    const auto out = statecentric::GdnStateCodecStateToQwen38Provider(
        std::span<const float>(codec, std::size_t{keys} * values), keys,
        values);
    std::memcpy(provider, out.data(), out.size() * sizeof(float));
    return 0;
  } catch (const std::exception&) {
    return 1;
  }
}

// ReadWindowState with `records` buffered updates (state_capsule.cpp:253-306):
// record u has per-key decay [keys], key [keys] and correction [values].
int gdnref_read_window(const std::int8_t* residual, const float* smoothing,
                       const float* value_scales, const float* compensator_keys,
                       const float* compensator_values, std::uint32_t keys,
                       std::uint32_t values, std::uint32_t rank,
                       const float* record_decay, const float* record_keys,
                       const float* record_corrections, std::uint32_t records,
                       const float* read, float* output) {
  try {
    const auto identity = MakeIdentity(keys, values);
    const auto parameters = MakeParameters(rank);
    statecentric::GdnStateCodecCapsule::Boundary boundary;
    boundary.residual.assign(residual, residual + std::size_t{keys} * values);
    boundary.smoothing.assign(smoothing, smoothing + keys);
    boundary.value_scales.assign(value_scales, value_scales + values);
    if (rank > 0) {
      boundary.compensator_keys.assign(
          compensator_keys, compensator_keys + std::size_t{keys} * rank);
      boundary.compensator_values.assign(
          compensator_values, compensator_values + std::size_t{values} * rank);
    }
    std::vector<statecentric::GdnStateCodecCapsule::UpdateRecord> updates(records);
    for (std::uint32_t u = 0; u < records; ++u) {
      updates[u].decay.assign(record_decay + std::size_t{u} * keys,
                              record_decay + std::size_t{u + 1} * keys);
      updates[u].key.assign(record_keys + std::size_t{u} * keys,
                            record_keys + std::size_t{u + 1} * keys);
      updates[u].correction.assign(record_corrections + std::size_t{u} * values,
                                   record_corrections + std::size_t{u + 1} * values);
    }
    const auto out = statecentric::ReadWindowState(
        boundary, updates, std::span<const float>(read, keys), identity,
        parameters);
    std::memcpy(output, out.data(), out.size() * sizeof(float));
    return 0;
  } catch (const std::exception&) {
    return 1;
  }
}

// The reference capsule stepped through `tokens` tokens: FromDenseBoundary at
// compensator_rank = rank (window 16; the public capsule admits rank 4
// only, state_capsule.cpp:26-38), then ApplyToken per token
// (state_capsule.cpp:318-335, 354-397).  Token inputs are [tokens][keys]
// (decay, key, read, query) and [tokens][values] (value); outputs
// [tokens][values], crossed[t] = 1 when token t refit the boundary, and
// final_dense = DenseState() after the last token.
int gdnref_apply_tokens(const float* dense, std::uint32_t keys,
                        std::uint32_t values, std::uint32_t rank,
                        std::uint32_t tokens, const float* decay,
                        const float* key, const float* value, const float* read,
                        const float* query, float* outputs,
                        std::uint8_t* crossed, float* final_dense) {
  try {
    auto capsule = statecentric::GdnStateCodecCapsule::FromDenseBoundary(
        std::span<const float>(dense, std::size_t{keys} * values),
        MakeIdentity(keys, values), MakeParameters(rank));
    for (std::uint32_t t = 0; t < tokens; ++t) {
      statecentric::GdnStateCodecTokenInput input;
      input.decay.assign(decay + std::size_t{t} * keys, decay + std::size_t{t + 1} * keys);
      input.key.assign(key + std::size_t{t} * keys, key + std::size_t{t + 1} * keys);
      input.read.assign(read + std::size_t{t} * keys, read + std::size_t{t + 1} * keys);
      input.query.assign(query + std::size_t{t} * keys, query + std::size_t{t + 1} * keys);
      input.value.assign(value + std::size_t{t} * values,
                         value + std::size_t{t + 1} * values);
      const auto result = capsule.ApplyToken(input);
      std::memcpy(outputs + std::size_t{t} * values, result.output.data(),
                  values * sizeof(float));
      crossed[t] = result.crossed_window_boundary ? 1 : 0;
    }
    const auto state = capsule.DenseState();
    std::memcpy(final_dense, state.data(), state.size() * sizeof(float));
    return 0;
  } catch (const std::exception&) {
    return 1;
  }
}

// Batched quant-only encode over `heads` contiguous [K][V] tiles, used as the
// reference CPU baseline (single thread, the reference's own code).
int gdnref_quantize_heads(const float* dense, std::uint64_t heads,
                          std::uint32_t keys, std::uint32_t values,
                          std::int8_t* residual, float* smoothing,
                          float* value_scales) {
  const std::size_t tile = std::size_t{keys} * values;
  for (std::uint64_t head = 0; head < heads; ++head) {
    const int status = gdnref_quantize_boundary(
        dense + head * tile, keys, values, 0, residual + head * tile,
        smoothing + head * keys, value_scales + head * values, nullptr,
        nullptr);
    if (status != 0) return status;
  }
  return 0;
}

int gdnref_dequantize_heads(const std::int8_t* residual,
                            const float* smoothing, const float* value_scales,
                            std::uint64_t heads, std::uint32_t keys,
                            std::uint32_t values, float* dense) {
  const std::size_t tile = std::size_t{keys} * values;
  for (std::uint64_t head = 0; head < heads; ++head) {
    const int status = gdnref_dequantize_boundary(
        residual + head * tile, smoothing + head * keys,
        value_scales + head * values, nullptr, nullptr, keys, values, 0,
        dense + head * tile);
    if (status != 0) return status;
  }
  return 0;
}

// The boundary readout (ReadWindowState with an empty window,
// state_capsule.cpp:253-306) of `heads` contiguous [K][V] boundaries, each
// read with `tokens` vectors: reads [heads][tokens][K], outputs
// [heads][tokens][V].  Each head's Boundary is built once and read `tokens`
// times, as a capsule is between window boundaries.  bench.py's CPU baseline of
// the encoded projection (decode: tokens = 1; chunked: tokens = T).
int gdnref_read_boundary_heads(const std::int8_t* residual, const float* smoothing,
                               const float* value_scales, std::uint64_t heads,
                               std::uint32_t tokens, std::uint32_t keys,
                               std::uint32_t values, const float* reads,
                               float* outputs) {
  try {
    const auto identity = MakeIdentity(keys, values);
    const auto parameters = MakeParameters(0);
    const std::vector<statecentric::GdnStateCodecCapsule::UpdateRecord> none;
    const std::size_t tile = std::size_t{keys} * values;
    for (std::uint64_t head = 0; head < heads; ++head) {
      statecentric::GdnStateCodecCapsule::Boundary boundary;
      boundary.residual.assign(residual + head * tile, residual + (head + 1) * tile);
      boundary.smoothing.assign(smoothing + head * keys, smoothing + (head + 1) * keys);
      boundary.value_scales.assign(value_scales + head * values,
                                   value_scales + (head + 1) * values);
      for (std::uint32_t t = 0; t < tokens; ++t) {
        const std::size_t row = head * tokens + t;
        const auto out = statecentric::ReadWindowState(
            boundary, none, std::span<const float>(reads + row * keys, keys), identity,
            parameters);
        std::memcpy(outputs + row * values, out.data(), values * sizeof(float));
      }
    }
    return 0;
  } catch (const std::exception&) {
    return 1;
  }
}

// Sha256Hex (native/src/sha256.cpp): 64 lowercase hex characters of the
// SHA-256 of `size` bytes.
int gdnref_sha256_hex(const std::uint8_t* data, std::uint64_t size, char* hex) {
  const std::string text = statecentric::Sha256Hex(
      std::string_view(reinterpret_cast<const char*>(data), size));
  std::memcpy(hex, text.data(), text.size());
  return 0;
}

// A capsule the reference builds itself: FromDenseBoundary (rank 4) of a
// [keys][values] state with identity (geometry, generation, epoch), ApplyToken
// per token (inputs as in gdnref_apply_tokens), then Serialize
// (state_capsule.cpp:446-474).  0 on success, 1 with `message` on an exception
// or when `capacity` is too small.
int gdnref_capsule_after_tokens(const float* dense, std::uint32_t keys,
                                std::uint32_t values, std::uint32_t tokens,
                                const float* decay, const float* key,
                                const float* value, const float* read,
                                const float* query, const char* geometry,
                                std::uint64_t generation, std::uint64_t epoch,
                                std::uint8_t* out, std::uint64_t capacity,
                                std::uint64_t* size, char* message,
                                std::uint64_t message_capacity) {
  try {
    statecentric::GdnStateCodecIdentity identity{std::string(geometry, 64),
                                                 generation, epoch, keys, values};
    auto capsule = statecentric::GdnStateCodecCapsule::FromDenseBoundary(
        std::span<const float>(dense, std::size_t{keys} * values), identity,
        MakeParameters(4));
    for (std::uint32_t t = 0; t < tokens; ++t) {
      statecentric::GdnStateCodecTokenInput input;
      input.decay.assign(decay + std::size_t{t} * keys, decay + std::size_t{t + 1} * keys);
      input.key.assign(key + std::size_t{t} * keys, key + std::size_t{t + 1} * keys);
      input.read.assign(read + std::size_t{t} * keys, read + std::size_t{t + 1} * keys);
      input.query.assign(query + std::size_t{t} * keys, query + std::size_t{t + 1} * keys);
      input.value.assign(value + std::size_t{t} * values,
                         value + std::size_t{t + 1} * values);
      (void)capsule.ApplyToken(input);
    }
    if (CopyBytes(capsule.Serialize(), out, capacity, size) != 0) {
      CopyMessage("output capacity too small", message, message_capacity);
      return 1;
    }
    return 0;
  } catch (const std::exception& error) {
    CopyMessage(error.what(), message, message_capacity);
    return 1;
  }
}

// Restore (state_capsule.cpp:476-578) against the expected identity,
// parameters and window position; on success the restored capsule's
// Serialize() goes to `out` and its DenseState() ([keys][values]) to `dense`.
// 0 on success, 1 with the exception's message on rejection.
int gdnref_capsule_restore(const std::uint8_t* encoded, std::uint64_t size,
                           const char* geometry, std::uint64_t generation,
                           std::uint64_t epoch, std::uint32_t keys,
                           std::uint32_t values, std::uint32_t schema,
                           std::uint32_t window, std::uint32_t rank,
                           std::uint32_t bits, float smoothing_floor,
                           std::uint32_t expected_position, std::uint8_t* out,
                           std::uint64_t capacity, std::uint64_t* out_size,
                           float* dense, char* message,
                           std::uint64_t message_capacity) {
  try {
    const statecentric::GdnStateCodecIdentity identity{
        std::string(geometry, 64), generation, epoch, keys, values};
    statecentric::GdnStateCodecParameters parameters{schema, window, rank, bits,
                                                     smoothing_floor};
    const auto restored = statecentric::GdnStateCodecCapsule::Restore(
        std::span<const std::uint8_t>(encoded, size), identity, parameters,
        expected_position);
    if (CopyBytes(restored.Serialize(), out, capacity, out_size) != 0) {
      CopyMessage("output capacity too small", message, message_capacity);
      return 1;
    }
    const auto state = restored.DenseState();
    std::memcpy(dense, state.data(), state.size() * sizeof(float));
    return 0;
  } catch (const std::exception& error) {
    CopyMessage(error.what(), message, message_capacity);
    return 1;
  }
}

}  // extern "C"
