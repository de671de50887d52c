/*
 * C-ABI of the MI355X (gfx950) capsule wire format: hibernate / migrate window
 * slots as LQCAPS01 capsules and restore them, on the device.
 *
 * A capsule is the byte string GdnStateCodecCapsule::Serialize writes
 * (native/src/gdn_state_codec_state_capsule.cpp:446-474): magic "LQCAPS01",
 * schema 1, window 16, rank 4, bits 8, smoothing floor 1e-8f, generation and
 * epoch (uint64), key and value dimensions (128), the window position p, the
 * model-geometry digest (64 lowercase hex characters), the int8 codes in
 * [key][value] order, fp32 smoothing, scales, compensators [key][4] /
 * [value][4], p update records {per-key decay, key, correction} in fp32, and
 * the lowercase hex SHA-256 of everything before it; integers and floats
 * little-endian.  A slot state at position p encodes to
 * 21688 + 1536 p bytes, so the reference's own Restore admits it and its
 * DenseState is the window's state: codes transposed from the slot layout,
 * fp16 compensators and records widened exactly, each record's gate repeated
 * over the keys.
 *
 * Slot buffers are those of gdn_state_codec_window.h (layout 0 = codes
 * [key][value], 1 = [value][key]).  Capsule i lives at capsules + offsets[i]
 * (offsets on the device, multiples of 8) and lengths[i] bytes, inside
 * `capacity` bytes.
 *
 * No counterpart exists on the reference's device side: the reference
 * serializes one CPU capsule at a time (state_capsule.cpp:446-578); these
 * entry points replace that pair for a whole batch of slots.
 *
 * Alignment: every device pointer argument must be 16-byte aligned (see
 * gdn_state_codec_kernel.h); a misaligned pointer returns 1 before any launch.
 */
#ifndef GDN_STATE_CODEC_CAPSULE_H
#define GDN_STATE_CODEC_CAPSULE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Per-capsule restore outcomes, one per check of GdnStateCodecCapsule::Restore
 * (state_capsule.cpp:476-578), made in the reference's order; the first check
 * that fails names the outcome. */
#define GDN_STATE_CODEC_CAPSULE_OK 0u
#define GDN_STATE_CODEC_CAPSULE_TRUNCATED 1u        /* too short / a field runs past the end */
#define GDN_STATE_CODEC_CAPSULE_MAGIC 2u
#define GDN_STATE_CODEC_CAPSULE_DIGEST_ENCODING 3u  /* digest not 64 lowercase hex */
#define GDN_STATE_CODEC_CAPSULE_DIGEST_MISMATCH 4u
#define GDN_STATE_CODEC_CAPSULE_PARAMETERS 5u       /* schema/window/rank/bits/floor */
#define GDN_STATE_CODEC_CAPSULE_IDENTITY 6u         /* geometry/generation/epoch/dims */
#define GDN_STATE_CODEC_CAPSULE_RANK 7u
#define GDN_STATE_CODEC_CAPSULE_POSITION 8u         /* window position >= 16 */
#define GDN_STATE_CODEC_CAPSULE_PHASE 9u            /* position != expected */
#define GDN_STATE_CODEC_CAPSULE_RESIDUAL_DOMAIN 10u /* a code equals -128 */
#define GDN_STATE_CODEC_CAPSULE_BOUNDARY_PAYLOAD 11u
#define GDN_STATE_CODEC_CAPSULE_RECORD_NONFINITE 12u
#define GDN_STATE_CODEC_CAPSULE_TRAILING 13u
#define GDN_STATE_CODEC_CAPSULE_STATE_NONFINITE 14u
/* Device-only outcomes.  DEVICE_FORMAT: a valid capsule the slot cannot hold
 * exactly (per-key decays differ within a record, or a compensator or record
 * value is not an fp16 number).  EXTENT: offsets[i] is not a multiple of 8 or
 * the capsule does not lie inside `capacity`. */
#define GDN_STATE_CODEC_CAPSULE_DEVICE_FORMAT 15u
#define GDN_STATE_CODEC_CAPSULE_EXTENT 16u

/* Bytes of the capsule of a slot state at window position p (0 for p >= 16). */
uint64_t statecentric_gdn_state_codec_capsule_bytes_v1(uint32_t window_position);

/* Serialize `states` slot states (GdnStateCodecCapsule::Serialize,
 * state_capsule.cpp:446-474) under the identity {geometry_sha256 (host
 * pointer to 64 lowercase hex characters), generation, epoch, 128, 128}.
 * lengths[i] receives the capsule's byte count, or 0 when state i is at
 * position >= 16 or its capsule would not fit at offsets[i] (misaligned or
 * past `capacity`).  Slot buffers are only read.
 * Returns 1 for a null pointer, states outside 1..16384, a layout other than
 * 0/1 or an invalid identity (ValidateIdentity, state_capsule.cpp:40-48). */
int32_t statecentric_gdn_state_codec_capsule_serialize_launch_v1(
    void* stream, const int8_t* residual, const float* smoothing, const float* scales,
    const uint16_t* compensator_keys, const uint16_t* compensator_values,
    const float* record_decay, const uint16_t* record_keys,
    const uint16_t* record_corrections, const uint32_t* positions, uint32_t layout,
    const char* geometry_sha256, uint64_t generation, uint64_t epoch, uint8_t* capsules,
    const uint64_t* offsets, uint64_t capacity, uint32_t* lengths, uint32_t states);

/* Restore `states` capsules (GdnStateCodecCapsule::Restore,
 * state_capsule.cpp:476-578) against the expected identity and the expected
 * window position expected_positions[i], into slot state i.  status[i]
 * receives a GDN_STATE_CODEC_CAPSULE_* outcome; state i's slot buffers are
 * written only when it is OK (codes, smoothing, scales, compensators, records
 * 0..p-1 and position word 0; records p..15 and position words 1..7 are left
 * as they were).  Same return codes as serialize. */
int32_t statecentric_gdn_state_codec_capsule_restore_launch_v1(
    void* stream, const uint8_t* capsules, const uint64_t* offsets, const uint32_t* lengths,
    uint64_t capacity, const char* geometry_sha256, uint64_t generation, uint64_t epoch,
    const uint32_t* expected_positions, uint32_t layout, int8_t* residual, float* smoothing,
    float* scales, uint16_t* compensator_keys, uint16_t* compensator_values,
    float* record_decay, uint16_t* record_keys, uint16_t* record_corrections,
    uint32_t* positions, uint32_t* status, uint32_t states);

#ifdef __cplusplus
}
#endif

#endif /* GDN_STATE_CODEC_CAPSULE_H */
