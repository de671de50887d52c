/*
 * C-ABI of the MI355X (gfx950) GDN state codec: int8 quantize / dequantize of
 * Qwen3.5 gated-delta-net recurrent-state head tiles (128 x 128 fp32).
 *
 * Every entry point is asynchronous on `stream` (a hipStream_t; NULL is HIP's
 * null stream, torch's default stream) and allocates nothing.  Pointers are
 * device addresses owned by the caller, who keeps them alive until the stream
 * has consumed them.  Return value: 0 on success, 1 for a null pointer or an
 * out-of-range count/enum (the reference's status 1), 5 when HIP rejects the
 * launch.
 *
 * Alignment: every device pointer argument must be 16-byte aligned (the
 * kernels move tiles as 16-byte vectors).  hipMalloc and torch allocations are
 * 256-byte aligned, and so is every per-tile view of them; a view that starts
 * at an arbitrary element offset may not be, and returns 1 before any launch.
 *
 * Numerics: codes, smoothing and scales are bit-identical to the reference's
 * portable C++ QuantizeBoundary quant stage (quant-only initializer) and dense
 * outputs to its DequantizeBoundary:
 *   native/src/gdn_state_codec_state_capsule.cpp:190-226, :229-251.
 *
 * Layouts of one tile: [key][value] is the codec/capsule layout
 * (native/include/statecentric/gdn_state_codec_qwen38_gdn_adapter.h:10-11);
 * [value][key] is the Qwen provider layout used by the vLLM runtime
 * (src/gdn_state_codec/runtime.py:378, 407-408).  smoothing is always indexed
 * by key ([tile][128]) and value_scales by value ([tile][128]).
 */
#ifndef GDN_STATE_CODEC_KERNEL_H
#define GDN_STATE_CODEC_KERNEL_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GDN_STATE_CODEC_LAYOUT_KEY_VALUE 0u
#define GDN_STATE_CODEC_LAYOUT_VALUE_KEY 1u
#define GDN_STATE_CODEC_DTYPE_F32 0u
#define GDN_STATE_CODEC_DTYPE_BF16 1u

/* ---- reference entry points (same names, arguments and admission) -------- */

/* One [key][value] tile: smoothing[key].
 * Replaces native/include/statecentric/gdn_state_codec_kernel.h:5-6
 * (kernel/gdn_state_codec_smoothing.cpp:126-130). */
int32_t statecentric_gdn_state_codec_smoothing_launch_v1(void* stream,
                                                         const float* residual,
                                                         float* smoothing);

/* Provider tiles [states][value][key]: smoothing[states][key]; 1 <= states <= 64.
 * Replaces gdn_state_codec_kernel.h:11-14 (kernel/...smoothing.cpp:140-152). */
int32_t statecentric_gdn_state_codec_provider_smoothing_launch_v2(
    void* stream, const float* provider_state, float* smoothing, uint32_t states);

/* One [key][value] tile with the caller's smoothing: codes [key][value] and
 * value_scales[value].  Replaces gdn_state_codec_kernel.h:16-18
 * (kernel/...quantize.cpp:188-192). */
int32_t statecentric_gdn_state_codec_quantize_launch_v1(void* stream,
                                                        const float* residual,
                                                        const float* smoothing,
                                                        int8_t* quantized,
                                                        float* value_scales);

/* Provider tiles with the caller's smoothing: codes [states][value][key],
 * value_scales[states][value]; 1 <= states <= 64.  Replaces
 * gdn_state_codec_kernel.h:20-23 (kernel/...quantize.cpp:203-217).  Rounding
 * follows the portable C++ path (std::lround), not the Ascend kernel's
 * fp16 RINT, so the codes are the reference CPU path's. */
int32_t statecentric_gdn_state_codec_provider_quantize_launch_v2(
    void* stream, const float* provider_state, const float* smoothing,
    int8_t* quantized, float* value_scales, uint32_t states);

/* Smoothing then quantization of provider tiles, one pass over HBM;
 * 1 <= states <= 64.  Replaces gdn_state_codec_kernel.h:28-31
 * (host/gdn_state_codec_provider_runtime.cpp:3-15). */
int32_t statecentric_gdn_state_codec_provider_initialize_launch_v3(
    void* stream, const float* provider_state, float* smoothing,
    int8_t* quantized, float* value_scales, uint32_t states);

/* One [key][value] tile: dense = ((s*code)/127)*scale + sum_r ck[k][r]*cv[v][r]
 * with fp32 rank-4 compensators ck [key][4], cv [value][4].  Replaces
 * gdn_state_codec_kernel.h:33-36 (kernel/...dequantize.cpp:85-89). */
int32_t statecentric_gdn_state_codec_dequantize_launch_v1(
    void* stream, const int8_t* quantized, const float* smoothing,
    const float* value_scales, const float* compensator_keys,
    const float* compensator_values, float* dense);

/* ---- batched extensions (no reference counterpart; the reference caps a
 * launch at 64 tiles, gdn_state_codec_quantize.cpp:207-211) ------------------ */

/* Quant-only encode of `heads` contiguous tiles in `layout` (e.g. a whole
 * [L,B,H,128,128] state).  1 <= heads <= 2^31-1.  Generalizes
 * provider_initialize_launch_v3 to both layouts and any count. */
int32_t statecentric_gdn_state_codec_encode_launch_v4(
    void* stream, const float* state, int8_t* quantized, float* smoothing,
    float* value_scales, uint64_t heads, uint32_t layout);

/* The public capsule path's boundary encode for `heads` [key][value] fp32
 * tiles: GdnStateCodecCapsule::FromDenseBoundary (state_capsule.cpp:318-335)
 * through QuantizeBoundary (:129-226), i.e. the rank-`rank` compensator fit by
 * power iteration from sinusoidal start vectors (:136-188), then the quant
 * stage of encode_launch_v4 on the fitted residual, bit-identical to the
 * reference's CPU code.  Outputs: residual (the fitted fp32 residual,
 * [heads][128][128], also the quant stage's input), quantized [key][value],
 * smoothing, value_scales, compensator_keys [heads][128][rank] and
 * compensator_values [heads][128][rank] in fp32 (NULL allowed when rank is 0),
 * and status[h]: 0, or 1 when head h holds a non-finite value (the reference
 * rejects it before the fit), or 2 when a singular value is non-finite (the
 * reference's check at :167-169); a head with a non-zero status has
 * unspecified outputs.  0 <= rank <= 4 (the capsule schema fixes 4),
 * 1 <= heads <= 2^31-1.  The reference exposes this only as the C++ capsule
 * factory; this batched entry point has no C-ABI counterpart. */
int32_t statecentric_gdn_state_codec_quantize_boundary_launch_v1(
    void* stream, const float* dense, float* residual, int8_t* quantized,
    float* smoothing, float* value_scales, float* compensator_keys,
    float* compensator_values, int32_t* status, uint64_t heads, uint32_t rank);

/* The runtime's exact-SVD boundary initializer for `heads` fp32 provider tiles
 * ([value][key], the dense [key][value] state transposed), replacing
 * GdnStateCodecRuntime._encode_dense_boundary(dense, "exact_svd")
 * (src/gdn_state_codec/runtime.py:335-389), which calls torch.linalg.svd:
 * the rank-4 truncated SVD of each dense head D = U S V^T by one-sided Jacobi,
 * compensator_keys fp16 [heads][128 key][4] = U[:, r] * S[r] and
 * compensator_values fp16 [heads][128 value][4] = V[:, r], r = 0..3 by
 * decreasing singular value; residual fp32 [heads][value][key] = the provider
 * tile minus the fp32 rank-4 product; then encode_launch_v4 of the residual in
 * the [value][key] layout (quantized [value][key], smoothing by key,
 * value_scales by value).  status[h] is 0; 1 when head h holds a
 * non-finite value (its outputs are then unspecified); or 2 when the Jacobi
 * iteration still rotated a pair in its last allowed sweep (30 here): the
 * outputs are then written from that sweep's rows, an unconverged fit the
 * caller should not take as the SVD.  The signs of each
 * (U, V) column pair are the iteration's own (an SVD fixes only their
 * product); the iteration runs in double, so the fp32 rank-4 product agrees
 * with a float64 SVD to the fp32 rounding of the outputs (about 1e-7 of the
 * largest singular value).  1 <= heads <= 2^31-1.  No C-ABI counterpart in
 * the reference. */
int32_t statecentric_gdn_state_codec_exact_svd_boundary_launch_v1(
    void* stream, const float* provider, float* residual, int8_t* quantized,
    float* smoothing, float* value_scales, uint16_t* compensator_keys,
    uint16_t* compensator_values, int32_t* status, uint64_t heads);

/* exact_svd_boundary_launch_v1 with a caller-chosen limit of
 * 1 <= max_sweeps <= 30 Jacobi sweeps (status 1 for a limit outside it): a
 * head that has not converged within the limit gets status 2.  For callers
 * that trade the fit's accuracy for time.  No counterpart in the reference. */
int32_t statecentric_gdn_state_codec_exact_svd_boundary_sweeps_launch_v1(
    void* stream, const float* provider, float* residual, int8_t* quantized,
    float* smoothing, float* value_scales, uint16_t* compensator_keys,
    uint16_t* compensator_values, int32_t* status, uint64_t heads, uint32_t max_sweeps);

/* Decode of `heads` tiles.  compensator_keys/values are both NULL (quant-only,
 * rank 0) or both fp32 [heads][128][4] (rank 4, the dequantize_launch_v1 form). */
int32_t statecentric_gdn_state_codec_decode_launch_v4(
    void* stream, const int8_t* quantized, const float* smoothing,
    const float* value_scales, const float* compensator_keys,
    const float* compensator_values, float* state, uint64_t heads,
    uint32_t layout);

/* Slot-indexed pool codec.  The pool holds [layers][slots][heads] tiles of
 * pool_dtype (fp32 or bf16); the encoded batch is compact
 * [layers][batch][heads].  Entry b of the batch is pool slot slot_ids[b]
 * (device int32[batch]); entries with a negative slot id are padding and are
 * skipped (their encoded/pool tiles are left untouched), as are ids >= slots.
 * Slot ids must be unique within one decode call.  Mirrors the runtime's
 * cache_index -> provider_state[cache_index] slot map
 * (src/gdn_state_codec/runtime.py:603-625) for a whole batch. */
int32_t statecentric_gdn_state_codec_pool_encode_launch_v4(
    void* stream, const void* pool, uint32_t pool_dtype,
    const int32_t* slot_ids, uint32_t batch, uint32_t layers, uint32_t slots,
    uint32_t heads, uint32_t layout, int8_t* quantized, float* smoothing,
    float* value_scales);

/* Decode of a compact encoded batch, scattered into the pool slots (bf16 pools
 * receive round-to-nearest-even of the fp32 dequantized value). */
int32_t statecentric_gdn_state_codec_pool_decode_launch_v4(
    void* stream, const int8_t* quantized, const float* smoothing,
    const float* value_scales, const int32_t* slot_ids, uint32_t batch,
    uint32_t layers, uint32_t slots, uint32_t heads, uint32_t layout,
    void* pool, uint32_t pool_dtype);

#ifdef __cplusplus
}
#endif

#endif /* GDN_STATE_CODEC_KERNEL_H */
