/*
 * C-ABI of the MI355X (gfx950) encoded projection: queries read directly
 * against the int8-encoded GDN state, with dequantization fused in, never
 * materializing the fp32 state.
 *
 * For one head tile (codes, smoothing s[key], value_scales[value]) and a query
 * x[k] = query_scale * q[k] (q bf16), the projection is the reference's
 * boundary readout with no buffered records and no compensators
 * (native/src/gdn_state_codec_state_capsule.cpp:281-290):
 *     out[v] = (sum_k code(v, k) * s[k] * x[k]) / 127 * scale[v].
 * Value head h reads query head h / (value_heads / query_heads), Qwen's GQA
 * pairing of consecutive value heads on one query/key head
 * (kernel/gdn_state_codec_windowed_gdn_step.cpp:340).  Outputs are fp32 and
 * agree with the fp64 evaluation of the same sum to within
 * 2^-15 * (sum_k |code * s * x|) * scale / 127 (decode) and 2^-14 times the
 * same magnitude (chunked, whose weights s * x enter the bf16 matrix cores as
 * two rounded bf16 parts; the bound holds for every finite weight of
 * magnitude at least 2^-110, the top of fp32's range included).
 *
 * Same conventions as gdn_state_codec_kernel.h: asynchronous on `stream`, no
 * allocation, status 0 / 1 (bad argument) / 5 (launch failed).
 *
 * Alignment: every device pointer argument must be 16-byte aligned (see
 * gdn_state_codec_kernel.h); a misaligned pointer returns 1 before any launch.
 */
#ifndef GDN_STATE_CODEC_PROJECTION_H
#define GDN_STATE_CODEC_PROJECTION_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Decode (one token per sequence).  residual [batch][value_heads] tiles in
 * `layout` (GDN_STATE_CODEC_LAYOUT_*), smoothing and value_scales
 * [batch][value_heads][128] fp32, queries [batch][query_heads][128] bf16,
 * outputs [batch][value_heads][128] fp32.  value_heads must be a multiple of
 * query_heads.  This is the readout the reference evaluates inside
 * windowed_gdn_step_bf16_quant_only_launch_v1 and the Cube chain
 * prepare_decode_pair_bf16 -> int8_cube_matmul -> finish_decode_pair_bf16
 * (native/include/statecentric/gdn_state_codec_windowed_gdn_kernel.h:31-40,
 * 108-149; host/gdn_state_codec_decode_runtime.cpp:121-148), without their
 * record-window bookkeeping and without their 16384-state cap. */
int32_t statecentric_gdn_state_codec_encoded_projection_decode_launch_v4(
    void* stream, const int8_t* residual, const float* smoothing,
    const float* value_scales, const uint16_t* queries, float* outputs,
    uint32_t batch, uint32_t value_heads, uint32_t query_heads,
    float query_scale, uint32_t layout);

/* Chunked (T > 1 tokens per sequence, e.g. chunked prefill).  residual
 * [seqs][value_heads] tiles, queries [seqs][tokens][query_heads][128] bf16,
 * outputs [seqs][tokens][value_heads][128] fp32.  The reference has no such
 * entry point (its prefill runs the dense chunk_gated_delta_rule,
 * src/gdn_state_codec/host_gdn.py:305-344); this is the same readout applied
 * to every token.  Returns 1 as well when one sequence's output rows span
 * 2^32 bytes or more (tokens * value_heads * 512 >= 2^32): the kernel
 * addresses them with 32-bit offsets from a per-sequence base. */
int32_t statecentric_gdn_state_codec_encoded_projection_chunked_launch_v4(
    void* stream, const int8_t* residual, const float* smoothing,
    const float* value_scales, const uint16_t* queries, float* outputs,
    uint32_t seqs, uint32_t tokens, uint32_t value_heads, uint32_t query_heads,
    float query_scale, uint32_t layout);

#ifdef __cplusplus
}
#endif

#endif /* GDN_STATE_CODEC_PROJECTION_H */
