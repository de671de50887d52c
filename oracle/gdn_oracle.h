/*
 * CPU oracle for the GDN state codec hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference's
 * portable C++ CPU path (native/src/gdn_state_codec_state_capsule.cpp and
 * native/src/gdn_state_codec_qwen38_gdn_adapter.cpp).  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it, and only as
 * the checker; the product library never links or calls it.
 *
 * Parity pins (each checked by a test under tests/):
 *   quantize (quant-only and rank-r)  : bit-exact vs oracle/_ref (the reference's
 *                                       own QuantizeBoundary) on random, adversarial
 *                                       and special heads; golden fixtures in
 *                                       tests/golden; invariants (max|code|==127 per
 *                                       live column, zero column -> scale 0, zero row
 *                                       -> s=sqrtf(1e-8f), codes never -128);
 *                                       brute force against exact rational rounding.
 *   dequantize                        : bit-exact vs oracle/_ref; closed form.
 *   boundary readout (projection)     : bit-exact vs oracle/_ref ReadWindowState;
 *                                       fp64 brute force within the gamma_n bound.
 *   layout transposes                 : the reference adapter test's 3x2 known answer
 *                                       and round trips.
 *   chunked projection                : no reference function exists; pinned by the
 *                                       closed form o[t] = readout(q[t]) per token,
 *                                       i.e. by the pinned boundary readout.
 *   pool gather/scatter               : by construction from the per-head functions
 *                                       plus index bookkeeping tests.
 */
#ifndef GDN_ORACLE_H
#define GDN_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Layout of one head tile: 0 = codec/capsule [key][value] (the reference's CPU
 * layout), 1 = Qwen provider [value][key] (runtime.py:378, 407-408). */
#define GDN_ORACLE_LAYOUT_KEY_VALUE 0u
#define GDN_ORACLE_LAYOUT_VALUE_KEY 1u

#define GDN_ORACLE_DTYPE_F32 0u
#define GDN_ORACLE_DTYPE_BF16 1u

/* ---- single head, general geometry, [key][value] layout ---------------- */

/* QuantizeBoundary (state_capsule.cpp:129-227).  rank = 0 is the quant-only
 * initializer (the residual is the dense state); rank > 0 runs the sinusoidal
 * power-iteration fit first.  comp_keys [keys][rank] and comp_values
 * [values][rank] may be NULL when rank == 0.  work needs keys*values floats. */
void gdn_oracle_quantize_kv(const float* dense, uint32_t keys, uint32_t values,
                            uint32_t rank, float smoothing_floor,
                            int8_t* codes, float* smoothing, float* value_scales,
                            float* comp_keys, float* comp_values, float* work);

/* DequantizeBoundary (state_capsule.cpp:229-251). */
void gdn_oracle_dequantize_kv(const int8_t* codes, const float* smoothing,
                              const float* value_scales, const float* comp_keys,
                              const float* comp_values, uint32_t keys,
                              uint32_t values, uint32_t rank, float* dense);

/* ReadWindowState with no buffered records (state_capsule.cpp:253-306). */
void gdn_oracle_read_boundary(const int8_t* codes, const float* smoothing,
                              const float* value_scales, const float* comp_keys,
                              const float* comp_values, uint32_t keys,
                              uint32_t values, uint32_t rank, const float* read,
                              float* output);

/* Qwen38ProviderStateToGdnStateCodec / GdnStateCodecStateToQwen38Provider
 * (gdn_state_codec_qwen38_gdn_adapter.cpp:21-57). */
void gdn_oracle_provider_to_codec(const float* provider, uint32_t keys,
                                  uint32_t values, float* codec);
void gdn_oracle_codec_to_provider(const float* codec, uint32_t keys,
                                  uint32_t values, float* provider);

/* ---- batched 128x128 heads ------------------------------------------------ */

/* Quant-only encode of `heads` contiguous 128x128 tiles in `layout`; codes keep
 * the input layout, smoothing is [heads][key], scales [heads][value]. */
void gdn_oracle_encode_heads(const float* state, uint64_t heads, uint32_t layout,
                             int8_t* codes, float* smoothing, float* value_scales,
                             int threads);

/* Quant-only decode (rank 0) of `heads` tiles. */
void gdn_oracle_decode_heads(const int8_t* codes, const float* smoothing,
                             const float* value_scales, uint64_t heads,
                             uint32_t layout, float* state, int threads);

/* Encoded decode projection, one boundary readout per (batch, value head):
 *   x[k]        = query_scale * bf16(queries[b][h * query_heads / value_heads][k])
 *   out[b][h][v]= (sum_k ((float)code[v,k] * s[k]) * x[k]) / 127 * scale[v]
 * in the reference's fp32 order (state_capsule.cpp:281-290).  out_f64 (nullable)
 * receives the same sum evaluated in double from the same x, and abs_bound
 * (nullable) receives sum_k |code*s*x| * scale / 127 in double, the magnitude
 * the fp32 error bound scales with. */
void gdn_oracle_project_decode(const int8_t* codes, const float* smoothing,
                               const float* value_scales, const uint16_t* queries,
                               uint32_t batch, uint32_t value_heads,
                               uint32_t query_heads, float query_scale,
                               uint32_t layout, float* out, double* out_f64,
                               double* abs_bound);

/* Chunked projection: the same readout for every token t of every sequence,
 * queries [seqs][tokens][query_heads][128] bf16, state [seqs][value_heads]
 * tiles, out [seqs][tokens][value_heads][128]. */
void gdn_oracle_project_chunked(const int8_t* codes, const float* smoothing,
                                const float* value_scales,
                                const uint16_t* queries, uint32_t seqs,
                                uint32_t tokens, uint32_t value_heads,
                                uint32_t query_heads, float query_scale,
                                uint32_t layout, float* out, double* out_f64,
                                double* abs_bound, int threads);

/* Slot-pool codec.  pool is [layers][slots][heads] tiles of dtype; the encoded
 * batch is compact [layers][batch][heads].  slot_ids[b] < 0 or >= slots skips
 * entry b (its encoded outputs and pool tiles are left untouched). */
void gdn_oracle_pool_encode(const void* pool, uint32_t pool_dtype,
                            const int32_t* slot_ids, uint32_t batch,
                            uint32_t layers, uint32_t slots, uint32_t heads,
                            uint32_t layout, int8_t* codes, float* smoothing,
                            float* value_scales, int threads);
void gdn_oracle_pool_decode(const int8_t* codes, const float* smoothing,
                            const float* value_scales, const int32_t* slot_ids,
                            uint32_t batch, uint32_t layers, uint32_t slots,
                            uint32_t heads, uint32_t layout, void* pool,
                            uint32_t pool_dtype, int threads);

/* bf16 helpers: widening is exact; narrowing is round-to-nearest-even, the
 * reference's FloatToBFloat16 (windowed_gdn_step.cpp:26-32). */
float gdn_oracle_bf16_to_f32(uint16_t value);
uint16_t gdn_oracle_f32_to_bf16(float value);

#ifdef __cplusplus
}
#endif

#endif /* GDN_ORACLE_H */
