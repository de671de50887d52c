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
/* gdn_oracle_f32_to_bf16 over an array. */
void gdn_oracle_f32_to_bf16_array(const float* values, uint64_t count, uint16_t* out);

/* fp16 helpers (IEEE binary16): widening is exact; narrowing rounds to nearest
 * even with subnormals and overflow to infinity. */
float gdn_oracle_f16_to_f32(uint16_t value);
uint16_t gdn_oracle_f32_to_f16(float value);

/* ---- windowed decode step (gdn_window_oracle.c) ---------------------------
 *
 * Parity pins:
 *   read_window / dense_state / apply_token : bit-exact vs oracle/_ref, which
 *        drives the reference capsule (ApplyToken over whole windows, rank 0
 *        and rank 4, including the window-boundary requantize).
 *   windowed_step_{bf16,f16}, gdn_step_f32 : built from read_window plus the
 *        device kernels' input conventions; checked against the dense fp32 GDN
 *        step on the reconstructed state (the reference probe's own check,
 *        windowed_gdn_runtime_probe.cpp:94-147, here to 2^-14 of the error
 *        scale instead of 0.25% RMS) and against their own double results.
 *   decode-pair chain : the reference kernels' scalar fp32 code restated
 *        statement by statement; the chain is checked end to end against
 *        windowed_step_* within its documented int8 vector quantization error.
 * Every device entry point takes g = RN_fp32(exp(log_decay)) (evaluated as
 * (float)exp((double)x)) where the reference evaluates Ascend's Exp. */

/* ReadWindowState (state_capsule.cpp:253-306): [key][value] boundary, records
 * u = 0..records-1 with per-key decay [records][keys], key [records][keys] and
 * correction [records][values]; output[v] = S^T read. */
void gdn_oracle_read_window(const int8_t* codes, const float* smoothing,
                            const float* value_scales, const float* comp_keys,
                            const float* comp_values, uint32_t keys,
                            uint32_t values, uint32_t rank,
                            const float* record_decay, const float* record_keys,
                            const float* record_corrections, uint32_t records,
                            const float* read, float* output);

/* DenseState (state_capsule.cpp:337-352). */
void gdn_oracle_dense_state(const int8_t* codes, const float* smoothing,
                            const float* value_scales, const float* comp_keys,
                            const float* comp_values, uint32_t keys,
                            uint32_t values, uint32_t rank,
                            const float* record_decay, const float* record_keys,
                            const float* record_corrections, uint32_t records,
                            float* state);

/* ApplyToken (state_capsule.cpp:354-397).  The boundary arrays are replaced in
 * place when the window fills (DenseState then QuantizeBoundary at the same
 * rank); record arrays hold `window` rows; *records is the window position.
 * Returns 1 when the token crossed the window boundary. */
int gdn_oracle_apply_token(int8_t* codes, float* smoothing, float* value_scales,
                           float* comp_keys, float* comp_values, uint32_t keys,
                           uint32_t values, uint32_t rank, uint32_t window,
                           float* record_decay, float* record_keys,
                           float* record_corrections, uint32_t* records,
                           const float* decay, const float* key,
                           const float* value, const float* read,
                           const float* query, float* output);

/* windowed_gdn_step_bf16{,_quant_only}_launch_v1 on device buffers
 * (kernel/gdn_state_codec_windowed_gdn_step.cpp:326-619, 720-775).
 * residual [S][value][key] int8; comp_keys [S][key][4] / comp_values
 * [S][value][4] fp16, both NULL for the quant-only form; record_decay [S][16]
 * fp32; record_keys / record_corrections [S][16][128] fp16; positions [S][8];
 * log_decay fp32 [S]; beta bf16 [S]; keys / queries bf16 [S/2][128] (value head
 * h reads head h/2); values / outputs bf16 [S][128].  With g = exp(log_decay),
 * key k, q = 0.08838834764831845 * query:
 *   read = g*k, output vector = q*g, write key = beta*k,
 *   correction = value - S^T read, out = S^T (q*g) + correction * (beta*k . q),
 * then record p = {g, fp16(beta*k), fp16(correction)} and position p+1.
 * States at position >= 16 are untouched.  out64 / corr64 (nullable) receive
 * the output and correction before rounding, in double, and out_bound /
 * corr_bound the magnitude their fp32 evaluation error scales with. */
void gdn_oracle_windowed_step_bf16(
    const int8_t* residual, const float* smoothing, const float* scales,
    const uint16_t* comp_keys, const uint16_t* comp_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    const float* log_decay, const uint16_t* beta, const uint16_t* keys,
    const uint16_t* queries, const uint16_t* values, uint16_t* outputs,
    uint32_t states, double* out64, double* out_bound, double* corr64,
    double* corr_bound);

/* windowed_gdn_step_launch_v1 (windowed_gdn_step.cpp:34-187, 667-688):
 * residual [S][key][value]; fp16 write_keys / reads / queries / values
 * [S][128]; linear decay fp32 [S]; fp32 outputs; fp16 rank-4 compensators.
 *   correction = value - S^T read, out = S^T (query*decay) + correction *
 *   (write_key . query); record p = {decay, write_key, fp16(correction)}. */
void gdn_oracle_windowed_step_f16(
    const int8_t* residual, const float* smoothing, const float* scales,
    const uint16_t* comp_keys, const uint16_t* comp_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    const float* decay, const uint16_t* write_keys, const uint16_t* reads,
    const uint16_t* queries, const uint16_t* values, float* outputs,
    uint32_t states, double* out64, double* out_bound, double* corr64,
    double* corr_bound);

/* fp32_gdn_step_launch_v1 (kernel/gdn_state_codec_fp32_gdn_step.cpp:13-18):
 * dense [S][key][value] fp32 state updated in place. */
void gdn_oracle_gdn_step_f32(float* state, const float* decay,
                             const uint16_t* keys, const uint16_t* reads,
                             const uint16_t* queries, const uint16_t* values,
                             float* outputs, uint32_t states);

/* The cube decode chain (kernel/gdn_state_codec_encoded_projection.cpp and
 * int8_cube_matmul.cpp), statement by statement: quantized [S][128][16] int8
 * (columns hi0, lo0, hi1, lo1, then zeros), dynamic_scale [S][8] (hi0, hi1,
 * lo0, lo1), projected [S][128][16] int32. */
void gdn_oracle_prepare_decode_pair_bf16(const uint16_t* keys,
                                         const uint16_t* queries,
                                         const float* log_decay,
                                         const float* smoothing,
                                         int8_t* quantized, float* dynamic_scale,
                                         uint32_t states);
void gdn_oracle_prepare_decode_pair(const uint16_t* reads, const uint16_t* queries,
                                    const float* decay, const float* smoothing,
                                    int8_t* quantized, float* dynamic_scale,
                                    uint32_t states);
void gdn_oracle_prepare_int8_vector(const uint16_t* input, const float* axis_scale,
                                    int8_t* quantized, float* dynamic_scale,
                                    uint32_t states);
void gdn_oracle_int8_matmul(const int8_t* a, const int8_t* b, int32_t* c,
                            uint32_t states, uint32_t transpose_a);
void gdn_oracle_finish_decode_pair_bf16(
    const int32_t* projected, const float* dynamic_scale, const float* scales,
    const uint16_t* comp_keys, const uint16_t* comp_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    const float* log_decay, const uint16_t* beta, const uint16_t* keys,
    const uint16_t* queries, const uint16_t* values, uint16_t* outputs,
    uint32_t states);
void gdn_oracle_finish_decode_pair(
    const int32_t* projected, const float* dynamic_scale, const float* scales,
    const uint16_t* comp_keys, const uint16_t* comp_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    const float* decay, const uint16_t* write_keys, const uint16_t* reads,
    const uint16_t* queries, const uint16_t* values, float* outputs,
    uint32_t states);

/* ---- window-boundary refit (gdn_boundary_oracle.c) ------------------------
 *
 * Parity pins: statement-by-statement restatements of
 * kernel/gdn_state_codec_window_boundary.cpp and bf16_cube_matmul.cpp; checked
 * against the capsule semantics they approximate (the refit dense state equals
 * DenseState of the window within the quantization error, the power
 * iteration's first pair is the dominant singular pair of the closed-form
 * residual operator computed independently in numpy) and the invariants of
 * their output formats.  Two evaluation orders the reference leaves to the
 * hardware are fixed: AscendC::Axpy is dst = src * s + dst with a rounded
 * product, and the fp16 record-merge GEMM sums its 16 products in ascending k.
 *
 * Boundaries are [value][key] (the provider layout); records, compensators and
 * positions as in the windowed step. */

/* The 20-step Newton square root of window_boundary.cpp:17-23. */
float gdn_oracle_boundary_sqrt(float value);

/* window_boundary_launch_v1 with power_iterations == 0 (ProcessQuantOnlyTask,
 * :368-499, plus the finalize kernel): every state is re-encoded with its
 * existing smoothing from the dequantized boundary plus all 16 records
 * (record_merge == NULL) or plus record_merge [S][value][key] fp32 (the
 * window_boundary_cube_finish_launch_v1 form); compensator outputs are zero,
 * records untouched, every position reset to 0. */
void gdn_oracle_window_boundary_quant_only(
    const int8_t* residual, const float* smoothing, const float* scales,
    const float* record_decay, const uint16_t* record_keys,
    const uint16_t* record_corrections, uint32_t* positions,
    int8_t* next_residual, float* next_smoothing, float* next_scales,
    uint16_t* next_comp_keys, uint16_t* next_comp_values,
    const float* record_merge, uint32_t states);

/* boundary_scale_records_launch_v1 (:537-587, 698-712). */
void gdn_oracle_boundary_scale_records(const float* record_decay,
                                       const uint16_t* record_keys,
                                       uint16_t* scaled_record_keys,
                                       uint32_t states);

/* bf16_cube_matmul_launch_v1: C[s] = A[s]^T B[s], A and B fp16 [16][128]. */
void gdn_oracle_f16_matmul_at_b(const uint16_t* a, const uint16_t* b, float* c,
                                uint32_t states);

/* window_boundary_launch_v1 with power_iterations in 1..32 (ProcessState,
 * :253-366): for each state at position 16, a rank-4 power-iteration fit of
 * the window's residual operator, re-encoding with fresh smoothing, records
 * cleared and position reset; other states untouched. */
void gdn_oracle_window_boundary_power(
    const int8_t* residual, const float* smoothing, const float* scales,
    const uint16_t* comp_keys, const uint16_t* comp_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    int8_t* next_residual, float* next_smoothing, float* next_scales,
    uint16_t* next_comp_keys, uint16_t* next_comp_values,
    float* residual_workspace, uint32_t states, uint32_t power_iterations);

/* ---- device rank-4 chain over an encoded boundary (gdn_encoded_oracle.c) ---
 *
 * encoded_projection.cpp:82-163, 778-865 and encoded_requantize.cpp:72-166;
 * layouts in the header of gdn_encoded_oracle.c.  Parity pins: the requantize
 * against the pinned power-refit restatement fed the same fit, float64 brute
 * force of the operator rows, closed forms of the commit outputs, and planted
 * negative controls (tests/test_oracle_encoded.py). */
void gdn_oracle_finish_encoded_projection(
    const int32_t* projected, const float* dynamic_scale, const uint16_t* input,
    const float* smoothing, const float* scales, const uint16_t* old_left,
    const uint16_t* old_right, const float* record_decay, const uint16_t* record_left,
    const uint16_t* record_right, const uint16_t* new_left, const uint16_t* new_right,
    uint16_t* output, uint32_t states, uint32_t fitted_ranks, uint32_t transpose);
void gdn_oracle_commit_encoded_rank(
    const int32_t* projected, const float* dynamic_scale, const uint16_t* input,
    const float* smoothing, const float* scales, const uint16_t* old_left,
    const uint16_t* old_right, const float* record_decay, const uint16_t* record_left,
    const uint16_t* record_right, uint16_t* new_left, uint16_t* new_right,
    float* corrected, uint32_t states, uint32_t rank);
void gdn_oracle_encoded_requantize(
    const int8_t* residual, const float* smoothing, const float* scales,
    const uint16_t* old_left, const uint16_t* old_right, const float* record_decay,
    const uint16_t* record_left, const uint16_t* record_right, const uint16_t* new_left,
    const uint16_t* new_right, int8_t* next_residual, float* next_smoothing,
    float* next_scales, uint16_t* next_left, uint16_t* next_right,
    float* residual_workspace, uint32_t states);

/* ---- capsule wire format LQCAPS01 (gdn_capsule_oracle.c) ------------------
 *
 * Parity pins: SHA-256 vs FIPS 180-4 vectors, hashlib and the reference's
 * Sha256Hex; serialize / restore vs the reference's Serialize / Restore
 * (oracle/_ref) on reference-built capsules, the reference test's corruptions
 * and slot capsules (see the header of gdn_capsule_oracle.c). */

/* Restore outcomes, one per check of GdnStateCodecCapsule::Restore
 * (state_capsule.cpp:476-578) in the order the reference makes them. */
#define GDN_ORACLE_CAPSULE_OK 0
#define GDN_ORACLE_CAPSULE_TRUNCATED 1          /* too short / truncated field */
#define GDN_ORACLE_CAPSULE_MAGIC 2
#define GDN_ORACLE_CAPSULE_DIGEST_ENCODING 3    /* digest not lowercase hex */
#define GDN_ORACLE_CAPSULE_DIGEST_MISMATCH 4
#define GDN_ORACLE_CAPSULE_PARAMETERS 5
#define GDN_ORACLE_CAPSULE_IDENTITY 6
#define GDN_ORACLE_CAPSULE_RANK 7
#define GDN_ORACLE_CAPSULE_POSITION 8           /* window position >= window */
#define GDN_ORACLE_CAPSULE_PHASE 9              /* position != expected */
#define GDN_ORACLE_CAPSULE_RESIDUAL_DOMAIN 10   /* a code equals -128 */
#define GDN_ORACLE_CAPSULE_BOUNDARY_PAYLOAD 11
#define GDN_ORACLE_CAPSULE_RECORD_NONFINITE 12
#define GDN_ORACLE_CAPSULE_TRAILING 13
#define GDN_ORACLE_CAPSULE_STATE_NONFINITE 14
#define GDN_ORACLE_CAPSULE_DEVICE_FORMAT 15     /* slot restore only */
#define GDN_ORACLE_CAPSULE_ARGUMENT 17          /* expected identity/parameters invalid */

void gdn_oracle_sha256(const uint8_t* data, uint64_t size, uint8_t digest[32]);
void gdn_oracle_sha256_hex(const uint8_t* data, uint64_t size, char hex[64]);

/* Encoded size: header 120 + codes + fp32 smoothing, scales, compensators and
 * records + 64 digest characters. */
uint64_t gdn_oracle_capsule_bytes(uint32_t keys, uint32_t values, uint32_t rank,
                                  uint32_t updates);

/* Serialize (state_capsule.cpp:446-474); returns the byte count. */
uint64_t gdn_oracle_capsule_serialize(
    const char* geometry, uint64_t generation, uint64_t epoch, uint32_t keys,
    uint32_t values, uint32_t schema, uint32_t window, uint32_t rank, uint32_t bits,
    float smoothing_floor, const int8_t* residual, const float* smoothing,
    const float* scales, const float* comp_keys, const float* comp_values,
    uint32_t updates, const float* decay, const float* key, const float* correction,
    uint8_t* out);

/* Restore (state_capsule.cpp:476-578): a GDN_ORACLE_CAPSULE_* outcome; the
 * fields are complete only on success.  dense_work holds keys*values floats. */
int gdn_oracle_capsule_restore(
    const uint8_t* encoded, uint64_t size, const char* geometry, uint64_t generation,
    uint64_t epoch, uint32_t keys, uint32_t values, uint32_t schema, uint32_t window,
    uint32_t rank, uint32_t bits, float smoothing_floor, uint32_t expected_position,
    int8_t* residual, float* smoothing, float* scales, float* comp_keys,
    float* comp_values, float* decay, float* key, float* correction,
    float* dense_work, uint32_t* updates_out);

/* One device window slot state (128x128, rank 4, window 16) as a capsule, and
 * back.  serialize returns 0 for a position >= 16; restore writes the slot
 * only on success and refuses (DEVICE_FORMAT) a capsule whose per-key decays
 * differ within a record or whose compensators / records are not fp16. */
uint64_t gdn_oracle_slot_capsule_bytes(uint32_t position);
uint64_t gdn_oracle_slot_capsule_serialize(
    uint32_t layout, const int8_t* residual, const float* smoothing, const float* scales,
    const uint16_t* comp_keys, const uint16_t* comp_values, const float* record_decay,
    const uint16_t* record_keys, const uint16_t* record_corrections, uint32_t position,
    const char* geometry, uint64_t generation, uint64_t epoch, uint8_t* out);
int gdn_oracle_slot_capsule_restore(
    const uint8_t* encoded, uint64_t size, const char* geometry, uint64_t generation,
    uint64_t epoch, uint32_t expected_position, uint32_t layout, int8_t* residual,
    float* smoothing, float* scales, uint16_t* comp_keys, uint16_t* comp_values,
    float* record_decay, uint16_t* record_keys, uint16_t* record_corrections,
    uint32_t* position_word);

#ifdef __cplusplus
}
#endif

#endif /* GDN_ORACLE_H */
