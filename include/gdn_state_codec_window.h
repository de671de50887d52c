/*
 * C-ABI of the MI355X (gfx950) windowed GDN decode step: one token of the gated
 * delta rule evaluated against the encoded state (int8 boundary, rank-4 fp16
 * compensators and up to 15 buffered fp16 rank-one records) without
 * materializing it, plus the reference's decode-pair chain and dense fp32
 * step.  Same names, arguments, admission and status codes as the reference
 * (native/include/statecentric/gdn_state_codec_windowed_gdn_kernel.h).
 *
 * Buffers (one "state" = one value head of one sequence):
 *   residual        int8  [S][128][128]  [key][value] for the fp16 v1 step,
 *                                         [value][key] for the bf16 steps and
 *                                         the decode-pair chain
 *   smoothing       fp32  [S][128] (by key)    scales fp32 [S][128] (by value)
 *   compensator_keys fp16 [S][128][4]         compensator_values fp16 [S][128][4]
 *   record_decay    fp32  [S][16]             record_keys / record_corrections
 *                                              fp16 [S][16][128]
 *   positions       uint32 [S][8]  (word 0 is the window position, 0..16; the
 *                                   other words are never touched)
 * A step on a state at position p < 16 reads records 0..p-1, writes record p
 * and sets position p + 1; states at position >= 16 are left untouched (the
 * boundary refit must run first).
 *
 * Semantics (native/src/gdn_state_codec_state_capsule.cpp:354-397 with the
 * per-entry-point input mapping stated below): with S the encoded state,
 *   correction = value - S^T read,  out = S^T (query*gate) + correction*(w.query)
 * and the new record is {gate, w, fp16(correction)}.  All arithmetic is fp32;
 * outputs are within 2^-14 of the double-precision result's error scale (sum
 * of |terms|) before their final rounding -- tighter than the reference's
 * Ascend kernels, which accumulate the boundary readout in fp16.
 *
 * Every entry point is asynchronous on `stream` (NULL = HIP's null stream) and
 * returns 0 on success, 1 for a null pointer or an out-of-range count (the
 * reference's status 1), 5 when HIP rejects a launch.
 *
 * Alignment: every device pointer argument must be 16-byte aligned (see
 * gdn_state_codec_kernel.h); a misaligned pointer returns 1 before any launch
 * (the runtime steps too, ahead of their per-stage statuses).
 */
#ifndef GDN_STATE_CODEC_WINDOW_H
#define GDN_STATE_CODEC_WINDOW_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fp16 step, [key][value] residual, 1 <= states <= 16384.  write_keys, reads,
 * queries, values fp16 [S][128]; decay fp32 [S] is the linear gate g.
 * read = reads, query vector = queries*g, w = write_keys (stored as given),
 * outputs fp32 [S][128].  Replaces windowed_gdn_kernel.h:8-16
 * (kernel/gdn_state_codec_windowed_gdn_step.cpp:34-187, 667-688). */
int32_t statecentric_gdn_state_codec_windowed_gdn_step_launch_v1(
    void* stream, const int8_t* residual, const float* smoothing,
    const float* scales, const uint16_t* compensator_keys,
    const uint16_t* compensator_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    const float* decay, const uint16_t* write_keys, const uint16_t* reads,
    const uint16_t* queries, const uint16_t* values, float* outputs,
    uint32_t states);

/* bf16 step for Qwen3.5 decode, [value][key] residual, even states in
 * 1..16384.  decay fp32 [S] is log(g); beta bf16 [S]; keys and queries bf16
 * [S/2][128] (value head h reads key/query head h/2); values and outputs bf16
 * [S][128].  With k the key and q = 0.08838834764831845 * query:
 * read = g*k, query vector = q*g, w = beta*k.  Replaces
 * windowed_gdn_kernel.h:18-29 (windowed_gdn_step.cpp:189-619, 720-746). */
int32_t statecentric_gdn_state_codec_windowed_gdn_step_bf16_launch_v1(
    void* stream, const int8_t* residual, const float* smoothing,
    const float* scales, const uint16_t* compensator_keys,
    const uint16_t* compensator_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    const float* decay, const uint16_t* beta, const uint16_t* keys,
    const uint16_t* queries, const uint16_t* values, uint16_t* outputs,
    uint32_t states);

/* The bf16 step of a quant-only boundary: as above without the compensator
 * term (the compensator pointers are still required, as in the reference).
 * Replaces windowed_gdn_kernel.h:31-40 (windowed_gdn_step.cpp:748-775). */
int32_t statecentric_gdn_state_codec_windowed_gdn_step_bf16_quant_only_launch_v1(
    void* stream, const int8_t* residual, const float* smoothing,
    const float* scales, const uint16_t* compensator_keys,
    const uint16_t* compensator_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    const float* decay, const uint16_t* beta, const uint16_t* keys,
    const uint16_t* queries, const uint16_t* values, uint16_t* outputs,
    uint32_t states);

/* Dense fp32 GDN step on a [S][key][value] fp32 state, updated in place:
 * per value column c, projection = sum_r S[r][c]*read[r], correction =
 * value[c] - projection, S'[r][c] = decay*S[r][c] + key[r]*correction,
 * out[c] = sum_r S'[r][c]*query[r] (sequential fp32 sums, bit-identical to the
 * CPU statement of the reference kernel).  Replaces windowed_gdn_kernel.h:42-46
 * (kernel/gdn_state_codec_fp32_gdn_step.cpp:1-23). */
int32_t statecentric_gdn_state_codec_fp32_gdn_step_launch_v1(
    void* stream, float* dense_state, const float* decay,
    const uint16_t* write_keys, const uint16_t* reads, const uint16_t* queries,
    const uint16_t* values, float* outputs, uint32_t states);

/* ---- the reference's cube decode chain ------------------------------------
 * quantized int8 [S][128][16]: column 2c / 2c+1 hold the high / low int8 code of
 * vector c (c = 0: the read vector x s, c = 1: the output vector x s), columns
 * 4..15 are zero; dynamic_scale fp32 [S][8] holds {hi0, hi1, lo0, lo1};
 * projected int32 [S][128][16] = residual[value][key] x quantized (exact).
 * Rounding adds +-0.5 and truncates, as the reference does.  These kernels are
 * bit-identical to the reference's scalar code restated on the CPU. */

/* Replaces windowed_gdn_kernel.h:113-115
 * (kernel/gdn_state_codec_encoded_projection.cpp:179-234, 867-876). */
int32_t statecentric_gdn_state_codec_prepare_int8_vector_launch_v1(
    void* stream, const uint16_t* input, const float* axis_scale,
    int8_t* quantized, float* dynamic_scale, uint32_t states);

/* Replaces windowed_gdn_kernel.h:117-120 (encoded_projection.cpp:236-353, 878-890). */
int32_t statecentric_gdn_state_codec_prepare_decode_pair_launch_v1(
    void* stream, const uint16_t* reads, const uint16_t* queries,
    const float* decay, const float* smoothing, int8_t* quantized,
    float* dynamic_scale, uint32_t states);

/* Replaces windowed_gdn_kernel.h:122-131 (encoded_projection.cpp:482-621, 892-918). */
int32_t statecentric_gdn_state_codec_finish_decode_pair_launch_v1(
    void* stream, const int32_t* projected, const float* dynamic_scale,
    const float* scales, const uint16_t* compensator_keys,
    const uint16_t* compensator_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    const float* decay, const uint16_t* write_keys, const uint16_t* reads,
    const uint16_t* queries, const uint16_t* values, float* outputs,
    uint32_t states);

/* Replaces windowed_gdn_kernel.h:133-137 (encoded_projection.cpp:355-479, 920-933). */
int32_t statecentric_gdn_state_codec_prepare_decode_pair_bf16_launch_v1(
    void* stream, const uint16_t* keys, const uint16_t* queries,
    const float* decay, const float* smoothing, int8_t* quantized,
    float* dynamic_scale, uint32_t states);

/* Replaces windowed_gdn_kernel.h:139-149 (encoded_projection.cpp:624-776, 935-963). */
int32_t statecentric_gdn_state_codec_finish_decode_pair_bf16_launch_v1(
    void* stream, const int32_t* projected, const float* dynamic_scale,
    const float* scales, const uint16_t* compensator_keys,
    const uint16_t* compensator_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    const float* decay, const uint16_t* beta, const uint16_t* keys,
    const uint16_t* queries, const uint16_t* values, uint16_t* outputs,
    uint32_t states);

/* c[s] = a[s] (transposed when transpose_a) x b[s], a int8 [128][128], b int8
 * [128][16], c int32 [128][16], exact.  Admission as the reference: workspace
 * and tiling non-null (they are not read here), 1 <= states <= 128,
 * blocks == (states + 1) / 2, transpose_a <= 1.  Replaces
 * windowed_gdn_kernel.h:108-111 (kernel/gdn_state_codec_int8_cube_matmul.cpp:53-68). */
int32_t statecentric_gdn_state_codec_int8_cube_matmul_launch_v1(
    void* stream, const int8_t* a, const int8_t* b, int32_t* c, uint32_t states,
    uint32_t transpose_a, void* workspace, void* tiling, uint32_t blocks);

/* The same product over any batch, 1 <= states <= 16384 (the window steps'
 * admission), in one launch: the v1 limit of 128 states is the reference's
 * Cube block count, not a property of the product.  No workspace or tiling.
 * Batched counterpart of int8_cube_matmul_launch_v1 above
 * (windowed_gdn_kernel.h:108-111), for callers that run the rank chain over a
 * whole decode batch. */
int32_t statecentric_gdn_state_codec_int8_matmul_launch_v4(
    void* stream, const int8_t* a, const int8_t* b, int32_t* c, uint32_t states,
    uint32_t transpose_a);

/* ---- the reference's device rank-4 chain over an encoded boundary ----------
 * (driven by host/gdn_state_codec_encoded_projection_probe.cpp:571-677:
 * prepare_int8_vector -> int8_cube_matmul -> finish_encoded_projection, forward
 * and transposed, per power iteration; then prepare -> GEMM ->
 * commit_encoded_rank per rank; then encoded_requantize.)  Per state: vector
 * operands fp16 / int32 / fp32 [128][16] of which column 0 is the vector;
 * dynamic_scale fp32 [8] (element 0); old_left / old_right fp16 [128][4]
 * ([dim][rank]); new_left / new_right fp16 [4][128] ([rank][dim]); record_left /
 * record_right fp16 [16][128]; record_decay fp32 [16]; smoothing / scales fp32
 * [128].  Each row of the window operator (transpose 0, rows on the smoothing
 * axis) or of its transpose is p * dyn / 127 * axis * B + the old ranks * B -
 * the first `fitted_ranks` fitted ranks + the records * their suffixes, with
 * every sum sequential in the reference's order: results are bit-identical to
 * the reference's scalar code restated on the CPU.  1 <= states <= 16384. */

/* output column 0 = fp16(value / |value|) (0 when |value|^2 <= 1e-20), columns
 * 1..15 = 0; fitted_ranks <= 4, transpose <= 1.  Replaces
 * windowed_gdn_kernel.h:151-160 (kernel/gdn_state_codec_encoded_projection.cpp:778-820,
 * 964-990). */
int32_t statecentric_gdn_state_codec_finish_encoded_projection_launch_v1(
    void* stream, const int32_t* projected, const float* dynamic_scale,
    const uint16_t* input, const float* smoothing, const float* scales,
    const uint16_t* old_left, const uint16_t* old_right, const float* record_decay,
    const uint16_t* record_left, const uint16_t* record_right, const uint16_t* new_left,
    const uint16_t* new_right, uint16_t* output, uint32_t states, uint32_t fitted_ranks,
    uint32_t transpose);

/* The forward rows with ranks 0..rank-1 deflated: corrected column 0 = value
 * (other columns untouched), new_left[rank] = fp16(value), new_right[rank] =
 * the input's fp16 bits; rank < 4.  Replaces windowed_gdn_kernel.h:162-169
 * (encoded_projection.cpp:822-865, 992-1015). */
int32_t statecentric_gdn_state_codec_commit_encoded_rank_launch_v1(
    void* stream, const int32_t* projected, const float* dynamic_scale,
    const uint16_t* input, const float* smoothing, const float* scales,
    const uint16_t* old_left, const uint16_t* old_right, const float* record_decay,
    const uint16_t* record_left, const uint16_t* record_right, uint16_t* new_left,
    uint16_t* new_right, float* corrected, uint32_t states, uint32_t rank);

/* The whole rank chain above in one launch, for callers that would
 * otherwise issue it stage by stage: for each rank r = 0..3 the vector
 * seeds[s][r] (fp16 [S][4][128]) is projected and finished forward and
 * transposed `iterations` times with r fitted ranks, then projected once more
 * and committed as rank r.  Every stage is the corresponding entry point's
 * arithmetic (prepare_int8_vector, the int8 product, finish / commit), so
 * new_left / new_right (fp16 [S][4][128], the layout commit writes) are
 * bit-identical to the launch-per-stage chain with reset (zero) fitted bases,
 * and corrected[s][r] (fp32 [S][4][128]) holds column 0 of rank r's commit.
 * The other operands are those of finish_encoded_projection_launch_v1.  One
 * 256-thread workgroup per state keeps the vector in LDS and the int8 boundary
 * in registers, so the [S][128][16] vector arrays are not used.
 * 1 <= states <= 16384, 1 <= iterations <= 64.  Batched counterpart of the
 * stage-by-stage chain host/gdn_state_codec_encoded_projection_probe.cpp:
 * 611-636 drives through windowed_gdn_kernel.h:108-169. */
int32_t statecentric_gdn_state_codec_encoded_rank_chain_launch_v4(
    void* stream, const int8_t* residual, const float* smoothing, const float* scales,
    const uint16_t* old_left, const uint16_t* old_right, const float* record_decay,
    const uint16_t* record_left, const uint16_t* record_right, const uint16_t* seeds,
    uint16_t* new_left, uint16_t* new_right, float* corrected, uint32_t states,
    uint32_t iterations);

/* residual int8 [S][128][128] as [smoothing axis][scale axis]; the window
 * operator minus new_left^T new_right, re-encoded exactly as the rank-4
 * window-boundary refit re-encodes (fresh smoothing, absmax scales,
 * round-half-away codes, the fitted residual into residual_workspace
 * [S][128][128]); next_left / next_right = the new bases as [dim][rank].
 * next_* must not alias the inputs.  Replaces windowed_gdn_kernel.h:171-179
 * (kernel/gdn_state_codec_encoded_requantize.cpp:102-166, 189-215). */
int32_t statecentric_gdn_state_codec_encoded_requantize_launch_v1(
    void* stream, const int8_t* residual, const float* smoothing, const float* scales,
    const uint16_t* old_left, const uint16_t* old_right, const float* record_decay,
    const uint16_t* record_left, const uint16_t* record_right, const uint16_t* new_left,
    const uint16_t* new_right, int8_t* next_residual, float* next_smoothing,
    float* next_scales, uint16_t* next_left, uint16_t* next_right,
    float* residual_workspace, uint32_t states);

/* ---- decode runtime (host/gdn_state_codec_decode_runtime.cpp:72-148) ------
 * create returns a process-wide handle for `states` (1..16384; nullptr when a
 * live handle has a different count), reference-counted; destroy drops one
 * reference and ignores foreign handles.  step runs prepare_decode_pair_bf16,
 * the int8 projection and finish_decode_pair_bf16 as ONE fused kernel (one
 * pass over the codes), with results bit-identical to running the three
 * stages; it returns 1 for a bad handle/stream/count.  Unlike the reference,
 * whose Cube GEMM admits at most 128 states, every admitted count runs. */
void* statecentric_gdn_state_codec_decode_runtime_create_v1(uint32_t states);
void statecentric_gdn_state_codec_decode_runtime_destroy_v1(void* runtime);
int32_t statecentric_gdn_state_codec_decode_runtime_step_v1(
    void* runtime, void* stream, const int8_t* residual, const float* smoothing,
    const float* scales, const uint16_t* compensator_keys,
    const uint16_t* compensator_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    const float* decay, const uint16_t* beta, const uint16_t* keys,
    const uint16_t* queries, const uint16_t* values, uint16_t* outputs,
    uint32_t states);

/* ---- window-boundary refit (kernel/gdn_state_codec_window_boundary.cpp) ---
 * Boundaries are [value][key]; next_* buffers must not alias the inputs.
 * All of these are bit-identical to the CPU statement of the reference
 * kernels (with Axpy's product rounded before the add and the fp16 record
 * GEMM summing in ascending record order). */

/* power_iterations == 0: every state is re-encoded with its EXISTING smoothing
 * from the dequantized boundary times the product S of its 16 record gates
 * plus the 16 record terms key_j[k] * (corr_j[v] * suffix_j):
 * m = w / s, scale' = max|m|, code' = rint_even(fp16(clamp(m * (127 / scale'))));
 * next compensators are zero, records are kept, every position is reset to 0
 * (the reference's finalize kernel).  power_iterations in 1..32: for each state
 * at position 16, a deflated rank-4 power-iteration fit of the window's
 * residual operator (stored as fp16 compensators), fresh smoothing
 * sqrt(mean|row|) by 20 Newton steps, absmax scales, round-half-away codes,
 * residual_workspace [S][key][value] receives the fitted residual, records are
 * cleared and the position reset; states at other positions are untouched.
 * 1 <= states <= 16384.  Replaces windowed_gdn_kernel.h:50-60
 * (window_boundary.cpp:253-499, 653-696). */
int32_t statecentric_gdn_state_codec_window_boundary_launch_v1(
    void* stream, const int8_t* residual, const float* smoothing,
    const float* scales, const uint16_t* compensator_keys,
    const uint16_t* compensator_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    int8_t* next_residual, float* next_smoothing, float* next_scales,
    uint16_t* next_compensator_keys, uint16_t* next_compensator_values,
    float* residual_workspace, uint32_t states, uint32_t power_iterations);

/* window_boundary_launch_v1 without the residual_workspace argument, for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops and harnesses that forbid hipMalloc).  No counterpart exists in
 * the reference.  The power refit's fitted residual goes to the library's own
 * 32 MiB scratch array, one per GPU (held from the library's first use on that
 * GPU until the process ends), so power_iterations in 1..32 admits
 * 1 <= states <= 512; power_iterations == 0 needs no workspace and admits
 * 1 <= states <= 16384.  Out-of-range counts and null pointers return 1, a
 * failed lookup of the scratch array's device address returns 5.  The call
 * allocates nothing.  Outputs are bit-identical to window_boundary_launch_v1.
 * Every call on one GPU shares that GPU's array: calls that overlap in time
 * on one GPU (other streams, other host threads) race on it. */
int32_t statecentric_gdn_state_codec_window_boundary_noalloc_launch_v1(
    void* stream, const int8_t* residual, const float* smoothing,
    const float* scales, const uint16_t* compensator_keys,
    const uint16_t* compensator_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    int8_t* next_residual, float* next_smoothing, float* next_scales,
    uint16_t* next_compensator_keys, uint16_t* next_compensator_values,
    uint32_t states, uint32_t power_iterations);

/* scaled_record_keys[s][j][k] = fp16(key_j[k] * fp16(prod_{i>j} gate_i)), the
 * gate product taken in ascending order; 1 <= states <= 128.  Replaces
 * windowed_gdn_kernel.h:62-67 (window_boundary.cpp:537-587, 698-712). */
int32_t statecentric_gdn_state_codec_boundary_scale_records_launch_v1(
    void* stream, const float* record_decay, const uint16_t* record_keys,
    uint16_t* scaled_record_keys, uint32_t states);

/* The quant-only refit above with the 16 record terms replaced by
 * record_merge [S][value][key] fp32 (the boundary runtime's output);
 * 1 <= states <= 128.  Replaces windowed_gdn_kernel.h:69-79
 * (window_boundary.cpp:714-750). */
int32_t statecentric_gdn_state_codec_window_boundary_cube_finish_launch_v1(
    void* stream, const int8_t* residual, const float* smoothing,
    const float* scales, const uint16_t* compensator_keys,
    const uint16_t* compensator_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    int8_t* next_residual, float* next_smoothing, float* next_scales,
    uint16_t* next_compensator_keys, uint16_t* next_compensator_values,
    float* record_merge, uint32_t states);

/* c[s] = a[s]^T b[s]: a, b fp16 [16][128], c fp32 [128][128], exact products
 * summed in ascending k.  Admission as the reference (workspace and tiling
 * non-null but unused, states <= 128, blocks == (states + 1) / 2).  Replaces
 * windowed_gdn_kernel.h:81-84 (kernel/gdn_state_codec_bf16_cube_matmul.cpp:50-68). */
int32_t statecentric_gdn_state_codec_bf16_cube_matmul_launch_v1(
    void* stream, const uint16_t* a, const uint16_t* b, float* c, uint32_t states,
    void* workspace, void* tiling, uint32_t blocks);

/* Boundary runtime (host/gdn_state_codec_boundary_runtime.cpp:60-128): one
 * process-wide reference-counted handle for 1..128 states; step scales the
 * record keys then forms record_merge = corrections^T x scaled keys, returning
 * 1 for a bad handle/pointer/count, 2 / 3 when the scaling / GEMM launch fails. */
void* statecentric_gdn_state_codec_boundary_runtime_create_v1(uint32_t states);
void statecentric_gdn_state_codec_boundary_runtime_destroy_v1(void* runtime);
int32_t statecentric_gdn_state_codec_boundary_runtime_step_v1(
    void* runtime, void* stream, const float* record_decay,
    const uint16_t* record_keys, const uint16_t* record_corrections,
    uint16_t* scaled_record_keys, float* record_merge, uint32_t states);

#ifdef __cplusplus
}
#endif

#endif /* GDN_STATE_CODEC_WINDOW_H */
