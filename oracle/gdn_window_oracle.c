/*
 * CPU oracle for the windowed GDN decode step.
 *
 * TEST INFRASTRUCTURE ONLY (see gdn_oracle.h): loaded by tests/ and
 * __graft_entry__.smoke() as the checker, never by the product library.
 *
 * Two layers:
 *   - the capsule semantics, restated in the reference's own fp32 operation
 *     order: ReadWindowState (native/src/gdn_state_codec_state_capsule.cpp:
 *     253-306), DenseState (:337-352) and ApplyToken (:354-397).  Pinned
 *     bit-exactly against oracle/_ref, which runs the reference capsule.
 *   - the device entry points' contracts on their own buffer formats (fp16 /
 *     bf16 vectors and records, [state][8] positions, log decay, GQA), from
 *     native/ascendc/gdn_state_codec/kernel/gdn_state_codec_windowed_gdn_step.cpp,
 *     ...encoded_projection.cpp and ...fp32_gdn_step.cpp.  The readouts use the
 *     capsule functions above; every step also returns the pre-rounding result
 *     in double with the magnitude its fp32 rounding error scales with.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "gdn_oracle.h"

#define DIM 128u
#define TILE (DIM * DIM)
#define RANK 4u
#define WINDOW 16u
#define POSITION_STRIDE 8u
#define QUERY_SCALE 0.08838834764831845f

/* ------------------------------------------------------------------ fp16 */

float gdn_oracle_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exponent = (h >> 10) & 0x1Fu;
  const uint32_t mantissa = h & 0x3FFu;
  if (exponent == 0) {
    const float v = ldexpf((float)mantissa, -24);
    return sign ? -v : v;
  }
  uint32_t bits;
  if (exponent == 31) {
    bits = sign | 0x7F800000u | (mantissa << 13);
  } else {
    bits = sign | ((exponent - 15u + 127u) << 23) | (mantissa << 13);
  }
  float out;
  memcpy(&out, &bits, 4);
  return out;
}

uint16_t gdn_oracle_f32_to_f16(float value) {
  uint32_t x;
  memcpy(&x, &value, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t magnitude = x & 0x7FFFFFFFu;
  if (magnitude >= 0x7F800000u) {  /* inf / nan */
    return (uint16_t)(sign | 0x7C00u |
                      (magnitude > 0x7F800000u ? 0x200u | ((magnitude >> 13) & 0x3FFu) : 0u));
  }
  if (magnitude < 0x38800000u) {  /* below 2^-14: subnormal (or zero) half */
    float v;
    memcpy(&v, &magnitude, 4);
    const float units = v * 16777216.0f;  /* exact: scaling by 2^24 */
    return (uint16_t)(sign | (uint16_t)nearbyintf(units));
  }
  uint32_t h = (((magnitude >> 23) - 112u) << 10) | ((magnitude >> 13) & 0x3FFu);
  const uint32_t rest = magnitude & 0x1FFFu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1u;  /* carries into inf */
  if (h > 0x7C00u) h = 0x7C00u;
  return (uint16_t)(sign | h);
}

/* The device steps take g = exp(log_decay) rounded once to fp32. */
static float exp_f32(float x) { return (float)exp((double)x); }

/* -------------------------------------------------------- capsule layer */

void gdn_oracle_read_window(const int8_t* codes, const float* smoothing,
                            const float* value_scales, const float* comp_keys,
                            const float* comp_values, uint32_t keys,
                            uint32_t values, uint32_t rank,
                            const float* record_decay, const float* record_keys,
                            const float* record_corrections, uint32_t records,
                            const float* read, float* output) {
  /* state_capsule.cpp:262-305, same loop order and expression order. */
  float* suffix_read = (float*)malloc(sizeof(float) * keys);
  for (uint32_t row = 0; row < keys; ++row) suffix_read[row] = read[row];
  for (uint32_t column = 0; column < values; ++column) output[column] = 0.0f;
  for (uint32_t index = records; index > 0; --index) {
    const uint32_t u = index - 1;
    float projection = 0.0f;
    for (uint32_t row = 0; row < keys; ++row) {
      projection += record_keys[(size_t)u * keys + row] * suffix_read[row];
    }
    for (uint32_t column = 0; column < values; ++column) {
      output[column] += record_corrections[(size_t)u * values + column] * projection;
    }
    for (uint32_t row = 0; row < keys; ++row) {
      suffix_read[row] *= record_decay[(size_t)u * keys + row];
    }
  }
  for (uint32_t column = 0; column < values; ++column) {
    float residual_projection = 0.0f;
    for (uint32_t row = 0; row < keys; ++row) {
      residual_projection += (float)codes[(size_t)row * values + column] *
                             smoothing[row] * suffix_read[row];
    }
    output[column] += residual_projection / 127.0f * value_scales[column];
  }
  for (uint32_t r = 0; r < rank; ++r) {
    float projection = 0.0f;
    for (uint32_t row = 0; row < keys; ++row) {
      projection += comp_keys[(size_t)row * rank + r] * suffix_read[row];
    }
    for (uint32_t column = 0; column < values; ++column) {
      output[column] += comp_values[(size_t)column * rank + r] * projection;
    }
  }
  free(suffix_read);
}

void gdn_oracle_dense_state(const int8_t* codes, const float* smoothing,
                            const float* value_scales, const float* comp_keys,
                            const float* comp_values, uint32_t keys,
                            uint32_t values, uint32_t rank,
                            const float* record_decay, const float* record_keys,
                            const float* record_corrections, uint32_t records,
                            float* state) {
  /* state_capsule.cpp:337-352: dequantize, then replay the records in order. */
  gdn_oracle_dequantize_kv(codes, smoothing, value_scales, comp_keys, comp_values,
                           keys, values, rank, state);
  for (uint32_t u = 0; u < records; ++u) {
    for (uint32_t row = 0; row < keys; ++row) {
      for (uint32_t column = 0; column < values; ++column) {
        const size_t cell = (size_t)row * values + column;
        state[cell] = record_decay[(size_t)u * keys + row] * state[cell] +
                      record_keys[(size_t)u * keys + row] *
                          record_corrections[(size_t)u * values + column];
      }
    }
  }
}

int gdn_oracle_apply_token(int8_t* codes, float* smoothing, float* value_scales,
                           float* comp_keys, float* comp_values, uint32_t keys,
                           uint32_t values, uint32_t rank, uint32_t window,
                           float* record_decay, float* record_keys,
                           float* record_corrections, uint32_t* records,
                           const float* decay, const float* key,
                           const float* value, const float* read,
                           const float* query, float* output) {
  /* state_capsule.cpp:354-397. */
  const uint32_t p = *records;
  float* state_read = (float*)malloc(sizeof(float) * values);
  float* decayed_query = (float*)malloc(sizeof(float) * keys);
  float* correction = record_corrections + (size_t)p * values;
  gdn_oracle_read_window(codes, smoothing, value_scales, comp_keys, comp_values,
                         keys, values, rank, record_decay, record_keys,
                         record_corrections, p, read, state_read);
  for (uint32_t column = 0; column < values; ++column) {
    correction[column] = value[column] - state_read[column];
  }
  float update_projection = 0.0f;
  for (uint32_t row = 0; row < keys; ++row) {
    decayed_query[row] = decay[row] * query[row];
    update_projection += key[row] * query[row];
  }
  gdn_oracle_read_window(codes, smoothing, value_scales, comp_keys, comp_values,
                         keys, values, rank, record_decay, record_keys,
                         record_corrections, p, decayed_query, output);
  for (uint32_t column = 0; column < values; ++column) {
    output[column] += correction[column] * update_projection;
  }
  memcpy(record_decay + (size_t)p * keys, decay, sizeof(float) * keys);
  memcpy(record_keys + (size_t)p * keys, key, sizeof(float) * keys);
  int crossed = 0;
  if (p + 1 == window) {
    float* state = (float*)malloc(sizeof(float) * keys * values);
    float* work = (float*)malloc(sizeof(float) * keys * values);
    gdn_oracle_dense_state(codes, smoothing, value_scales, comp_keys, comp_values,
                           keys, values, rank, record_decay, record_keys,
                           record_corrections, p + 1, state);
    gdn_oracle_quantize_kv(state, keys, values, rank, 1.0e-8f, codes, smoothing,
                           value_scales, comp_keys, comp_values, work);
    free(work);
    free(state);
    *records = 0;
    crossed = 1;
  } else {
    *records = p + 1;
  }
  free(decayed_query);
  free(state_read);
  return crossed;
}

/* ------------------------------------------------- device-format layer */

/* The same readout as gdn_oracle_read_window for scalar record decays, in
 * double, with sum |term| as the error scale.  Inputs are the fp32 values the
 * device forms, so only the arithmetic after them differs. */
static void read_window_f64(const int8_t* codes, uint32_t layout,
                            const float* smoothing, const float* value_scales,
                            const float* comp_keys, const float* comp_values,
                            uint32_t rank, const float* record_decay,
                            const float* record_keys,
                            const float* record_corrections, uint32_t records,
                            const float* x, double* out, double* bound) {
  double suffix[WINDOW];
  double running = 1.0;
  for (uint32_t index = records; index > 0; --index) {
    suffix[index - 1] = running;
    running *= record_decay[index - 1];
  }
  const double boundary_suffix = running;
  double comp_projection[RANK], comp_abs[RANK];
  for (uint32_t r = 0; r < rank; ++r) {
    double p = 0.0, a = 0.0;
    for (uint32_t k = 0; k < DIM; ++k) {
      p += (double)comp_keys[k * rank + r] * x[k];
      a += fabs((double)comp_keys[k * rank + r] * x[k]);
    }
    comp_projection[r] = p * boundary_suffix;
    comp_abs[r] = a * boundary_suffix;
  }
  double record_projection[WINDOW], record_abs[WINDOW];
  for (uint32_t j = 0; j < records; ++j) {
    double p = 0.0, a = 0.0;
    for (uint32_t k = 0; k < DIM; ++k) {
      p += (double)record_keys[j * DIM + k] * x[k];
      a += fabs((double)record_keys[j * DIM + k] * x[k]);
    }
    record_projection[j] = p * suffix[j];
    record_abs[j] = a * suffix[j];
  }
  for (uint32_t v = 0; v < DIM; ++v) {
    double sum = 0.0, a = 0.0;
    for (uint32_t k = 0; k < DIM; ++k) {
      const int8_t code = layout == GDN_ORACLE_LAYOUT_KEY_VALUE ? codes[k * DIM + v]
                                                                : codes[v * DIM + k];
      const double term = (double)code * smoothing[k] * x[k];
      sum += term;
      a += fabs(term);
    }
    const double scale = (double)value_scales[v] / 127.0 * boundary_suffix;
    double o = sum * scale;
    double b = a * fabs(scale);
    for (uint32_t r = 0; r < rank; ++r) {
      o += (double)comp_values[v * rank + r] * comp_projection[r];
      b += fabs((double)comp_values[v * rank + r]) * comp_abs[r];
    }
    for (uint32_t j = 0; j < records; ++j) {
      o += (double)record_corrections[j * DIM + v] * record_projection[j];
      b += fabs((double)record_corrections[j * DIM + v]) * record_abs[j];
    }
    out[v] = o;
    bound[v] = b;
  }
}

/* One state of a device step, given the fp32 vectors the device forms:
 * read[k], decayed query dq[k], write key wk[k], query q[k] (so that
 * update = sum wk*q), value[v].  Boundary codes in `layout`; compensators and
 * records already widened to fp32.  Fills the fp32 result in the capsule's
 * order (out32, corr32) and the double result with bounds. */
static void device_state_step(const int8_t* codes, uint32_t layout,
                              const float* smoothing, const float* value_scales,
                              const float* comp_keys, const float* comp_values,
                              uint32_t rank, const float* record_decay,
                              const float* record_keys,
                              const float* record_corrections, uint32_t records,
                              const float* read, const float* dq,
                              const float* wk, const float* q,
                              const float* value, float* out32, float* corr32,
                              double* out64, double* out_bound, double* corr64,
                              double* corr_bound) {
  int8_t kv[TILE];
  const int8_t* boundary = codes;
  if (layout == GDN_ORACLE_LAYOUT_VALUE_KEY) {
    for (uint32_t k = 0; k < DIM; ++k)
      for (uint32_t v = 0; v < DIM; ++v) kv[k * DIM + v] = codes[v * DIM + k];
    boundary = kv;
  }
  float decay_rows[WINDOW * DIM];
  for (uint32_t j = 0; j < records; ++j)
    for (uint32_t k = 0; k < DIM; ++k) decay_rows[j * DIM + k] = record_decay[j];
  float state_read[DIM], output_read[DIM];
  gdn_oracle_read_window(boundary, smoothing, value_scales, comp_keys, comp_values,
                         DIM, DIM, rank, decay_rows, record_keys,
                         record_corrections, records, read, state_read);
  gdn_oracle_read_window(boundary, smoothing, value_scales, comp_keys, comp_values,
                         DIM, DIM, rank, decay_rows, record_keys,
                         record_corrections, records, dq, output_read);
  float update = 0.0f;
  double update64 = 0.0, update_abs = 0.0;
  for (uint32_t k = 0; k < DIM; ++k) {
    update += wk[k] * q[k];
    update64 += (double)wk[k] * q[k];
    update_abs += fabs((double)wk[k] * q[k]);
  }
  double sr64[DIM], sr_bound[DIM], or64[DIM], or_bound[DIM];
  read_window_f64(codes, layout, smoothing, value_scales, comp_keys, comp_values,
                  rank, record_decay, record_keys, record_corrections, records,
                  read, sr64, sr_bound);
  read_window_f64(codes, layout, smoothing, value_scales, comp_keys, comp_values,
                  rank, record_decay, record_keys, record_corrections, records, dq,
                  or64, or_bound);
  for (uint32_t v = 0; v < DIM; ++v) {
    corr32[v] = value[v] - state_read[v];
    out32[v] = output_read[v] + corr32[v] * update;
    const double c = (double)value[v] - sr64[v];
    if (corr64) corr64[v] = c;
    if (corr_bound) corr_bound[v] = sr_bound[v];
    if (out64) out64[v] = or64[v] + c * update64;
    if (out_bound) out_bound[v] = or_bound[v] + fabs(update64) * sr_bound[v] + fabs(c) * update_abs;
  }
}

void gdn_oracle_windowed_step_bf16(
    const int8_t* residual, const float* smoothing, const float* scales,
    const uint16_t* comp_keys, const uint16_t* comp_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    const float* log_decay, const uint16_t* beta, const uint16_t* keys,
    const uint16_t* queries, const uint16_t* values, uint16_t* outputs,
    uint32_t states, double* out64, double* out_bound, double* corr64,
    double* corr_bound) {
  /* windowed_gdn_step.cpp:326-619 (compensated: Process<true>, quant-only:
   * Process<false> when comp_keys == comp_values == NULL). */
  const uint32_t rank = comp_keys != NULL ? RANK : 0u;
  for (uint32_t s = 0; s < states; ++s) {
    const uint32_t p = positions[(size_t)s * POSITION_STRIDE];
    if (p >= WINDOW) continue;
    const float g = exp_f32(log_decay[s]);
    const float b = gdn_oracle_bf16_to_f32(beta[s]);
    const uint16_t* key_in = keys + (size_t)(s / 2) * DIM;
    const uint16_t* query_in = queries + (size_t)(s / 2) * DIM;
    float read[DIM], dq[DIM], wk[DIM], q[DIM], value[DIM];
    for (uint32_t k = 0; k < DIM; ++k) {
      const float key = gdn_oracle_bf16_to_f32(key_in[k]);
      q[k] = QUERY_SCALE * gdn_oracle_bf16_to_f32(query_in[k]);
      read[k] = g * key;
      dq[k] = q[k] * g;
      wk[k] = b * key;
      value[k] = gdn_oracle_bf16_to_f32(values[(size_t)s * DIM + k]);
    }
    float ck[DIM * RANK], cv[DIM * RANK];
    for (uint32_t i = 0; i < DIM * rank; ++i) {
      ck[i] = gdn_oracle_f16_to_f32(comp_keys[(size_t)s * DIM * RANK + i]);
      cv[i] = gdn_oracle_f16_to_f32(comp_values[(size_t)s * DIM * RANK + i]);
    }
    float rk[WINDOW * DIM], rc[WINDOW * DIM];
    for (uint32_t i = 0; i < p * DIM; ++i) {
      rk[i] = gdn_oracle_f16_to_f32(record_keys[(size_t)s * WINDOW * DIM + i]);
      rc[i] = gdn_oracle_f16_to_f32(record_corrections[(size_t)s * WINDOW * DIM + i]);
    }
    float out32[DIM], corr32[DIM];
    device_state_step(residual + (size_t)s * TILE, GDN_ORACLE_LAYOUT_VALUE_KEY,
                      smoothing + (size_t)s * DIM, scales + (size_t)s * DIM, ck, cv,
                      rank, record_decay + (size_t)s * WINDOW, rk, rc, p, read, dq,
                      wk, q, value, out32, corr32,
                      out64 ? out64 + (size_t)s * DIM : NULL,
                      out_bound ? out_bound + (size_t)s * DIM : NULL,
                      corr64 ? corr64 + (size_t)s * DIM : NULL,
                      corr_bound ? corr_bound + (size_t)s * DIM : NULL);
    uint16_t* key_out = record_keys + ((size_t)s * WINDOW + p) * DIM;
    uint16_t* corr_out = record_corrections + ((size_t)s * WINDOW + p) * DIM;
    for (uint32_t v = 0; v < DIM; ++v) {
      outputs[(size_t)s * DIM + v] = gdn_oracle_f32_to_bf16(out32[v]);
      key_out[v] = gdn_oracle_f32_to_f16(wk[v]);
      corr_out[v] = gdn_oracle_f32_to_f16(corr32[v]);
    }
    record_decay[(size_t)s * WINDOW + p] = g;
    positions[(size_t)s * POSITION_STRIDE] = p + 1;
  }
}

void gdn_oracle_windowed_step_f16(
    const int8_t* residual, const float* smoothing, const float* scales,
    const uint16_t* comp_keys, const uint16_t* comp_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    const float* decay, const uint16_t* write_keys, const uint16_t* reads,
    const uint16_t* queries, const uint16_t* values, float* outputs,
    uint32_t states, double* out64, double* out_bound, double* corr64,
    double* corr_bound) {
  /* windowed_gdn_step.cpp:62-176: [key][value] boundary, fp16 vectors, linear
   * decay, fp32 outputs, rank-4 fp16 compensators. */
  for (uint32_t s = 0; s < states; ++s) {
    const uint32_t p = positions[(size_t)s * POSITION_STRIDE];
    if (p >= WINDOW) continue;
    const float g = decay[s];
    float read[DIM], dq[DIM], wk[DIM], q[DIM], value[DIM];
    for (uint32_t k = 0; k < DIM; ++k) {
      read[k] = gdn_oracle_f16_to_f32(reads[(size_t)s * DIM + k]);
      q[k] = gdn_oracle_f16_to_f32(queries[(size_t)s * DIM + k]);
      dq[k] = q[k] * g;
      wk[k] = gdn_oracle_f16_to_f32(write_keys[(size_t)s * DIM + k]);
      value[k] = gdn_oracle_f16_to_f32(values[(size_t)s * DIM + k]);
    }
    float ck[DIM * RANK], cv[DIM * RANK];
    for (uint32_t i = 0; i < DIM * RANK; ++i) {
      ck[i] = gdn_oracle_f16_to_f32(comp_keys[(size_t)s * DIM * RANK + i]);
      cv[i] = gdn_oracle_f16_to_f32(comp_values[(size_t)s * DIM * RANK + i]);
    }
    float rk[WINDOW * DIM], rc[WINDOW * DIM];
    for (uint32_t i = 0; i < p * DIM; ++i) {
      rk[i] = gdn_oracle_f16_to_f32(record_keys[(size_t)s * WINDOW * DIM + i]);
      rc[i] = gdn_oracle_f16_to_f32(record_corrections[(size_t)s * WINDOW * DIM + i]);
    }
    float out32[DIM], corr32[DIM];
    device_state_step(residual + (size_t)s * TILE, GDN_ORACLE_LAYOUT_KEY_VALUE,
                      smoothing + (size_t)s * DIM, scales + (size_t)s * DIM, ck, cv,
                      RANK, record_decay + (size_t)s * WINDOW, rk, rc, p, read, dq,
                      wk, q, value, out32, corr32,
                      out64 ? out64 + (size_t)s * DIM : NULL,
                      out_bound ? out_bound + (size_t)s * DIM : NULL,
                      corr64 ? corr64 + (size_t)s * DIM : NULL,
                      corr_bound ? corr_bound + (size_t)s * DIM : NULL);
    uint16_t* key_out = record_keys + ((size_t)s * WINDOW + p) * DIM;
    uint16_t* corr_out = record_corrections + ((size_t)s * WINDOW + p) * DIM;
    for (uint32_t v = 0; v < DIM; ++v) {
      outputs[(size_t)s * DIM + v] = out32[v];
      key_out[v] = write_keys[(size_t)s * DIM + v];
      corr_out[v] = gdn_oracle_f32_to_f16(corr32[v]);
    }
    record_decay[(size_t)s * WINDOW + p] = g;
    positions[(size_t)s * POSITION_STRIDE] = p + 1;
  }
}

void gdn_oracle_gdn_step_f32(float* state, const float* decay,
                             const uint16_t* keys, const uint16_t* reads,
                             const uint16_t* queries, const uint16_t* values,
                             float* outputs, uint32_t states) {
  /* fp32_gdn_step.cpp:13-18: per column, projection = sum_r S[r][c] read[r],
   * correction = value[c] - projection, S' = decay S + key correction,
   * out[c] = sum_r S'[r][c] query[r]. */
  for (uint32_t s = 0; s < states; ++s) {
    float* S = state + (size_t)s * TILE;
    const size_t vb = (size_t)s * DIM;
    for (uint32_t c = 0; c < DIM; ++c) {
      float projection = 0.0f;
      for (uint32_t r = 0; r < DIM; ++r) {
        projection += S[r * DIM + c] * gdn_oracle_f16_to_f32(reads[vb + r]);
      }
      const float correction = gdn_oracle_f16_to_f32(values[vb + c]) - projection;
      float out = 0.0f;
      for (uint32_t r = 0; r < DIM; ++r) {
        const float next = decay[s] * S[r * DIM + c] +
                           gdn_oracle_f16_to_f32(keys[vb + r]) * correction;
        S[r * DIM + c] = next;
        out += next * gdn_oracle_f16_to_f32(queries[vb + r]);
      }
      outputs[vb + c] = out;
    }
  }
}

/* ------------------------------------------- cube decode-pair chain */

/* Reference rounding of the vector quantizers: add +-0.5 in fp32, clamp, then
 * truncate toward zero (encoded_projection.cpp:222-226, 328-340). */
static int8_t pair_round(float value) {
  float r = value + (value >= 0.0f ? 0.5f : -0.5f);
  r = r > 127.0f ? 127.0f : r;
  r = r < -127.0f ? -127.0f : r;
  return (int8_t)r;
}

/* Two-level int8 split of two fp32 vectors (encoded_projection.cpp:257-352,
 * :375-479): column 2c is the high code, 2c+1 the low code of vector c;
 * dynamic_scale[s][0..3] = {hi0, hi1, lo0, lo1}; columns 4..15 are zero. */
static void split_pair(const float* pair0, const float* pair1, int8_t* quantized,
                       float* dynamic_scale) {
  const float* pair[2] = {pair0, pair1};
  float maxima[2] = {0.0f, 0.0f};
  for (uint32_t row = 0; row < DIM; ++row)
    for (uint32_t c = 0; c < 2; ++c) {
      const float m = fabsf(pair[c][row]);
      maxima[c] = m > maxima[c] ? m : maxima[c];
    }
  float scale[4];
  for (uint32_t c = 0; c < 2; ++c)
    scale[c] = maxima[c] > 1.0e-20f ? maxima[c] / 127.0f : 1.0f;
  float residual_maxima[2] = {0.0f, 0.0f};
  for (uint32_t row = 0; row < DIM; ++row)
    for (uint32_t c = 0; c < 2; ++c) {
      const int8_t high = pair_round(pair[c][row] / scale[c]);
      const float residual = pair[c][row] - high * scale[c];
      const float m = fabsf(residual);
      residual_maxima[c] = m > residual_maxima[c] ? m : residual_maxima[c];
    }
  for (uint32_t c = 0; c < 2; ++c)
    scale[c + 2] = residual_maxima[c] > 1.0e-20f ? residual_maxima[c] / 127.0f : 1.0f;
  for (uint32_t c = 0; c < 4; ++c) dynamic_scale[c] = scale[c];
  for (uint32_t row = 0; row < DIM; ++row) {
    for (uint32_t c = 0; c < 2; ++c) {
      const int8_t high = pair_round(pair[c][row] / scale[c]);
      const int8_t low = pair_round((pair[c][row] - high * scale[c]) / scale[c + 2]);
      quantized[row * 16 + 2 * c] = high;
      quantized[row * 16 + 2 * c + 1] = low;
    }
    for (uint32_t c = 4; c < 16; ++c) quantized[row * 16 + c] = 0;
  }
}

void gdn_oracle_prepare_decode_pair_bf16(const uint16_t* keys,
                                         const uint16_t* queries,
                                         const float* log_decay,
                                         const float* smoothing,
                                         int8_t* quantized, float* dynamic_scale,
                                         uint32_t states) {
  /* encoded_projection.cpp:355-479. */
  for (uint32_t s = 0; s < states; ++s) {
    const float g = exp_f32(log_decay[s]);
    float pair0[DIM], pair1[DIM];
    for (uint32_t row = 0; row < DIM; ++row) {
      const float sm = smoothing[(size_t)s * DIM + row];
      pair0[row] = g * gdn_oracle_bf16_to_f32(keys[(size_t)(s / 2) * DIM + row]) * sm;
      pair1[row] = QUERY_SCALE * g *
                   gdn_oracle_bf16_to_f32(queries[(size_t)(s / 2) * DIM + row]) * sm;
    }
    split_pair(pair0, pair1, quantized + (size_t)s * DIM * 16,
               dynamic_scale + (size_t)s * POSITION_STRIDE);
  }
}

void gdn_oracle_prepare_decode_pair(const uint16_t* reads, const uint16_t* queries,
                                    const float* decay, const float* smoothing,
                                    int8_t* quantized, float* dynamic_scale,
                                    uint32_t states) {
  /* encoded_projection.cpp:236-353. */
  for (uint32_t s = 0; s < states; ++s) {
    float pair0[DIM], pair1[DIM];
    for (uint32_t row = 0; row < DIM; ++row) {
      const float sm = smoothing[(size_t)s * DIM + row];
      pair0[row] = gdn_oracle_f16_to_f32(reads[(size_t)s * DIM + row]) * sm;
      pair1[row] = gdn_oracle_f16_to_f32(queries[(size_t)s * DIM + row]) * decay[s] * sm;
    }
    split_pair(pair0, pair1, quantized + (size_t)s * DIM * 16,
               dynamic_scale + (size_t)s * POSITION_STRIDE);
  }
}

void gdn_oracle_prepare_int8_vector(const uint16_t* input, const float* axis_scale,
                                    int8_t* quantized, float* dynamic_scale,
                                    uint32_t states) {
  /* encoded_projection.cpp:179-234: column 0 of a [128][16] f16 input. */
  for (uint32_t s = 0; s < states; ++s) {
    float maximum = 0.0f;
    for (uint32_t row = 0; row < DIM; ++row) {
      const float v = gdn_oracle_f16_to_f32(input[((size_t)s * DIM + row) * 16]) *
                      axis_scale[(size_t)s * DIM + row];
      const float m = fabsf(v);
      maximum = m > maximum ? m : maximum;
    }
    const float scale = maximum > 1.0e-20f ? maximum / 127.0f : 1.0f;
    dynamic_scale[(size_t)s * POSITION_STRIDE] = scale;
    for (uint32_t row = 0; row < DIM; ++row) {
      const float v = gdn_oracle_f16_to_f32(input[((size_t)s * DIM + row) * 16]) *
                      axis_scale[(size_t)s * DIM + row] / scale;
      int8_t* out = quantized + ((size_t)s * DIM + row) * 16;
      out[0] = pair_round(v);
      for (uint32_t c = 1; c < 16; ++c) out[c] = 0;
    }
  }
}

void gdn_oracle_int8_matmul(const int8_t* a, const int8_t* b, int32_t* c,
                            uint32_t states, uint32_t transpose_a) {
  /* int8_cube_matmul.cpp:19-52: per state C[128][16] = A[128][128] B[128][16]
   * (A transposed when transpose_a), exact int32. */
  for (uint32_t s = 0; s < states; ++s) {
    const int8_t* A = a + (size_t)s * TILE;
    const int8_t* B = b + (size_t)s * DIM * 16;
    int32_t* C = c + (size_t)s * DIM * 16;
    for (uint32_t m = 0; m < DIM; ++m)
      for (uint32_t n = 0; n < 16; ++n) {
        int32_t sum = 0;
        for (uint32_t k = 0; k < DIM; ++k) {
          const int32_t av = transpose_a ? A[k * DIM + m] : A[m * DIM + k];
          sum += av * B[k * 16 + n];
        }
        C[m * 16 + n] = sum;
      }
  }
}

/* Shared body of finish_decode_pair{,_bf16} (encoded_projection.cpp:
 * 532-603, :668-752).  The caller provides the per-row vectors read[k],
 * oq[k] = query * decay (the output-side vector) and the update sum. */
static void finish_state(const int32_t* projected, const float* dynamic_scale,
                         const float* scales, const float* ck, const float* cv,
                         const float* record_decay, const float* rk,
                         const float* rc, uint32_t p, const float* read,
                         const float* query, float g, float update,
                         const float* value, float* out, float* corr) {
  float old_projection[2][RANK] = {{0}};
  float record_projection[2][WINDOW] = {{0}};
  for (uint32_t row = 0; row < DIM; ++row) {
    for (uint32_t r = 0; r < RANK; ++r) {
      const float basis = ck[row * RANK + r];
      old_projection[0][r] += basis * read[row];
      old_projection[1][r] += basis * query[row] * g;
    }
    for (uint32_t j = 0; j < p; ++j) {
      const float basis = rk[j * DIM + row];
      record_projection[0][j] += basis * read[row];
      record_projection[1][j] += basis * query[row] * g;
    }
  }
  float suffix[WINDOW];
  float boundary_suffix = 1.0f;
  for (uint32_t index = p; index > 0; --index) {
    suffix[index - 1] = boundary_suffix;
    boundary_suffix *= record_decay[index - 1];
  }
  for (uint32_t column = 0; column < DIM; ++column) {
    const int32_t* P = projected + column * 16;
    float state_read = ((float)P[0] * dynamic_scale[0] + (float)P[1] * dynamic_scale[2]) /
                       127.0f * scales[column] * boundary_suffix;
    float output_read = ((float)P[2] * dynamic_scale[1] + (float)P[3] * dynamic_scale[3]) /
                        127.0f * scales[column] * boundary_suffix;
    for (uint32_t r = 0; r < RANK; ++r) {
      const float basis = cv[column * RANK + r];
      state_read += basis * old_projection[0][r] * boundary_suffix;
      output_read += basis * old_projection[1][r] * boundary_suffix;
    }
    for (uint32_t j = 0; j < p; ++j) {
      const float basis = rc[j * DIM + column];
      state_read += basis * record_projection[0][j] * suffix[j];
      output_read += basis * record_projection[1][j] * suffix[j];
    }
    corr[column] = value[column] - state_read;
    out[column] = output_read + corr[column] * update;
  }
}

void gdn_oracle_finish_decode_pair_bf16(
    const int32_t* projected, const float* dynamic_scale, const float* scales,
    const uint16_t* comp_keys, const uint16_t* comp_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    const float* log_decay, const uint16_t* beta, const uint16_t* keys,
    const uint16_t* queries, const uint16_t* values, uint16_t* outputs,
    uint32_t states) {
  /* encoded_projection.cpp:624-776. */
  for (uint32_t s = 0; s < states; ++s) {
    const uint32_t p = positions[(size_t)s * POSITION_STRIDE];
    if (p >= WINDOW) continue;
    const float g = exp_f32(log_decay[s]);
    const float b = gdn_oracle_bf16_to_f32(beta[s]);
    float read[DIM], query[DIM], value[DIM], key[DIM];
    float update = 0.0f;
    for (uint32_t row = 0; row < DIM; ++row) {
      key[row] = gdn_oracle_bf16_to_f32(keys[(size_t)(s / 2) * DIM + row]);
      query[row] = QUERY_SCALE * gdn_oracle_bf16_to_f32(queries[(size_t)(s / 2) * DIM + row]);
      read[row] = g * key[row];
      const float write_key = b * key[row];
      update += write_key * query[row];
      value[row] = gdn_oracle_bf16_to_f32(values[(size_t)s * DIM + row]);
    }
    float ck[DIM * RANK], cv[DIM * RANK], rk[WINDOW * DIM], rc[WINDOW * DIM];
    for (uint32_t i = 0; i < DIM * RANK; ++i) {
      ck[i] = gdn_oracle_f16_to_f32(comp_keys[(size_t)s * DIM * RANK + i]);
      cv[i] = gdn_oracle_f16_to_f32(comp_values[(size_t)s * DIM * RANK + i]);
    }
    for (uint32_t i = 0; i < p * DIM; ++i) {
      rk[i] = gdn_oracle_f16_to_f32(record_keys[(size_t)s * WINDOW * DIM + i]);
      rc[i] = gdn_oracle_f16_to_f32(record_corrections[(size_t)s * WINDOW * DIM + i]);
    }
    float out[DIM], corr[DIM];
    finish_state(projected + (size_t)s * DIM * 16,
                 dynamic_scale + (size_t)s * POSITION_STRIDE,
                 scales + (size_t)s * DIM, ck, cv, record_decay + (size_t)s * WINDOW,
                 rk, rc, p, read, query, g, update, value, out, corr);
    uint16_t* key_out = record_keys + ((size_t)s * WINDOW + p) * DIM;
    uint16_t* corr_out = record_corrections + ((size_t)s * WINDOW + p) * DIM;
    for (uint32_t v = 0; v < DIM; ++v) {
      outputs[(size_t)s * DIM + v] = gdn_oracle_f32_to_bf16(out[v]);
      key_out[v] = gdn_oracle_f32_to_f16(b * key[v]);
      corr_out[v] = gdn_oracle_f32_to_f16(corr[v]);
    }
    record_decay[(size_t)s * WINDOW + p] = g;
    positions[(size_t)s * POSITION_STRIDE] = p + 1;
  }
}

void gdn_oracle_finish_decode_pair(
    const int32_t* projected, const float* dynamic_scale, const float* scales,
    const uint16_t* comp_keys, const uint16_t* comp_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    const float* decay, const uint16_t* write_keys, const uint16_t* reads,
    const uint16_t* queries, const uint16_t* values, float* outputs,
    uint32_t states) {
  /* encoded_projection.cpp:482-621. */
  for (uint32_t s = 0; s < states; ++s) {
    const uint32_t p = positions[(size_t)s * POSITION_STRIDE];
    if (p >= WINDOW) continue;
    const float g = decay[s];
    float read[DIM], query[DIM], value[DIM];
    float update = 0.0f;
    for (uint32_t row = 0; row < DIM; ++row) {
      read[row] = gdn_oracle_f16_to_f32(reads[(size_t)s * DIM + row]);
      query[row] = gdn_oracle_f16_to_f32(queries[(size_t)s * DIM + row]);
      update += gdn_oracle_f16_to_f32(write_keys[(size_t)s * DIM + row]) * query[row];
      value[row] = gdn_oracle_f16_to_f32(values[(size_t)s * DIM + row]);
    }
    float ck[DIM * RANK], cv[DIM * RANK], rk[WINDOW * DIM], rc[WINDOW * DIM];
    for (uint32_t i = 0; i < DIM * RANK; ++i) {
      ck[i] = gdn_oracle_f16_to_f32(comp_keys[(size_t)s * DIM * RANK + i]);
      cv[i] = gdn_oracle_f16_to_f32(comp_values[(size_t)s * DIM * RANK + i]);
    }
    for (uint32_t i = 0; i < p * DIM; ++i) {
      rk[i] = gdn_oracle_f16_to_f32(record_keys[(size_t)s * WINDOW * DIM + i]);
      rc[i] = gdn_oracle_f16_to_f32(record_corrections[(size_t)s * WINDOW * DIM + i]);
    }
    float out[DIM], corr[DIM];
    finish_state(projected + (size_t)s * DIM * 16,
                 dynamic_scale + (size_t)s * POSITION_STRIDE,
                 scales + (size_t)s * DIM, ck, cv, record_decay + (size_t)s * WINDOW,
                 rk, rc, p, read, query, g, update, value, out, corr);
    uint16_t* key_out = record_keys + ((size_t)s * WINDOW + p) * DIM;
    uint16_t* corr_out = record_corrections + ((size_t)s * WINDOW + p) * DIM;
    for (uint32_t v = 0; v < DIM; ++v) {
      outputs[(size_t)s * DIM + v] = out[v];
      key_out[v] = write_keys[(size_t)s * DIM + v];
      corr_out[v] = gdn_oracle_f32_to_f16(corr[v]);
    }
    record_decay[(size_t)s * WINDOW + p] = g;
    positions[(size_t)s * POSITION_STRIDE] = p + 1;
  }
}
