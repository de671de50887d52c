/*
 * CPU oracle for the window-boundary refit of the windowed GDN decode path.
 *
 * TEST INFRASTRUCTURE ONLY (see gdn_oracle.h): loaded by tests/ as the checker,
 * never by the product library.
 *
 * Statement-by-statement restatements of
 *   native/ascendc/gdn_state_codec/kernel/gdn_state_codec_window_boundary.cpp
 *   (ProcessQuantOnlyTask :368-499, ProcessState :253-366 with ApplyRight,
 *   ApplyTranspose and ResidualCell :102-251, BoundaryRecordScaleKernel
 *   :537-587, the finalize kernel :589-611 and the launchers :653-750) and the
 *   record-merge GEMM of kernel/gdn_state_codec_bf16_cube_matmul.cpp.
 * Each `a += b * c * d` of the reference is evaluated as written (separately
 * rounded fp32 operations, left to right).  Two reference operations have no
 * documented evaluation order and are fixed here: AscendC::Axpy(dst, src, s)
 * is dst = src * s + dst with a rounded product, and the fp16 Cube GEMM sums
 * its 16 exact products in ascending k.
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
#define FLOOR 1.0e-8f

static float h2f(uint16_t h) { return gdn_oracle_f16_to_f32(h); }
static uint16_t f2h(float f) { return gdn_oracle_f32_to_f16(f); }

/* window_boundary.cpp:17-23: 20 Newton steps from max(value, 1). */
float gdn_oracle_boundary_sqrt(float value) {
  float estimate = value > 1.0f ? value : 1.0f;
  for (uint32_t iteration = 0; iteration < 20; ++iteration) {
    estimate = 0.5f * (estimate + value / estimate);
  }
  return estimate;
}

/* window_boundary.cpp:25-37. */
static int normalize(float* vector) {
  float squared_norm = 0.0f;
  for (uint32_t axis = 0; axis < DIM; ++axis) squared_norm += vector[axis] * vector[axis];
  if (squared_norm <= 1.0e-20f) return 0;
  const float inverse_norm = 1.0f / gdn_oracle_boundary_sqrt(squared_norm);
  for (uint32_t axis = 0; axis < DIM; ++axis) vector[axis] *= inverse_norm;
  return 1;
}

/* BuildSuffix (:102-111): record_suffix[j] = prod over later records, taken
 * from the last record down. */
static float build_suffix(const float* record_decay, float* record_suffix) {
  float suffix = 1.0f;
  for (uint32_t reverse = WINDOW; reverse > 0; --reverse) {
    record_suffix[reverse - 1] = suffix;
    suffix *= record_decay[reverse - 1];
  }
  return suffix;
}

/* Rounding to int8 through fp16 with round-half-even (Cast CAST_NONE to half,
 * then CAST_RINT to int8; :478-483). */
static int8_t rint_through_half(float value) {
  const float h = h2f(f2h(value));
  return (int8_t)nearbyintf(h);
}

void gdn_oracle_window_boundary_quant_only(
    const int8_t* residual, const float* smoothing, const float* scales,
    const float* record_decay, const uint16_t* record_keys,
    const uint16_t* record_corrections, uint32_t* positions,
    int8_t* next_residual, float* next_smoothing, float* next_scales,
    uint16_t* next_comp_keys, uint16_t* next_comp_values,
    const float* record_merge, uint32_t states) {
  for (uint32_t s = 0; s < states; ++s) {
    float record_suffix[WINDOW];
    const float boundary_suffix = build_suffix(record_decay + (size_t)s * WINDOW, record_suffix);
    const float* sm = smoothing + (size_t)s * DIM;
    float keys_f[WINDOW * DIM];
    for (uint32_t i = 0; i < WINDOW * DIM; ++i) {
      keys_f[i] = h2f(record_keys[(size_t)s * WINDOW * DIM + i]);
    }
    for (uint32_t column = 0; column < DIM; ++column) {
      const int8_t* code = residual + (size_t)s * TILE + (size_t)column * DIM;
      const float factor = scales[(size_t)s * DIM + column] * boundary_suffix / 127.0f;
      float working[DIM];
      for (uint32_t k = 0; k < DIM; ++k) working[k] = (float)code[k] * factor * sm[k];
      if (record_merge != NULL) {
        const float* merge = record_merge + (size_t)s * TILE + (size_t)column * DIM;
        for (uint32_t k = 0; k < DIM; ++k) working[k] = working[k] + merge[k];
      } else {
        for (uint32_t j = 0; j < WINDOW; ++j) {
          const float scalar =
              h2f(record_corrections[((size_t)s * WINDOW + j) * DIM + column]) * record_suffix[j];
          for (uint32_t k = 0; k < DIM; ++k) {
            working[k] = keys_f[j * DIM + k] * scalar + working[k];
          }
        }
      }
      float maximum = 0.0f;
      for (uint32_t k = 0; k < DIM; ++k) {
        working[k] = working[k] / sm[k];
        const float m = fabsf(working[k]);
        maximum = m > maximum ? m : maximum;
      }
      next_scales[(size_t)s * DIM + column] = maximum;
      const float multiplier = maximum > 0.0f ? 127.0f / maximum : 0.0f;
      int8_t* out = next_residual + (size_t)s * TILE + (size_t)column * DIM;
      for (uint32_t k = 0; k < DIM; ++k) {
        float t = working[k] * multiplier;
        t = t > -127.0f ? t : -127.0f;  /* Maxs(-127) then Mins(127) */
        t = t < 127.0f ? t : 127.0f;
        out[k] = rint_through_half(t);
      }
    }
    memcpy(next_smoothing + (size_t)s * DIM, sm, sizeof(float) * DIM);
    memset(next_comp_keys + (size_t)s * DIM * RANK, 0, sizeof(uint16_t) * DIM * RANK);
    memset(next_comp_values + (size_t)s * DIM * RANK, 0, sizeof(uint16_t) * DIM * RANK);
    positions[(size_t)s * POSITION_STRIDE] = 0; /* the finalize kernel */
  }
}

void gdn_oracle_boundary_scale_records(const float* record_decay,
                                       const uint16_t* record_keys,
                                       uint16_t* scaled_record_keys,
                                       uint32_t states) {
  /* :550-580: suffix over later records in ascending order, then an fp16
   * multiply of every key by the fp16 suffix. */
  for (uint32_t s = 0; s < states; ++s) {
    for (uint32_t j = 0; j < WINDOW; ++j) {
      float suffix = 1.0f;
      for (uint32_t later = j + 1; later < WINDOW; ++later) {
        suffix *= record_decay[(size_t)s * WINDOW + later];
      }
      const float hs = h2f(f2h(suffix));
      const size_t base = ((size_t)s * WINDOW + j) * DIM;
      for (uint32_t k = 0; k < DIM; ++k) {
        scaled_record_keys[base + k] = f2h(h2f(record_keys[base + k]) * hs);
      }
    }
  }
}

void gdn_oracle_f16_matmul_at_b(const uint16_t* a, const uint16_t* b, float* c,
                                uint32_t states) {
  /* bf16_cube_matmul.cpp:17-48: per state C[m][n] = sum_k A[k][m] B[k][n],
   * A and B fp16 [16][128], C fp32 [128][128]. */
  for (uint32_t s = 0; s < states; ++s) {
    const uint16_t* A = a + (size_t)s * WINDOW * DIM;
    const uint16_t* B = b + (size_t)s * WINDOW * DIM;
    float* C = c + (size_t)s * TILE;
    for (uint32_t m = 0; m < DIM; ++m) {
      for (uint32_t n = 0; n < DIM; ++n) {
        float sum = 0.0f;
        for (uint32_t k = 0; k < WINDOW; ++k) sum += h2f(A[k * DIM + m]) * h2f(B[k * DIM + n]);
        C[m * DIM + n] = sum;
      }
    }
  }
}

/* ------------------------------------------------ rank-4 power iteration */

struct BoundaryState {
  const int8_t* residual;  /* [column][row] */
  const float* smoothing;  /* by row */
  const float* scales;     /* by column */
  float ck[DIM * RANK], cv[DIM * RANK];
  float rk[WINDOW * DIM], rc[WINDOW * DIM];
  float record_suffix[WINDOW];
  float boundary_suffix;
};

static void apply_right(const struct BoundaryState* b, const float* vector,
                        const float* new_keys, const float* new_values,
                        uint32_t fitted, float* output) {
  /* :113-166 */
  float old_projection[RANK] = {0, 0, 0, 0}, fitted_projection[RANK] = {0, 0, 0, 0};
  float record_projection[WINDOW];
  for (uint32_t r = 0; r < RANK; ++r)
    for (uint32_t column = 0; column < DIM; ++column)
      old_projection[r] += b->cv[column * RANK + r] * vector[column];
  for (uint32_t j = 0; j < WINDOW; ++j) {
    record_projection[j] = 0.0f;
    for (uint32_t column = 0; column < DIM; ++column)
      record_projection[j] += b->rc[j * DIM + column] * vector[column];
  }
  for (uint32_t r = 0; r < fitted; ++r)
    for (uint32_t column = 0; column < DIM; ++column)
      fitted_projection[r] += new_values[column * RANK + r] * vector[column];
  for (uint32_t row = 0; row < DIM; ++row) {
    float value = 0.0f;
    for (uint32_t column = 0; column < DIM; ++column) {
      value += (float)b->residual[column * DIM + row] / 127.0f * b->smoothing[row] *
               b->scales[column] * vector[column] * b->boundary_suffix;
    }
    for (uint32_t r = 0; r < RANK; ++r)
      value += b->ck[row * RANK + r] * old_projection[r] * b->boundary_suffix;
    for (uint32_t j = 0; j < WINDOW; ++j)
      value += b->rk[j * DIM + row] * record_projection[j] * b->record_suffix[j];
    for (uint32_t r = 0; r < fitted; ++r)
      value -= new_keys[row * RANK + r] * fitted_projection[r];
    output[row] = value;
  }
}

static void apply_transpose(const struct BoundaryState* b, const float* vector,
                            const float* new_keys, const float* new_values,
                            uint32_t fitted, float* output) {
  /* :168-221 */
  float old_projection[RANK] = {0, 0, 0, 0}, fitted_projection[RANK] = {0, 0, 0, 0};
  float record_projection[WINDOW];
  for (uint32_t r = 0; r < RANK; ++r)
    for (uint32_t row = 0; row < DIM; ++row)
      old_projection[r] += b->ck[row * RANK + r] * vector[row];
  for (uint32_t j = 0; j < WINDOW; ++j) {
    record_projection[j] = 0.0f;
    for (uint32_t row = 0; row < DIM; ++row)
      record_projection[j] += b->rk[j * DIM + row] * vector[row];
  }
  for (uint32_t r = 0; r < fitted; ++r)
    for (uint32_t row = 0; row < DIM; ++row)
      fitted_projection[r] += new_keys[row * RANK + r] * vector[row];
  for (uint32_t column = 0; column < DIM; ++column) {
    float value = 0.0f;
    for (uint32_t row = 0; row < DIM; ++row) {
      value += (float)b->residual[column * DIM + row] / 127.0f * b->smoothing[row] *
               b->scales[column] * vector[row] * b->boundary_suffix;
    }
    for (uint32_t r = 0; r < RANK; ++r)
      value += b->cv[column * RANK + r] * old_projection[r] * b->boundary_suffix;
    for (uint32_t j = 0; j < WINDOW; ++j)
      value += b->rc[j * DIM + column] * record_projection[j] * b->record_suffix[j];
    for (uint32_t r = 0; r < fitted; ++r)
      value -= new_values[column * RANK + r] * fitted_projection[r];
    output[column] = value;
  }
}

static float residual_cell(const struct BoundaryState* b, uint32_t row, uint32_t column,
                           const float* new_keys, const float* new_values) {
  /* :223-251 */
  float value = (float)b->residual[column * DIM + row] / 127.0f * b->smoothing[row] *
                b->scales[column] * b->boundary_suffix;
  for (uint32_t r = 0; r < RANK; ++r) {
    value += b->ck[row * RANK + r] * b->cv[column * RANK + r] * b->boundary_suffix;
    value -= new_keys[row * RANK + r] * new_values[column * RANK + r];
  }
  for (uint32_t j = 0; j < WINDOW; ++j)
    value += b->rk[j * DIM + row] * b->rc[j * DIM + column] * b->record_suffix[j];
  return value;
}

void gdn_oracle_window_boundary_power(
    const int8_t* residual, const float* smoothing, const float* scales,
    const uint16_t* comp_keys, const uint16_t* comp_values, float* record_decay,
    uint16_t* record_keys, uint16_t* record_corrections, uint32_t* positions,
    int8_t* next_residual, float* next_smoothing, float* next_scales,
    uint16_t* next_comp_keys, uint16_t* next_comp_values,
    float* residual_workspace, uint32_t states, uint32_t power_iterations) {
  /* ProcessState (:253-366) for every state at position 16. */
  struct BoundaryState* b = (struct BoundaryState*)malloc(sizeof(struct BoundaryState));
  for (uint32_t s = 0; s < states; ++s) {
    if (positions[(size_t)s * POSITION_STRIDE] != WINDOW) continue;
    b->residual = residual + (size_t)s * TILE;
    b->smoothing = smoothing + (size_t)s * DIM;
    b->scales = scales + (size_t)s * DIM;
    for (uint32_t i = 0; i < DIM * RANK; ++i) {
      b->ck[i] = h2f(comp_keys[(size_t)s * DIM * RANK + i]);
      b->cv[i] = h2f(comp_values[(size_t)s * DIM * RANK + i]);
    }
    for (uint32_t i = 0; i < WINDOW * DIM; ++i) {
      b->rk[i] = h2f(record_keys[(size_t)s * WINDOW * DIM + i]);
      b->rc[i] = h2f(record_corrections[(size_t)s * WINDOW * DIM + i]);
    }
    b->boundary_suffix = build_suffix(record_decay + (size_t)s * WINDOW, b->record_suffix);
    float new_keys[DIM * RANK], new_values[DIM * RANK];
    for (uint32_t i = 0; i < DIM * RANK; ++i) new_keys[i] = new_values[i] = 0.0f;
    float left[DIM], right[DIM];
    const uint32_t limit = power_iterations == 0 ? 0 : RANK;
    for (uint32_t rank = 0; rank < limit; ++rank) {
      for (uint32_t column = 0; column < DIM; ++column) {
        right[column] = (float)((int32_t)(((rank + 1) * (column + 3)) % 17) - 8);
      }
      (void)normalize(right);
      for (uint32_t it = 0; it < power_iterations; ++it) {
        apply_right(b, right, new_keys, new_values, rank, left);
        if (!normalize(left)) break;
        apply_transpose(b, left, new_keys, new_values, rank, right);
        if (!normalize(right)) break;
      }
      apply_right(b, right, new_keys, new_values, rank, left);
      float singular = 0.0f;
      for (uint32_t row = 0; row < DIM; ++row) singular += left[row] * left[row];
      singular = gdn_oracle_boundary_sqrt(singular);
      if (singular > 1.0e-20f) {
        const float inverse = 1.0f / singular;
        for (uint32_t row = 0; row < DIM; ++row)
          new_keys[row * RANK + rank] = h2f(f2h(left[row] * inverse * singular));
        for (uint32_t column = 0; column < DIM; ++column)
          new_values[column * RANK + rank] = h2f(f2h(right[column]));
      }
    }
    float* work = residual_workspace + (size_t)s * TILE;
    for (uint32_t row = 0; row < DIM; ++row) {
      float mean_absolute = 0.0f;
      for (uint32_t column = 0; column < DIM; ++column) {
        const float value = residual_cell(b, row, column, new_keys, new_values);
        work[row * DIM + column] = value;
        mean_absolute += fabsf(value);
      }
      const float mean = mean_absolute / 128.0f;
      next_smoothing[(size_t)s * DIM + row] = gdn_oracle_boundary_sqrt(mean > FLOOR ? mean : FLOOR);
    }
    for (uint32_t column = 0; column < DIM; ++column) {
      float maximum = 0.0f;
      for (uint32_t row = 0; row < DIM; ++row) {
        const float value = fabsf(work[row * DIM + column] / next_smoothing[(size_t)s * DIM + row]);
        maximum = value > maximum ? value : maximum;
      }
      next_scales[(size_t)s * DIM + column] = maximum;
      for (uint32_t row = 0; row < DIM; ++row) {
        const float smoothed = work[row * DIM + column] / next_smoothing[(size_t)s * DIM + row];
        float q = maximum == 0.0f ? 0.0f : smoothed / maximum * 127.0f;
        q += q >= 0.0f ? 0.5f : -0.5f;
        q = q > 127.0f ? 127.0f : q;
        q = q < -127.0f ? -127.0f : q;
        next_residual[(size_t)s * TILE + column * DIM + row] = (int8_t)q;
      }
    }
    for (uint32_t i = 0; i < DIM * RANK; ++i) {
      next_comp_keys[(size_t)s * DIM * RANK + i] = f2h(new_keys[i]);
      next_comp_values[(size_t)s * DIM * RANK + i] = f2h(new_values[i]);
    }
    for (uint32_t j = 0; j < WINDOW; ++j) {
      record_decay[(size_t)s * WINDOW + j] = 0.0f;
      for (uint32_t k = 0; k < DIM; ++k) {
        record_keys[((size_t)s * WINDOW + j) * DIM + k] = 0;
        record_corrections[((size_t)s * WINDOW + j) * DIM + k] = 0;
      }
    }
    positions[(size_t)s * POSITION_STRIDE] = 0;
  }
  free(b);
}
