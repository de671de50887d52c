/*
 * CPU oracle for the reference's device rank-4 chain over an encoded boundary.
 *
 * TEST INFRASTRUCTURE ONLY (see gdn_oracle.h): loaded by tests/ as the checker,
 * never by the product library.
 *
 * Statement-by-statement restatements of
 *   native/ascendc/gdn_state_codec/kernel/gdn_state_codec_encoded_projection.cpp
 *     EncodedProjection::PrepareState / Value (:82-163),
 *     finish_encoded_projection (:778-820, admission :964-990),
 *     commit_encoded_rank (:822-865, admission :992-1015)
 *   native/ascendc/gdn_state_codec/kernel/gdn_state_codec_encoded_requantize.cpp
 *     EncodedRequantize::Cell / Process (:72-166, admission :189-215).
 * Each `a += b * c` is evaluated as written (separately rounded fp32
 * operations, left to right); half <-> float conversions round to nearest
 * even with subnormals.
 *
 * Operand layouts (per state): vectors fp16 / int32 / fp32 [128][16] of which
 * column 0 is the vector; dynamic_scale fp32 [8] (element 0 used); old_left /
 * old_right fp16 [128][4] ([dim][rank]); new_left / new_right fp16 [4][128]
 * ([rank][dim]); record_left / record_right fp16 [16][128]; the encoded
 * residual of encoded_requantize int8 [128 rows][128 columns], rows on the
 * smoothing axis and columns on the scale axis.
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
#define COLUMNS 16u
#define SCALAR_STRIDE 8u
#define FLOOR 1.0e-8f

static float h2f(uint16_t h) { return gdn_oracle_f16_to_f32(h); }
static uint16_t f2h(float f) { return gdn_oracle_f32_to_f16(f); }

struct EncodedOperands {
  const int32_t* projected;
  const float* dynamic_scale;
  const uint16_t* input;
  const float* smoothing;
  const float* scales;
  const uint16_t* old_left;
  const uint16_t* old_right;
  const float* record_decay;
  const uint16_t* record_left;
  const uint16_t* record_right;
  const uint16_t* new_left;
  const uint16_t* new_right;
};

/* PrepareState (:82-123): the projections of the input vector (column 0 of
 * `input`) on the old, fitted and record bases of the input side, the record
 * ones scaled by their window suffixes; returns the whole window's decay
 * product. */
static float prepare_state(const struct EncodedOperands* e, uint32_t state,
                           uint32_t fitted_ranks, uint32_t transpose,
                           float* coefficients, float* record_coefficients) {
  const size_t vector_base = (size_t)state * DIM * COLUMNS;
  const size_t old_base = (size_t)state * DIM * RANK;
  const size_t new_base = (size_t)state * RANK * DIM;
  for (uint32_t rank = 0; rank < RANK; ++rank) coefficients[rank] = 0.0f;
  for (uint32_t record = 0; record < WINDOW; ++record) record_coefficients[record] = 0.0f;
  for (uint32_t axis = 0; axis < DIM; ++axis) {
    const float input = h2f(e->input[vector_base + axis * COLUMNS]);
    for (uint32_t rank = 0; rank < RANK; ++rank) {
      const size_t old_index = old_base + axis * RANK + rank;
      const size_t new_index = new_base + rank * DIM + axis;
      const float old_basis =
          transpose == 0 ? h2f(e->old_right[old_index]) : h2f(e->old_left[old_index]);
      coefficients[rank] += old_basis * input;
      if (rank < fitted_ranks) {
        const float new_basis =
            transpose == 0 ? h2f(e->new_right[new_index]) : h2f(e->new_left[new_index]);
        coefficients[RANK + rank] += new_basis * input;
      }
    }
    for (uint32_t record = 0; record < WINDOW; ++record) {
      const size_t index = ((size_t)state * WINDOW + record) * DIM + axis;
      const float basis =
          transpose == 0 ? h2f(e->record_right[index]) : h2f(e->record_left[index]);
      record_coefficients[record] += basis * input;
    }
  }
  float suffix = 1.0f;
  for (uint32_t reverse = WINDOW; reverse > 0; --reverse) {
    const uint32_t record = reverse - 1;
    record_coefficients[record] *= suffix;
    suffix *= e->record_decay[(size_t)state * WINDOW + record];
  }
  return suffix;
}

/* Value (:125-163): row `row` of the window operator (or its transpose)
 * applied to the input vector, from the int32 projection of the encoded
 * boundary and the coefficients of prepare_state. */
static float row_value(const struct EncodedOperands* e, uint32_t state, uint32_t row,
                       uint32_t fitted_ranks, uint32_t transpose, const float* coefficients,
                       const float* record_coefficients, float boundary_suffix) {
  const size_t vector_base = (size_t)state * DIM;
  const size_t projected_base = (size_t)state * DIM * COLUMNS;
  const size_t old_base = (size_t)state * DIM * RANK;
  const size_t new_base = (size_t)state * RANK * DIM;
  float value = (float)e->projected[projected_base + row * COLUMNS] *
                e->dynamic_scale[(size_t)state * SCALAR_STRIDE] / 127.0f *
                (transpose == 0 ? e->smoothing[vector_base + row]
                                : e->scales[vector_base + row]) *
                boundary_suffix;
  for (uint32_t rank = 0; rank < RANK; ++rank) {
    const size_t old_index = old_base + row * RANK + rank;
    const float output_basis =
        transpose == 0 ? h2f(e->old_left[old_index]) : h2f(e->old_right[old_index]);
    value += output_basis * coefficients[rank] * boundary_suffix;
    if (rank < fitted_ranks) {
      const size_t new_index = new_base + rank * DIM + row;
      const float new_basis =
          transpose == 0 ? h2f(e->new_left[new_index]) : h2f(e->new_right[new_index]);
      value -= new_basis * coefficients[RANK + rank];
    }
  }
  for (uint32_t record = 0; record < WINDOW; ++record) {
    const size_t index = ((size_t)state * WINDOW + record) * DIM + row;
    const float output_basis =
        transpose == 0 ? h2f(e->record_left[index]) : h2f(e->record_right[index]);
    value += output_basis * record_coefficients[record];
  }
  return value;
}

/* finish_encoded_projection (:778-820): the operator row values normalized by
 * 1 / SquareRoot(sum of squares) (0 when that sum is <= 1e-20), written as fp16
 * to column 0 of `output`, columns 1..15 zero. */
void gdn_oracle_finish_encoded_projection(
    const int32_t* projected, const float* dynamic_scale, const uint16_t* input,
    const float* smoothing, const float* scales, const uint16_t* old_left,
    const uint16_t* old_right, const float* record_decay, const uint16_t* record_left,
    const uint16_t* record_right, const uint16_t* new_left, const uint16_t* new_right,
    uint16_t* output, uint32_t states, uint32_t fitted_ranks, uint32_t transpose) {
  const struct EncodedOperands e = {projected, dynamic_scale, input, smoothing, scales,
                                    old_left, old_right, record_decay, record_left,
                                    record_right, new_left, new_right};
  for (uint32_t state = 0; state < states; ++state) {
    float coefficients[RANK * 2] = {0, 0, 0, 0, 0, 0, 0, 0};
    float record_coefficients[WINDOW];
    const float boundary_suffix = prepare_state(&e, state, fitted_ranks, transpose,
                                                coefficients, record_coefficients);
    float values[DIM];
    float squared_norm = 0.0f;
    for (uint32_t row = 0; row < DIM; ++row) {
      values[row] = row_value(&e, state, row, fitted_ranks, transpose, coefficients,
                              record_coefficients, boundary_suffix);
      squared_norm += values[row] * values[row];
    }
    const float inverse =
        squared_norm > 1.0e-20f ? 1.0f / gdn_oracle_boundary_sqrt(squared_norm) : 0.0f;
    const size_t base = (size_t)state * DIM * COLUMNS;
    for (uint32_t row = 0; row < DIM; ++row) {
      output[base + row * COLUMNS] = f2h(values[row] * inverse);
      for (uint32_t column = 1; column < COLUMNS; ++column) {
        output[base + row * COLUMNS + column] = 0;
      }
    }
  }
}

/* commit_encoded_rank (:822-865): the forward operator row values with `rank`
 * fitted ranks deflated; corrected column 0 = value, new_left[rank] =
 * fp16(value), new_right[rank] = the input vector's fp16 bits.  Other columns
 * of `corrected` and other ranks of the bases are untouched. */
void gdn_oracle_commit_encoded_rank(
    const int32_t* projected, const float* dynamic_scale, const uint16_t* input,
    const float* smoothing, const float* scales, const uint16_t* old_left,
    const uint16_t* old_right, const float* record_decay, const uint16_t* record_left,
    const uint16_t* record_right, uint16_t* new_left, uint16_t* new_right,
    float* corrected, uint32_t states, uint32_t rank) {
  const struct EncodedOperands e = {projected, dynamic_scale, input, smoothing, scales,
                                    old_left, old_right, record_decay, record_left,
                                    record_right, new_left, new_right};
  for (uint32_t state = 0; state < states; ++state) {
    float coefficients[RANK * 2] = {0, 0, 0, 0, 0, 0, 0, 0};
    float record_coefficients[WINDOW];
    const float boundary_suffix =
        prepare_state(&e, state, rank, 0, coefficients, record_coefficients);
    const size_t vector_base = (size_t)state * DIM * COLUMNS;
    const size_t basis_base = (size_t)state * RANK * DIM + (size_t)rank * DIM;
    for (uint32_t row = 0; row < DIM; ++row) {
      const float value = row_value(&e, state, row, rank, 0, coefficients,
                                    record_coefficients, boundary_suffix);
      corrected[vector_base + row * COLUMNS] = value;
      new_left[basis_base + row] = f2h(value);
      new_right[basis_base + row] = input[vector_base + row * COLUMNS];
    }
  }
}

/* EncodedRequantize::Cell (:72-100). */
static float requantize_cell(const struct EncodedOperands* e, const int8_t* residual,
                             uint32_t state, uint32_t row, uint32_t column,
                             const float* record_suffix, float boundary_suffix) {
  const size_t old_base = (size_t)state * DIM * RANK;
  const size_t new_base = (size_t)state * RANK * DIM;
  float value = (float)residual[(size_t)state * TILE + row * DIM + column] / 127.0f *
                e->smoothing[(size_t)state * DIM + row] *
                e->scales[(size_t)state * DIM + column] * boundary_suffix;
  for (uint32_t rank = 0; rank < RANK; ++rank) {
    value += h2f(e->old_left[old_base + row * RANK + rank]) *
             h2f(e->old_right[old_base + column * RANK + rank]) * boundary_suffix;
    value -= h2f(e->new_left[new_base + rank * DIM + row]) *
             h2f(e->new_right[new_base + rank * DIM + column]);
  }
  for (uint32_t record = 0; record < WINDOW; ++record) {
    const size_t record_base = ((size_t)state * WINDOW + record) * DIM;
    value += h2f(e->record_left[record_base + row]) * h2f(e->record_right[record_base + column]) *
             record_suffix[record];
  }
  return value;
}

/* encoded_requantize (:102-166): the window operator minus the committed ranks,
 * re-encoded with fresh smoothing (20-step Newton square root of the mean
 * |row|), absmax scales and round-half-away codes; the fitted residual goes to
 * residual_workspace [row][column] and the committed bases are transposed to
 * next_left / next_right [dim][rank]. */
void gdn_oracle_encoded_requantize(
    const int8_t* residual, const float* smoothing, const float* scales,
    const uint16_t* old_left, const uint16_t* old_right, const float* record_decay,
    const uint16_t* record_left, const uint16_t* record_right, const uint16_t* new_left,
    const uint16_t* new_right, int8_t* next_residual, float* next_smoothing,
    float* next_scales, uint16_t* next_left, uint16_t* next_right,
    float* residual_workspace, uint32_t states) {
  const struct EncodedOperands e = {NULL, NULL, NULL, smoothing, scales, old_left,
                                    old_right, record_decay, record_left, record_right,
                                    new_left, new_right};
  for (uint32_t state = 0; state < states; ++state) {
    float record_suffix[WINDOW];
    float suffix = 1.0f;
    for (uint32_t reverse = WINDOW; reverse > 0; --reverse) {
      const uint32_t record = reverse - 1;
      record_suffix[record] = suffix;
      suffix *= record_decay[(size_t)state * WINDOW + record];
    }
    float* work = residual_workspace + (size_t)state * TILE;
    for (uint32_t row = 0; row < DIM; ++row) {
      float mean_absolute = 0.0f;
      for (uint32_t column = 0; column < DIM; ++column) {
        const float value = requantize_cell(&e, residual, state, row, column, record_suffix,
                                            suffix);
        work[row * DIM + column] = value;
        mean_absolute += fabsf(value);
      }
      const float mean = mean_absolute / 128.0f;
      next_smoothing[(size_t)state * DIM + row] =
          gdn_oracle_boundary_sqrt(mean > FLOOR ? mean : FLOOR);
    }
    for (uint32_t column = 0; column < DIM; ++column) {
      float maximum = 0.0f;
      for (uint32_t row = 0; row < DIM; ++row) {
        const float value =
            fabsf(work[row * DIM + column] / next_smoothing[(size_t)state * DIM + row]);
        maximum = value > maximum ? value : maximum;
      }
      next_scales[(size_t)state * DIM + column] = maximum;
      for (uint32_t row = 0; row < DIM; ++row) {
        const float smoothed = work[row * DIM + column] / next_smoothing[(size_t)state * DIM + row];
        float quantized = maximum > 0.0f ? smoothed / maximum * 127.0f : 0.0f;
        quantized += quantized >= 0.0f ? 0.5f : -0.5f;
        quantized = quantized > 127.0f ? 127.0f : quantized;
        quantized = quantized < -127.0f ? -127.0f : quantized;
        next_residual[(size_t)state * TILE + row * DIM + column] = (int8_t)quantized;
      }
    }
    const size_t output_base = (size_t)state * DIM * RANK;
    const size_t new_base = (size_t)state * RANK * DIM;
    for (uint32_t axis = 0; axis < DIM; ++axis) {
      for (uint32_t rank = 0; rank < RANK; ++rank) {
        next_left[output_base + axis * RANK + rank] = new_left[new_base + rank * DIM + axis];
        next_right[output_base + axis * RANK + rank] = new_right[new_base + rank * DIM + axis];
      }
    }
  }
}
