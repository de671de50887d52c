/*
 * CPU oracle for the GDN state codec hot path -- TEST INFRASTRUCTURE ONLY.
 * See gdn_oracle.h for scope and for the checks that pin each function.
 *
 * Every float expression below keeps the reference's operand order and its
 * float/double types; the library is built with -ffp-contract=off and without
 * -march, so nothing is fused or reassociated.
 */
#include "gdn_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stddef.h>
#include <stdlib.h>
#include <string.h>

#define TILE_DIM 128u
#define TILE_ELEMENTS (TILE_DIM * TILE_DIM)
#define SMOOTHING_FLOOR 1.0e-8f
#define QUANTIZED_MAXIMUM 127.0f /* kQuantizedMaximum, state_capsule.cpp:20 */

/* ---------------------------------------------------------------- helpers */

/* Norm (state_capsule.cpp:50-54): double sum of squares, float result. */
static float norm_f(const float* values, size_t count) {
  double sum = 0.0;
  for (size_t i = 0; i < count; ++i) sum += (double)values[i] * values[i];
  return (float)sqrt(sum);
}

/* Normalize (state_capsule.cpp:61-66). Returns 0 (and leaves values alone)
 * when the norm is not above FLT_EPSILON. */
static int normalize_f(float* values, size_t count) {
  const float norm = norm_f(values, count);
  if (!(norm > FLT_EPSILON)) return 0;
  for (size_t i = 0; i < count; ++i) values[i] /= norm;
  return 1;
}

/* std::max(a, b) for floats: (a < b) ? b : a, so ties keep a. */
static float max_keep_first(float a, float b) { return (a < b) ? b : a; }

float gdn_oracle_bf16_to_f32(uint16_t value) {
  const uint32_t bits = (uint32_t)value << 16;
  float out;
  memcpy(&out, &bits, sizeof(out));
  return out;
}

uint16_t gdn_oracle_f32_to_bf16(float value) {
  uint32_t bits;
  memcpy(&bits, &value, sizeof(bits));
  const uint32_t least_significant = (bits >> 16) & 1u;
  return (uint16_t)((bits + 0x7FFFu + least_significant) >> 16);
}

void gdn_oracle_f32_to_bf16_array(const float* values, uint64_t count, uint16_t* out) {
  for (uint64_t i = 0; i < count; ++i) out[i] = gdn_oracle_f32_to_bf16(values[i]);
}

/* ------------------------------------------------------ single head, [K][V] */

void gdn_oracle_quantize_kv(const float* dense, uint32_t keys, uint32_t values,
                            uint32_t rank, float smoothing_floor,
                            int8_t* codes, float* smoothing, float* value_scales,
                            float* comp_keys, float* comp_values, float* work) {
  const size_t K = keys, V = values;
  /* work holds the residual, then the smoothed residual in place: each
   * smoothed element depends only on its own residual element and its row's
   * smoothing, which is fixed before the row is overwritten. */
  float* residual = work;
  memcpy(residual, dense, K * V * sizeof(float));

  /* Rank-r sinusoidal power-iteration fit (state_capsule.cpp:136-188). */
  if (rank > 0) {
    memset(comp_keys, 0, K * rank * sizeof(float));
    memset(comp_values, 0, V * rank * sizeof(float));
    float* right = (float*)malloc(V * sizeof(float));
    float* left = (float*)malloc(K * sizeof(float));
    for (size_t r = 0; r < rank; ++r) {
      for (size_t column = 0; column < V; ++column) {
        right[column] = sinf((float)((r + 1) * (column + 1)));
      }
      if (!normalize_f(right, V)) right[0] = 1.0f;
      for (int iteration = 0; iteration < 32; ++iteration) {
        for (size_t row = 0; row < K; ++row) left[row] = 0.0f;
        for (size_t row = 0; row < K; ++row) {
          for (size_t column = 0; column < V; ++column) {
            left[row] += residual[row * V + column] * right[column];
          }
        }
        if (!normalize_f(left, K)) break;
        for (size_t column = 0; column < V; ++column) right[column] = 0.0f;
        for (size_t column = 0; column < V; ++column) {
          for (size_t row = 0; row < K; ++row) {
            right[column] += residual[row * V + column] * left[row];
          }
        }
        if (!normalize_f(right, V)) break;
      }
      float singular_value = 0.0f;
      for (size_t row = 0; row < K; ++row) {
        for (size_t column = 0; column < V; ++column) {
          singular_value += left[row] * residual[row * V + column] * right[column];
        }
      }
      for (size_t row = 0; row < K; ++row) {
        comp_keys[row * rank + r] = left[row] * singular_value;
      }
      for (size_t column = 0; column < V; ++column) {
        comp_values[column * rank + r] = right[column];
      }
      for (size_t row = 0; row < K; ++row) {
        for (size_t column = 0; column < V; ++column) {
          residual[row * V + column] -= left[row] * singular_value * right[column];
        }
      }
    }
    free(left);
    free(right);
  }

  /* Smoothing: fp64 sequential mean of |residual| per key row, float sqrt
   * (state_capsule.cpp:190-205). */
  for (size_t row = 0; row < K; ++row) {
    double mean_absolute = 0.0;
    for (size_t column = 0; column < V; ++column) {
      mean_absolute += fabsf(residual[row * V + column]);
    }
    mean_absolute /= (double)V;
    const float s = sqrtf(max_keep_first((float)mean_absolute, smoothing_floor));
    smoothing[row] = s;
    for (size_t column = 0; column < V; ++column) {
      residual[row * V + column] = residual[row * V + column] / s;
    }
  }

  /* Per-value absmax scale and int8 codes (state_capsule.cpp:207-225). */
  for (size_t column = 0; column < V; ++column) {
    float maximum = 0.0f;
    for (size_t row = 0; row < K; ++row) {
      maximum = max_keep_first(maximum, fabsf(residual[row * V + column]));
    }
    value_scales[column] = maximum;
    for (size_t row = 0; row < K; ++row) {
      const float scaled = maximum == 0.0f
                               ? 0.0f
                               : residual[row * V + column] / maximum *
                                     QUANTIZED_MAXIMUM;
      long quantized = lroundf(scaled);
      if (quantized < -127L) quantized = -127L;
      if (quantized > 127L) quantized = 127L;
      codes[row * V + column] = (int8_t)quantized;
    }
  }
}

void gdn_oracle_dequantize_kv(const int8_t* codes, const float* smoothing,
                              const float* value_scales, const float* comp_keys,
                              const float* comp_values, uint32_t keys,
                              uint32_t values, uint32_t rank, float* dense) {
  const size_t K = keys, V = values;
  for (size_t row = 0; row < K; ++row) {
    for (size_t column = 0; column < V; ++column) {
      float value = smoothing[row] * (float)codes[row * V + column] /
                    QUANTIZED_MAXIMUM * value_scales[column];
      for (size_t r = 0; r < rank; ++r) {
        value += comp_keys[row * rank + r] * comp_values[column * rank + r];
      }
      dense[row * V + column] = value;
    }
  }
}

void gdn_oracle_read_boundary(const int8_t* codes, const float* smoothing,
                              const float* value_scales, const float* comp_keys,
                              const float* comp_values, uint32_t keys,
                              uint32_t values, uint32_t rank, const float* read,
                              float* output) {
  const size_t K = keys, V = values;
  for (size_t column = 0; column < V; ++column) output[column] = 0.0f;
  for (size_t column = 0; column < V; ++column) {
    float residual_projection = 0.0f;
    for (size_t row = 0; row < K; ++row) {
      residual_projection +=
          (float)codes[row * V + column] * smoothing[row] * read[row];
    }
    output[column] += residual_projection / QUANTIZED_MAXIMUM * value_scales[column];
  }
  for (size_t r = 0; r < rank; ++r) {
    float projection = 0.0f;
    for (size_t row = 0; row < K; ++row) {
      projection += comp_keys[row * rank + r] * read[row];
    }
    for (size_t column = 0; column < V; ++column) {
      output[column] += comp_values[column * rank + r] * projection;
    }
  }
}

void gdn_oracle_provider_to_codec(const float* provider, uint32_t keys,
                                  uint32_t values, float* codec) {
  for (size_t value = 0; value < values; ++value) {
    for (size_t key = 0; key < keys; ++key) {
      codec[key * values + value] = provider[value * keys + key];
    }
  }
}

void gdn_oracle_codec_to_provider(const float* codec, uint32_t keys,
                                  uint32_t values, float* provider) {
  for (size_t key = 0; key < keys; ++key) {
    for (size_t value = 0; value < values; ++value) {
      provider[value * keys + key] = codec[key * values + value];
    }
  }
}

/* ------------------------------------------------------------ threading */

typedef void (*range_fn)(void* ctx, uint64_t begin, uint64_t end);

typedef struct {
  range_fn fn;
  void* ctx;
  uint64_t begin, end;
} range_job;

static void* range_thread(void* arg) {
  range_job* job = (range_job*)arg;
  job->fn(job->ctx, job->begin, job->end);
  return NULL;
}

/* Splits [0, count) into contiguous chunks, one per thread. */
static void parallel_for(uint64_t count, int threads, range_fn fn, void* ctx) {
  if (threads <= 1 || count < 2) {
    fn(ctx, 0, count);
    return;
  }
  if ((uint64_t)threads > count) threads = (int)count;
  pthread_t* ids = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
  range_job* jobs = (range_job*)malloc(sizeof(range_job) * (size_t)threads);
  for (int t = 0; t < threads; ++t) {
    jobs[t].fn = fn;
    jobs[t].ctx = ctx;
    jobs[t].begin = count * (uint64_t)t / (uint64_t)threads;
    jobs[t].end = count * (uint64_t)(t + 1) / (uint64_t)threads;
    pthread_create(&ids[t], NULL, range_thread, &jobs[t]);
  }
  for (int t = 0; t < threads; ++t) pthread_join(ids[t], NULL);
  free(jobs);
  free(ids);
}

/* --------------------------------------------------- batched 128x128 heads */

/* Quant-only encode of one 128x128 tile in either layout.  The provider layout
 * is the transpose of the codec layout (adapter.cpp:21-57), so the tile is
 * transposed, encoded, and its codes transposed back; smoothing stays indexed
 * by key and scales by value. */
static void encode_tile(const float* tile, uint32_t layout, int8_t* codes,
                        float* smoothing, float* value_scales, float* kv,
                        float* work, int8_t* codes_kv) {
  if (layout == GDN_ORACLE_LAYOUT_KEY_VALUE) {
    gdn_oracle_quantize_kv(tile, TILE_DIM, TILE_DIM, 0, SMOOTHING_FLOOR, codes,
                           smoothing, value_scales, NULL, NULL, work);
    return;
  }
  gdn_oracle_provider_to_codec(tile, TILE_DIM, TILE_DIM, kv);
  gdn_oracle_quantize_kv(kv, TILE_DIM, TILE_DIM, 0, SMOOTHING_FLOOR, codes_kv,
                         smoothing, value_scales, NULL, NULL, work);
  for (size_t key = 0; key < TILE_DIM; ++key) {
    for (size_t value = 0; value < TILE_DIM; ++value) {
      codes[value * TILE_DIM + key] = codes_kv[key * TILE_DIM + value];
    }
  }
}

static void decode_tile(const int8_t* codes, const float* smoothing,
                        const float* value_scales, uint32_t layout, float* tile,
                        int8_t* codes_kv, float* kv) {
  if (layout == GDN_ORACLE_LAYOUT_KEY_VALUE) {
    gdn_oracle_dequantize_kv(codes, smoothing, value_scales, NULL, NULL, TILE_DIM,
                             TILE_DIM, 0, tile);
    return;
  }
  for (size_t value = 0; value < TILE_DIM; ++value) {
    for (size_t key = 0; key < TILE_DIM; ++key) {
      codes_kv[key * TILE_DIM + value] = codes[value * TILE_DIM + key];
    }
  }
  gdn_oracle_dequantize_kv(codes_kv, smoothing, value_scales, NULL, NULL,
                           TILE_DIM, TILE_DIM, 0, kv);
  gdn_oracle_codec_to_provider(kv, TILE_DIM, TILE_DIM, tile);
}

typedef struct {
  const float* state;
  uint32_t layout;
  int8_t* codes;
  float* smoothing;
  float* value_scales;
} encode_ctx;

static void encode_range(void* arg, uint64_t begin, uint64_t end) {
  encode_ctx* c = (encode_ctx*)arg;
  float* kv = (float*)malloc(TILE_ELEMENTS * sizeof(float));
  float* work = (float*)malloc(TILE_ELEMENTS * sizeof(float));
  int8_t* codes_kv = (int8_t*)malloc(TILE_ELEMENTS);
  for (uint64_t h = begin; h < end; ++h) {
    encode_tile(c->state + h * TILE_ELEMENTS, c->layout,
                c->codes + h * TILE_ELEMENTS, c->smoothing + h * TILE_DIM,
                c->value_scales + h * TILE_DIM, kv, work, codes_kv);
  }
  free(codes_kv);
  free(work);
  free(kv);
}

void gdn_oracle_encode_heads(const float* state, uint64_t heads, uint32_t layout,
                             int8_t* codes, float* smoothing, float* value_scales,
                             int threads) {
  encode_ctx c = {state, layout, codes, smoothing, value_scales};
  parallel_for(heads, threads, encode_range, &c);
}

typedef struct {
  const int8_t* codes;
  const float* smoothing;
  const float* value_scales;
  uint32_t layout;
  float* state;
} decode_ctx;

static void decode_range(void* arg, uint64_t begin, uint64_t end) {
  decode_ctx* c = (decode_ctx*)arg;
  float* kv = (float*)malloc(TILE_ELEMENTS * sizeof(float));
  int8_t* codes_kv = (int8_t*)malloc(TILE_ELEMENTS);
  for (uint64_t h = begin; h < end; ++h) {
    decode_tile(c->codes + h * TILE_ELEMENTS, c->smoothing + h * TILE_DIM,
                c->value_scales + h * TILE_DIM, c->layout,
                c->state + h * TILE_ELEMENTS, codes_kv, kv);
  }
  free(codes_kv);
  free(kv);
}

void gdn_oracle_decode_heads(const int8_t* codes, const float* smoothing,
                             const float* value_scales, uint64_t heads,
                             uint32_t layout, float* state, int threads) {
  decode_ctx c = {codes, smoothing, value_scales, layout, state};
  parallel_for(heads, threads, decode_range, &c);
}

/* ----------------------------------------------------- encoded projection */

/* One boundary readout of a 128x128 tile against x (state_capsule.cpp:281-290,
 * records and compensators absent).  code(v, k) follows the tile layout. */
static void readout_tile(const int8_t* codes, const float* smoothing,
                         const float* value_scales, uint32_t layout,
                         const float* x, float* out, double* out_f64,
                         double* abs_bound) {
  for (size_t v = 0; v < TILE_DIM; ++v) {
    float residual_projection = 0.0f;
    double exact = 0.0, magnitude = 0.0;
    for (size_t k = 0; k < TILE_DIM; ++k) {
      const int8_t code = layout == GDN_ORACLE_LAYOUT_KEY_VALUE
                              ? codes[k * TILE_DIM + v]
                              : codes[v * TILE_DIM + k];
      residual_projection += (float)code * smoothing[k] * x[k];
      const double term = (double)code * (double)smoothing[k] * (double)x[k];
      exact += term;
      magnitude += fabs(term);
    }
    float o = 0.0f;
    o += residual_projection / QUANTIZED_MAXIMUM * value_scales[v];
    out[v] = o;
    if (out_f64) out_f64[v] = exact / 127.0 * (double)value_scales[v];
    if (abs_bound) abs_bound[v] = magnitude / 127.0 * (double)value_scales[v];
  }
}

static void load_query(const uint16_t* q, float query_scale, float* x) {
  for (size_t k = 0; k < TILE_DIM; ++k) {
    x[k] = query_scale * gdn_oracle_bf16_to_f32(q[k]);
  }
}

void gdn_oracle_project_decode(const int8_t* codes, const float* smoothing,
                               const float* value_scales, const uint16_t* queries,
                               uint32_t batch, uint32_t value_heads,
                               uint32_t query_heads, float query_scale,
                               uint32_t layout, float* out, double* out_f64,
                               double* abs_bound) {
  float x[TILE_DIM];
  for (uint64_t b = 0; b < batch; ++b) {
    for (uint64_t h = 0; h < value_heads; ++h) {
      const uint64_t state = b * value_heads + h;
      const uint64_t qh = h * query_heads / value_heads;
      load_query(queries + (b * query_heads + qh) * TILE_DIM, query_scale, x);
      readout_tile(codes + state * TILE_ELEMENTS, smoothing + state * TILE_DIM,
                   value_scales + state * TILE_DIM, layout, x,
                   out + state * TILE_DIM,
                   out_f64 ? out_f64 + state * TILE_DIM : NULL,
                   abs_bound ? abs_bound + state * TILE_DIM : NULL);
    }
  }
}

typedef struct {
  const int8_t* codes;
  const float* smoothing;
  const float* value_scales;
  const uint16_t* queries;
  uint32_t tokens, value_heads, query_heads, layout;
  float query_scale;
  float* out;
  double* out_f64;
  double* abs_bound;
} chunked_ctx;

static void chunked_range(void* arg, uint64_t begin, uint64_t end) {
  chunked_ctx* c = (chunked_ctx*)arg;
  float x[TILE_DIM];
  for (uint64_t pair = begin; pair < end; ++pair) {
    const uint64_t n = pair / c->value_heads, h = pair % c->value_heads;
    const uint64_t qh = h * c->query_heads / c->value_heads;
    for (uint64_t t = 0; t < c->tokens; ++t) {
      const uint64_t row = (n * c->tokens + t);
      load_query(c->queries + (row * c->query_heads + qh) * TILE_DIM,
                 c->query_scale, x);
      const uint64_t o = (row * c->value_heads + h) * TILE_DIM;
      readout_tile(c->codes + pair * TILE_ELEMENTS, c->smoothing + pair * TILE_DIM,
                   c->value_scales + pair * TILE_DIM, c->layout, x, c->out + o,
                   c->out_f64 ? c->out_f64 + o : NULL,
                   c->abs_bound ? c->abs_bound + o : NULL);
    }
  }
}

void gdn_oracle_project_chunked(const int8_t* codes, const float* smoothing,
                                const float* value_scales,
                                const uint16_t* queries, uint32_t seqs,
                                uint32_t tokens, uint32_t value_heads,
                                uint32_t query_heads, float query_scale,
                                uint32_t layout, float* out, double* out_f64,
                                double* abs_bound, int threads) {
  chunked_ctx c = {codes, smoothing, value_scales, queries, tokens, value_heads,
                   query_heads, layout, query_scale, out, out_f64, abs_bound};
  parallel_for((uint64_t)seqs * value_heads, threads, chunked_range, &c);
}

/* ------------------------------------------------------------ slot pools */

typedef struct {
  const void* pool;
  void* pool_out;
  uint32_t dtype;
  const int32_t* slot_ids;
  uint32_t batch, slots, heads, layout;
  const int8_t* codes_in;
  const float* smoothing_in;
  const float* scales_in;
  int8_t* codes;
  float* smoothing;
  float* value_scales;
} pool_ctx;

static void load_pool_tile(const void* pool, uint32_t dtype, uint64_t entry,
                           float* tile) {
  if (dtype == GDN_ORACLE_DTYPE_F32) {
    memcpy(tile, (const float*)pool + entry * TILE_ELEMENTS,
           TILE_ELEMENTS * sizeof(float));
  } else {
    const uint16_t* src = (const uint16_t*)pool + entry * TILE_ELEMENTS;
    for (size_t i = 0; i < TILE_ELEMENTS; ++i) tile[i] = gdn_oracle_bf16_to_f32(src[i]);
  }
}

static void store_pool_tile(void* pool, uint32_t dtype, uint64_t entry,
                            const float* tile) {
  if (dtype == GDN_ORACLE_DTYPE_F32) {
    memcpy((float*)pool + entry * TILE_ELEMENTS, tile, TILE_ELEMENTS * sizeof(float));
  } else {
    uint16_t* dst = (uint16_t*)pool + entry * TILE_ELEMENTS;
    for (size_t i = 0; i < TILE_ELEMENTS; ++i) dst[i] = gdn_oracle_f32_to_bf16(tile[i]);
  }
}

/* Work items are (layer, batch entry, head) in compact order. */
static void pool_encode_range(void* arg, uint64_t begin, uint64_t end) {
  pool_ctx* c = (pool_ctx*)arg;
  float* tile = (float*)malloc(TILE_ELEMENTS * sizeof(float));
  float* kv = (float*)malloc(TILE_ELEMENTS * sizeof(float));
  float* work = (float*)malloc(TILE_ELEMENTS * sizeof(float));
  int8_t* codes_kv = (int8_t*)malloc(TILE_ELEMENTS);
  for (uint64_t item = begin; item < end; ++item) {
    const uint64_t h = item % c->heads;
    const uint64_t b = (item / c->heads) % c->batch;
    const uint64_t l = item / ((uint64_t)c->heads * c->batch);
    const int32_t slot = c->slot_ids[b];
    if (slot < 0 || (uint32_t)slot >= c->slots) continue;
    const uint64_t entry = ((l * c->slots) + (uint64_t)slot) * c->heads + h;
    load_pool_tile(c->pool, c->dtype, entry, tile);
    encode_tile(tile, c->layout, c->codes + item * TILE_ELEMENTS,
                c->smoothing + item * TILE_DIM, c->value_scales + item * TILE_DIM,
                kv, work, codes_kv);
  }
  free(codes_kv);
  free(work);
  free(kv);
  free(tile);
}

void gdn_oracle_pool_encode(const void* pool, uint32_t pool_dtype,
                            const int32_t* slot_ids, uint32_t batch,
                            uint32_t layers, uint32_t slots, uint32_t heads,
                            uint32_t layout, int8_t* codes, float* smoothing,
                            float* value_scales, int threads) {
  pool_ctx c;
  memset(&c, 0, sizeof(c));
  c.pool = pool;
  c.dtype = pool_dtype;
  c.slot_ids = slot_ids;
  c.batch = batch;
  c.slots = slots;
  c.heads = heads;
  c.layout = layout;
  c.codes = codes;
  c.smoothing = smoothing;
  c.value_scales = value_scales;
  parallel_for((uint64_t)layers * batch * heads, threads, pool_encode_range, &c);
}

static void pool_decode_range(void* arg, uint64_t begin, uint64_t end) {
  pool_ctx* c = (pool_ctx*)arg;
  float* tile = (float*)malloc(TILE_ELEMENTS * sizeof(float));
  float* kv = (float*)malloc(TILE_ELEMENTS * sizeof(float));
  int8_t* codes_kv = (int8_t*)malloc(TILE_ELEMENTS);
  for (uint64_t item = begin; item < end; ++item) {
    const uint64_t h = item % c->heads;
    const uint64_t b = (item / c->heads) % c->batch;
    const uint64_t l = item / ((uint64_t)c->heads * c->batch);
    const int32_t slot = c->slot_ids[b];
    if (slot < 0 || (uint32_t)slot >= c->slots) continue;
    const uint64_t entry = ((l * c->slots) + (uint64_t)slot) * c->heads + h;
    decode_tile(c->codes_in + item * TILE_ELEMENTS, c->smoothing_in + item * TILE_DIM,
                c->scales_in + item * TILE_DIM, c->layout, tile, codes_kv, kv);
    store_pool_tile(c->pool_out, c->dtype, entry, tile);
  }
  free(codes_kv);
  free(kv);
  free(tile);
}

void gdn_oracle_pool_decode(const int8_t* codes, const float* smoothing,
                            const float* value_scales, const int32_t* slot_ids,
                            uint32_t batch, uint32_t layers, uint32_t slots,
                            uint32_t heads, uint32_t layout, void* pool,
                            uint32_t pool_dtype, int threads) {
  pool_ctx c;
  memset(&c, 0, sizeof(c));
  c.pool_out = pool;
  c.dtype = pool_dtype;
  c.slot_ids = slot_ids;
  c.batch = batch;
  c.slots = slots;
  c.heads = heads;
  c.layout = layout;
  c.codes_in = codes;
  c.smoothing_in = smoothing;
  c.scales_in = value_scales;
  /* Two batch entries naming the same slot would race; callers pass unique
   * slot ids, as vLLM's cache indices are. */
  parallel_for((uint64_t)layers * batch * heads, threads, pool_decode_range, &c);
}
