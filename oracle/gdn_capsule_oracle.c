/*
 * CPU oracle of the capsule wire format (LQCAPS01) -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of GdnStateCodecCapsule::Serialize / Restore
 * (native/src/gdn_state_codec_state_capsule.cpp:446-578) and of the SHA-256
 * the format carries (FIPS 180-4), plus the mapping between the device window
 * slot (fp16 compensators and records, one scalar gate per record, [V][K] or
 * [K][V] codes) and a capsule.  Only tests/ and bench.py's cpu_baseline leg
 * load it; the product library never links or calls it.
 *
 * Pins (tests/test_capsule_oracle.py):
 *   SHA-256         : FIPS 180-4 example vectors and hashlib on every length
 *                     0..300 and multi-block messages; the reference's own
 *                     Sha256Hex (native/src/sha256.cpp) through oracle/_ref.
 *   serialize       : byte equality with the reference's Serialize of capsules
 *                     the reference built itself (FromDenseBoundary + ApplyToken,
 *                     oracle/_ref), after an oracle restore of those bytes.
 *   restore         : the accept/reject decision and the failing check agree
 *                     with the reference's Restore (oracle/_ref, its exception
 *                     message) on the reference test's own corruptions
 *                     (native/tests/gdn_state_codec_state_capsule_test.cpp:
 *                     292-371) and on truncations, trailing bytes, non-finite
 *                     records and overflowing boundaries.
 *   slot mapping    : the reference's Restore admits every slot capsule, its
 *                     Serialize re-emits the same bytes, and its DenseState is
 *                     the window's dense state (numpy float64, fp32 tolerance).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "gdn_oracle.h"

/* ---- SHA-256 (FIPS 180-4 sections 4.1.2, 4.2.2, 5.1.1, 5.3.3, 6.2) ---- */

/* First 32 bits of the fractional parts of the cube roots of the first 64
 * primes (FIPS 180-4 section 4.2.2). */
static const uint32_t kRoundConstants[64] = {
    0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u,
    0x923f82a4u, 0xab1c5ed5u, 0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u,
    0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u, 0xe49b69c1u, 0xefbe4786u,
    0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
    0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u,
    0x06ca6351u, 0x14292967u, 0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u,
    0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u, 0xa2bfe8a1u, 0xa81a664bu,
    0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
    0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au,
    0x5b9cca4fu, 0x682e6ff3u, 0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u,
    0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};

/* First 32 bits of the fractional parts of the square roots of the first 8
 * primes (FIPS 180-4 section 5.3.3). */
static const uint32_t kInitialHash[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u,
                                         0xa54ff53au, 0x510e527fu, 0x9b05688cu,
                                         0x1f83d9abu, 0x5be0cd19u};

static uint32_t rotr(uint32_t x, unsigned n) { return (x >> n) | (x << (32u - n)); }

static void sha256_block(uint32_t state[8], const uint8_t block[64]) {
  uint32_t w[64];
  for (int t = 0; t < 16; ++t) {
    w[t] = ((uint32_t)block[4 * t] << 24) | ((uint32_t)block[4 * t + 1] << 16) |
           ((uint32_t)block[4 * t + 2] << 8) | (uint32_t)block[4 * t + 3];
  }
  for (int t = 16; t < 64; ++t) {
    const uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
    const uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
    w[t] = w[t - 16] + s0 + w[t - 7] + s1;
  }
  uint32_t a = state[0], b = state[1], c = state[2], d = state[3];
  uint32_t e = state[4], f = state[5], g = state[6], h = state[7];
  for (int t = 0; t < 64; ++t) {
    const uint32_t t1 = h + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) +
                        ((e & f) ^ (~e & g)) + kRoundConstants[t] + w[t];
    const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) +
                        ((a & b) ^ (a & c) ^ (b & c));
    h = g;
    g = f;
    f = e;
    e = d + t1;
    d = c;
    c = b;
    b = a;
    a = t1 + t2;
  }
  state[0] += a;
  state[1] += b;
  state[2] += c;
  state[3] += d;
  state[4] += e;
  state[5] += f;
  state[6] += g;
  state[7] += h;
}

void gdn_oracle_sha256(const uint8_t* data, uint64_t size, uint8_t digest[32]) {
  uint32_t state[8];
  memcpy(state, kInitialHash, sizeof(state));
  uint64_t offset = 0;
  for (; size - offset >= 64; offset += 64) sha256_block(state, data + offset);
  /* Padding (section 5.1.1): 0x80, zeros, the 64-bit big-endian bit length. */
  uint8_t tail[128];
  memset(tail, 0, sizeof(tail));
  const uint64_t rest = size - offset;
  if (rest) memcpy(tail, data + offset, rest);
  tail[rest] = 0x80u;
  const uint64_t blocks = rest + 9 <= 64 ? 1 : 2;
  const uint64_t bits = size * 8u;
  for (int i = 0; i < 8; ++i) tail[blocks * 64 - 1 - i] = (uint8_t)(bits >> (8 * i));
  for (uint64_t b = 0; b < blocks; ++b) sha256_block(state, tail + 64 * b);
  for (int i = 0; i < 8; ++i) {
    digest[4 * i] = (uint8_t)(state[i] >> 24);
    digest[4 * i + 1] = (uint8_t)(state[i] >> 16);
    digest[4 * i + 2] = (uint8_t)(state[i] >> 8);
    digest[4 * i + 3] = (uint8_t)state[i];
  }
}

void gdn_oracle_sha256_hex(const uint8_t* data, uint64_t size, char hex[64]) {
  static const char kDigits[] = "0123456789abcdef";
  uint8_t digest[32];
  gdn_oracle_sha256(data, size, digest);
  for (int i = 0; i < 32; ++i) {
    hex[2 * i] = kDigits[digest[i] >> 4];
    hex[2 * i + 1] = kDigits[digest[i] & 15u];
  }
}

/* ---- capsule layout (state_capsule.cpp:446-474) ------------------------- */

static const char kMagic[8] = {'L', 'Q', 'C', 'A', 'P', 'S', '0', '1'};
enum { kHeaderBytes = 120, kDigestChars = 64, kGeometryOffset = 56 };

uint64_t gdn_oracle_capsule_bytes(uint32_t keys, uint32_t values, uint32_t rank,
                                  uint32_t updates) {
  const uint64_t k = keys, v = values;
  return kHeaderBytes + k * v + 4u * (k + v) + 4u * (uint64_t)rank * (k + v) +
         (uint64_t)updates * 4u * (2u * k + v) + kDigestChars;
}

static uint8_t* put_u32(uint8_t* p, uint32_t value) {
  for (int i = 0; i < 4; ++i) *p++ = (uint8_t)(value >> (8 * i));
  return p;
}

static uint8_t* put_u64(uint8_t* p, uint64_t value) {
  for (int i = 0; i < 8; ++i) *p++ = (uint8_t)(value >> (8 * i));
  return p;
}

static uint8_t* put_f32(uint8_t* p, float value) {
  uint32_t bits;
  memcpy(&bits, &value, 4);
  return put_u32(p, bits);
}

static uint8_t* put_floats(uint8_t* p, const float* values, uint64_t count) {
  for (uint64_t i = 0; i < count; ++i) p = put_f32(p, values[i]);
  return p;
}

static uint32_t get_u32(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
         ((uint32_t)p[3] << 24);
}

static uint64_t get_u64(const uint8_t* p) {
  return (uint64_t)get_u32(p) | ((uint64_t)get_u32(p + 4) << 32);
}

static float get_f32(const uint8_t* p) {
  const uint32_t bits = get_u32(p);
  float value;
  memcpy(&value, &bits, 4);
  return value;
}

uint64_t gdn_oracle_capsule_serialize(
    const char* geometry, uint64_t generation, uint64_t epoch, uint32_t keys,
    uint32_t values, uint32_t schema, uint32_t window, uint32_t rank, uint32_t bits,
    float smoothing_floor, const int8_t* residual, const float* smoothing,
    const float* scales, const float* comp_keys, const float* comp_values,
    uint32_t updates, const float* decay, const float* key, const float* correction,
    uint8_t* out) {
  uint8_t* p = out;
  memcpy(p, kMagic, 8);
  p += 8;
  p = put_u32(p, schema);
  p = put_u32(p, window);
  p = put_u32(p, rank);
  p = put_u32(p, bits);
  p = put_f32(p, smoothing_floor);
  p = put_u64(p, generation);
  p = put_u64(p, epoch);
  p = put_u32(p, keys);
  p = put_u32(p, values);
  p = put_u32(p, updates);
  memcpy(p, geometry, kDigestChars);
  p += kDigestChars;
  const uint64_t tile = (uint64_t)keys * values;
  memcpy(p, residual, tile);
  p += tile;
  p = put_floats(p, smoothing, keys);
  p = put_floats(p, scales, values);
  p = put_floats(p, comp_keys, (uint64_t)keys * rank);
  p = put_floats(p, comp_values, (uint64_t)values * rank);
  for (uint32_t u = 0; u < updates; ++u) {
    p = put_floats(p, decay + (uint64_t)u * keys, keys);
    p = put_floats(p, key + (uint64_t)u * keys, keys);
    p = put_floats(p, correction + (uint64_t)u * values, values);
  }
  gdn_oracle_sha256_hex(out, (uint64_t)(p - out), (char*)p);
  return (uint64_t)(p - out) + kDigestChars;
}

/* ---- Restore (state_capsule.cpp:476-578) ---------------------------------- */

static int lowercase_hex(const uint8_t* text) {
  for (int i = 0; i < kDigestChars; ++i) {
    const uint8_t c = text[i];
    if (!((c >= '0' && c <= '9') || (c >= 'a' && c <= 'f'))) return 0;
  }
  return 1;
}

static int all_finite(const float* values, uint64_t count) {
  for (uint64_t i = 0; i < count; ++i) {
    if (!isfinite(values[i])) return 0;
  }
  return 1;
}

/* ReadFloats (state_capsule.cpp:96-104): `count` floats at *offset of the
 * `content` bytes, or 0 when they do not fit. */
static int read_floats(const uint8_t* content, uint64_t content_size, uint64_t* offset,
                       float* out, uint64_t count) {
  const uint64_t available = content_size - (*offset < content_size ? *offset : content_size);
  if (count > available / 4u) return 0;
  for (uint64_t i = 0; i < count; ++i) out[i] = get_f32(content + *offset + 4u * i);
  *offset += 4u * count;
  return 1;
}

int gdn_oracle_capsule_restore(
    const uint8_t* encoded, uint64_t size, const char* geometry, uint64_t generation,
    uint64_t epoch, uint32_t keys, uint32_t values, uint32_t schema, uint32_t window,
    uint32_t rank, uint32_t bits, float smoothing_floor, uint32_t expected_position,
    int8_t* residual, float* smoothing, float* scales, float* comp_keys,
    float* comp_values, float* decay, float* key, float* correction,
    float* dense_work, uint32_t* updates_out) {
  /* ValidateIdentity / ValidateParameters of the expected values (:26-48). */
  if (!lowercase_hex((const uint8_t*)geometry) || generation == 0 || epoch == 0 ||
      keys == 0 || values == 0 || schema != 1 || window != 16 || rank != 4 ||
      bits != 8 || !isfinite(smoothing_floor) || !(smoothing_floor > 0.0f)) {
    return GDN_ORACLE_CAPSULE_ARGUMENT;
  }
  if (size < sizeof(kMagic) + kDigestChars) return GDN_ORACLE_CAPSULE_TRUNCATED;
  if (memcmp(encoded, kMagic, 8) != 0) return GDN_ORACLE_CAPSULE_MAGIC;
  const uint64_t content_size = size - kDigestChars;
  if (!lowercase_hex(encoded + content_size)) return GDN_ORACLE_CAPSULE_DIGEST_ENCODING;
  char digest[kDigestChars];
  gdn_oracle_sha256_hex(encoded, content_size, digest);
  if (memcmp(digest, encoded + content_size, kDigestChars) != 0) {
    return GDN_ORACLE_CAPSULE_DIGEST_MISMATCH;
  }
  /* The header integers are read from the whole encoding (digest included);
   * size >= 72 > 56 so they never run out.  The geometry digest must lie in
   * the content. */
  if (content_size < kHeaderBytes) return GDN_ORACLE_CAPSULE_TRUNCATED;
  const uint32_t got_schema = get_u32(encoded + 8);
  const uint32_t got_window = get_u32(encoded + 12);
  const uint32_t got_rank = get_u32(encoded + 16);
  const uint32_t got_bits = get_u32(encoded + 20);
  const float got_floor = get_f32(encoded + 24);
  const uint64_t got_generation = get_u64(encoded + 28);
  const uint64_t got_epoch = get_u64(encoded + 36);
  const uint32_t got_keys = get_u32(encoded + 44);
  const uint32_t got_values = get_u32(encoded + 48);
  const uint32_t count = get_u32(encoded + 52);
  if (got_schema != schema || got_window != window || got_rank != rank ||
      got_bits != bits || !(got_floor == smoothing_floor)) {
    return GDN_ORACLE_CAPSULE_PARAMETERS;
  }
  if (memcmp(encoded + kGeometryOffset, geometry, kDigestChars) != 0 ||
      got_generation != generation || got_epoch != epoch || got_keys != keys ||
      got_values != values) {
    return GDN_ORACLE_CAPSULE_IDENTITY;
  }
  if (rank > (keys < values ? keys : values)) return GDN_ORACLE_CAPSULE_RANK;
  if (count >= window) return GDN_ORACLE_CAPSULE_POSITION;
  if (count != expected_position) return GDN_ORACLE_CAPSULE_PHASE;

  uint64_t offset = kHeaderBytes;
  const uint64_t tile = (uint64_t)keys * values;
  if (content_size - offset < tile) return GDN_ORACLE_CAPSULE_TRUNCATED;
  for (uint64_t i = 0; i < tile; ++i) {
    if (encoded[offset + i] == 0x80u) return GDN_ORACLE_CAPSULE_RESIDUAL_DOMAIN;
  }
  memcpy(residual, encoded + offset, tile);
  offset += tile;
  if (!read_floats(encoded, content_size, &offset, smoothing, keys) ||
      !read_floats(encoded, content_size, &offset, scales, values) ||
      !read_floats(encoded, content_size, &offset, comp_keys, (uint64_t)keys * rank) ||
      !read_floats(encoded, content_size, &offset, comp_values, (uint64_t)values * rank)) {
    return GDN_ORACLE_CAPSULE_TRUNCATED;
  }
  int payload = all_finite(smoothing, keys) && all_finite(scales, values) &&
                all_finite(comp_keys, (uint64_t)keys * rank) &&
                all_finite(comp_values, (uint64_t)values * rank);
  for (uint32_t k = 0; payload && k < keys; ++k) payload = smoothing[k] > 0.0f;
  for (uint32_t v = 0; payload && v < values; ++v) payload = scales[v] >= 0.0f;
  if (!payload) return GDN_ORACLE_CAPSULE_BOUNDARY_PAYLOAD;
  for (uint32_t u = 0; u < count; ++u) {
    float* d = decay + (uint64_t)u * keys;
    float* k = key + (uint64_t)u * keys;
    float* c = correction + (uint64_t)u * values;
    if (!read_floats(encoded, content_size, &offset, d, keys) ||
        !read_floats(encoded, content_size, &offset, k, keys) ||
        !read_floats(encoded, content_size, &offset, c, values)) {
      return GDN_ORACLE_CAPSULE_TRUNCATED;
    }
    if (!all_finite(d, keys) || !all_finite(k, keys) || !all_finite(c, values)) {
      return GDN_ORACLE_CAPSULE_RECORD_NONFINITE;
    }
  }
  if (offset != content_size) return GDN_ORACLE_CAPSULE_TRAILING;
  gdn_oracle_dense_state(residual, smoothing, scales, comp_keys, comp_values, keys,
                         values, rank, decay, key, correction, count, dense_work);
  if (!all_finite(dense_work, tile)) return GDN_ORACLE_CAPSULE_STATE_NONFINITE;
  *updates_out = count;
  return GDN_ORACLE_CAPSULE_OK;
}

/* ---- device window slot <-> capsule --------------------------------------- */

enum { DIM = 128, RANK = 4, WINDOW = 16 };
static const float kSmoothingFloor = 1.0e-8f;

uint64_t gdn_oracle_slot_capsule_bytes(uint32_t position) {
  return position < WINDOW ? gdn_oracle_capsule_bytes(DIM, DIM, RANK, position) : 0;
}

/* The capsule of one slot state: codes transposed to the capsule's [key][value]
 * order, fp16 compensators and records widened exactly to fp32, and each
 * record's scalar gate repeated over the keys (the per-key decay the capsule
 * stores, state_capsule.cpp:365, 382-393). */
uint64_t gdn_oracle_slot_capsule_serialize(
    uint32_t layout, const int8_t* residual, const float* smoothing, const float* scales,
    const uint16_t* comp_keys, const uint16_t* comp_values, const float* record_decay,
    const uint16_t* record_keys, const uint16_t* record_corrections, uint32_t position,
    const char* geometry, uint64_t generation, uint64_t epoch, uint8_t* out) {
  if (position >= WINDOW) return 0;
  /* Per-thread scratch: callers serialize from several threads at once. */
  static _Thread_local int8_t codes[DIM * DIM];
  static _Thread_local float ck[DIM * RANK], cv[DIM * RANK];
  static _Thread_local float decay[WINDOW * DIM], key[WINDOW * DIM], correction[WINDOW * DIM];
  for (int k = 0; k < DIM; ++k) {
    for (int v = 0; v < DIM; ++v) {
      codes[k * DIM + v] = layout == GDN_ORACLE_LAYOUT_VALUE_KEY ? residual[v * DIM + k]
                                                                 : residual[k * DIM + v];
    }
  }
  for (int i = 0; i < DIM * RANK; ++i) {
    ck[i] = gdn_oracle_f16_to_f32(comp_keys[i]);
    cv[i] = gdn_oracle_f16_to_f32(comp_values[i]);
  }
  for (uint32_t j = 0; j < position; ++j) {
    for (int i = 0; i < DIM; ++i) {
      decay[j * DIM + i] = record_decay[j];
      key[j * DIM + i] = gdn_oracle_f16_to_f32(record_keys[j * DIM + i]);
      correction[j * DIM + i] = gdn_oracle_f16_to_f32(record_corrections[j * DIM + i]);
    }
  }
  return gdn_oracle_capsule_serialize(geometry, generation, epoch, DIM, DIM, 1, WINDOW, RANK,
                                      8, kSmoothingFloor, codes, smoothing, scales, ck, cv,
                                      position, decay, key, correction, out);
}

static int half_exact(float value, uint16_t* bits) {
  *bits = gdn_oracle_f32_to_f16(value);
  const float back = gdn_oracle_f16_to_f32(*bits);
  return memcmp(&back, &value, 4) == 0;
}

int gdn_oracle_slot_capsule_restore(
    const uint8_t* encoded, uint64_t size, const char* geometry, uint64_t generation,
    uint64_t epoch, uint32_t expected_position, uint32_t layout, int8_t* residual,
    float* smoothing, float* scales, uint16_t* comp_keys, uint16_t* comp_values,
    float* record_decay, uint16_t* record_keys, uint16_t* record_corrections,
    uint32_t* position_word) {
  /* Per-thread scratch: callers restore from several threads at once. */
  static _Thread_local int8_t codes[DIM * DIM];
  static _Thread_local float sm[DIM], sc[DIM], ck[DIM * RANK], cv[DIM * RANK], dense[DIM * DIM];
  static _Thread_local float decay[WINDOW * DIM], key[WINDOW * DIM], correction[WINDOW * DIM];
  static _Thread_local uint16_t ck16[DIM * RANK], cv16[DIM * RANK], key16[WINDOW * DIM],
      correction16[WINDOW * DIM];
  uint32_t count = 0;
  const int status = gdn_oracle_capsule_restore(
      encoded, size, geometry, generation, epoch, DIM, DIM, 1, WINDOW, RANK, 8,
      kSmoothingFloor, expected_position, codes, sm, sc, ck, cv, decay, key, correction,
      dense, &count);
  if (status != GDN_ORACLE_CAPSULE_OK) return status;
  /* The slot holds one gate per record and fp16 compensators and records: a
   * capsule outside that format is refused rather than rounded. */
  for (int i = 0; i < DIM * RANK; ++i) {
    if (!half_exact(ck[i], &ck16[i]) || !half_exact(cv[i], &cv16[i])) {
      return GDN_ORACLE_CAPSULE_DEVICE_FORMAT;
    }
  }
  for (uint32_t j = 0; j < count; ++j) {
    for (int i = 0; i < DIM; ++i) {
      if (memcmp(&decay[j * DIM + i], &decay[j * DIM], 4) != 0 ||
          !half_exact(key[j * DIM + i], &key16[j * DIM + i]) ||
          !half_exact(correction[j * DIM + i], &correction16[j * DIM + i])) {
        return GDN_ORACLE_CAPSULE_DEVICE_FORMAT;
      }
    }
  }
  for (int k = 0; k < DIM; ++k) {
    for (int v = 0; v < DIM; ++v) {
      if (layout == GDN_ORACLE_LAYOUT_VALUE_KEY) {
        residual[v * DIM + k] = codes[k * DIM + v];
      } else {
        residual[k * DIM + v] = codes[k * DIM + v];
      }
    }
  }
  memcpy(smoothing, sm, sizeof(sm));
  memcpy(scales, sc, sizeof(sc));
  memcpy(comp_keys, ck16, sizeof(ck16));
  memcpy(comp_values, cv16, sizeof(cv16));
  for (uint32_t j = 0; j < count; ++j) {
    record_decay[j] = decay[j * DIM];
    memcpy(record_keys + j * DIM, key16 + j * DIM, DIM * sizeof(uint16_t));
    memcpy(record_corrections + j * DIM, correction16 + j * DIM, DIM * sizeof(uint16_t));
  }
  *position_word = count;
  return GDN_ORACLE_CAPSULE_OK;
}
