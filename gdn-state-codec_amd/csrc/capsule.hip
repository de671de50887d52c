// LQCAPS01 capsules of device window slots (include/gdn_state_codec_capsule.h).
//
// Serialize = capsule_pack_kernel (one 256-thread workgroup per state: header,
// codes transposed to the capsule's [key][value] order through LDS, fp16 ->
// fp32 widening of compensators and records; coalesced 4/8-byte stores) then
// capsule_digest_kernel<false> (one lane per capsule: SHA-256 of the content,
// written as 64 lowercase hex characters after it).
//
// Restore = capsule_digest_kernel<true> (extent, length, magic, digest
// encoding and digest checks; one lane per capsule) then capsule_unpack_kernel
// (one workgroup per state: the remaining checks of
// GdnStateCodecCapsule::Restore in the reference's order -- parameters,
// identity, window position and phase, codes != -128, boundary payload,
// records, trailing bytes, a finite DenseState -- then the fp16 device-format
// check, and only then the slot writes).
//
// SHA-256 is a serial chain per message (FIPS 180-4 section 6.2), so the
// digest kernel gives each capsule one lane and is bound by integer VALU
// issue, not HBM: a producer wavefront expands each 64-byte block's message
// schedule and the consumer's round chain is about 900 VALU instructions per
// block.  The pack and unpack kernels move 22-45 KB per state and are
// HBM-bound.
#include <hip/hip_runtime.h>
#include <float.h>
#include <stdint.h>
#include <string.h>

#include "gdn_state_codec_capsule.h"
#include "launch.h"
#include "window_common.h"

namespace gdn {
namespace {

// Capsule layout of a 128x128 rank-4 slot state (state_capsule.cpp:446-474).
constexpr uint32_t kDigestChars = 64;
constexpr uint32_t kHeaderWords = 30;
constexpr uint32_t kResidualOffset = 4 * kHeaderWords;                      // 120
constexpr uint32_t kSmoothingOffset = kResidualOffset + kTile;              // 16504
constexpr uint32_t kScalesOffset = kSmoothingOffset + 4 * kDim;             // 17016
constexpr uint32_t kCompKeysOffset = kScalesOffset + 4 * kDim;              // 17528
constexpr uint32_t kCompValuesOffset = kCompKeysOffset + 4 * kDim * kRank;  // 19576
constexpr uint32_t kRecordsOffset = kCompValuesOffset + 4 * kDim * kRank;   // 21624
constexpr uint32_t kRecordFloats = 3 * kDim;  // decay[K], key[K], correction[V]
constexpr uint32_t kRecordBytes = 4 * kRecordFloats;                        // 1536
constexpr uint32_t kMinimumCapsule = 8 + kDigestChars;  // magic + digest
constexpr uint64_t kMagicWord = 0x313053504143514Cull;  // "LQCAPS01" little-endian
constexpr float kSmoothingFloor = 1.0e-8f;

__host__ __device__ constexpr uint32_t content_bytes(uint32_t position) {
  return kRecordsOffset + kRecordBytes * position;
}

static_assert(content_bytes(0) + kDigestChars == 21688, "capsule size");
static_assert(content_bytes(0) % 64 == 56, "the digest tail spans two blocks");

constexpr int kThreads = 256;
constexpr int kDigestLanes = 64;                 // capsules per digest workgroup
constexpr int kDigestThreads = 2 * kDigestLanes;  // producer + consumer wavefront

// The expected / written identity, as kernel-argument words.
struct Identity {
  uint32_t geometry[16];  // 64 hex characters, 4 per word, little-endian
  uint64_t generation;
  uint64_t epoch;
};

// ---- SHA-256 (FIPS 180-4) -------------------------------------------------

// First 32 bits of the fractional parts of the cube roots of the first 64
// primes (section 4.2.2) and of the square roots of the first 8 (5.3.3).
__device__ constexpr uint32_t kRound[64] = {
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
__device__ constexpr uint32_t kInitial[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u,
                                             0xa54ff53au, 0x510e527fu, 0x9b05688cu,
                                             0x1f83d9abu, 0x5be0cd19u};

__device__ __forceinline__ uint32_t rotr(uint32_t x, uint32_t n) {
  return __builtin_amdgcn_alignbit(x, x, n);
}

__device__ __forceinline__ uint32_t big_endian(uint32_t x) { return __builtin_bswap32(x); }

// Three-input bitwise functions as one gfx950 v_bitop3_b32 each; the table is
// the function's value on (x, y, z) = (0xF0, 0xCC, 0xAA).
__device__ __forceinline__ uint32_t xor3(uint32_t x, uint32_t y, uint32_t z) {
  return __builtin_amdgcn_bitop3_b32(x, y, z, 0x96);  // x ^ y ^ z
}
__device__ __forceinline__ uint32_t choose(uint32_t x, uint32_t y, uint32_t z) {
  return __builtin_amdgcn_bitop3_b32(x, y, z, 0xCA);  // (x & y) ^ (~x & z)
}
__device__ __forceinline__ uint32_t majority(uint32_t x, uint32_t y, uint32_t z) {
  return __builtin_amdgcn_bitop3_b32(x, y, z, 0xE8);  // (x&y) ^ (x&z) ^ (y&z)
}

// Block `block` of the padded message of content[0, size) (FIPS 180-4
// section 5.1.1: the bytes, 0x80, zeros, the 64-bit big-endian bit length) as
// 16 big-endian words.  Full blocks come from `full_words` (the caller's
// prefetched loads); the tail reads aligned words and may read up to 3 bytes
// past `size`, which the caller guarantees lie inside the capsule (the digest
// follows the content).
__device__ __forceinline__ void message_block(const uint8_t* content, uint32_t size,
                                              uint32_t block, const uint64_t (&full_words)[8],
                                              uint32_t (&w)[16]) {
  const uint32_t full = size / 64;
  if (block < full) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      w[2 * i] = big_endian(static_cast<uint32_t>(full_words[i]));
      w[2 * i + 1] = big_endian(static_cast<uint32_t>(full_words[i] >> 32));
    }
    return;
  }
  const uint32_t rest = size - 64 * full;
  const uint64_t bits = static_cast<uint64_t>(size) * 8u;
  if (block == full) {
    const uint32_t* tail = reinterpret_cast<const uint32_t*>(content + 64 * full);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t start = 4u * i;
      uint32_t word = 0;
      if (start + 4 <= rest) {
        word = big_endian(tail[i]);
      } else if (start < rest) {
        const uint32_t keep = rest - start;  // 1..3 message bytes in this word
        word = (big_endian(tail[i]) & (0xFFFFFFFFu << (8 * (4 - keep)))) |
               (0x80u << (8 * (3 - keep)));
      } else if (start == rest) {
        word = 0x80000000u;
      }
      w[i] = word;
    }
    if (rest <= 55) {
      w[14] = static_cast<uint32_t>(bits >> 32);
      w[15] = static_cast<uint32_t>(bits);
    }
  } else {  // the length block after a tail of more than 55 bytes
#pragma unroll
    for (int i = 0; i < 14; ++i) w[i] = 0;
    w[14] = static_cast<uint32_t>(bits >> 32);
    w[15] = static_cast<uint32_t>(bits);
  }
}

// Compression blocks of the padded message of `size` bytes.
__device__ __forceinline__ uint32_t message_blocks(uint32_t size) { return (size + 9 + 63) / 64; }

// 16 words of lowercase hex characters of the digest (the reference's
// Sha256Hex string, 4 characters per little-endian word).
__device__ __forceinline__ void digest_hex(const uint32_t (&h)[8], uint32_t (&hex)[16]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint32_t chars[2] = {0, 0};
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      const uint32_t nibble = (h[i] >> (28 - 4 * n)) & 15u;
      const uint32_t ch = nibble < 10 ? '0' + nibble : 'a' + nibble - 10;
      chars[n >> 2] |= ch << (8 * (n & 3));
    }
    hex[2 * i] = chars[0];
    hex[2 * i + 1] = chars[1];
  }
}

struct DigestArgs {
  uint8_t* capsules;
  const uint64_t* offsets;
  const uint32_t* lengths;
  uint64_t capacity;
  uint32_t* status;  // verify only
  uint32_t states;
};

// One workgroup hashes 64 capsules, one per lane, with two wavefronts: the
// producer loads each 64-byte block, expands the message schedule and writes
// K[t] + W[t] for the block's 64 rounds to a double-buffered LDS ring; the
// consumer runs only the round function from the ring (section 6.2.2), so
// the serial chain of each capsule carries about two thirds of the
// instructions of a full compression.  One barrier per block: the producer
// fills slot b + 1 while the consumer works on slot b, and a slot is
// refilled only after the barrier the consumer reaches when done with it.
//
// kVerify = false: write the digest of each serialized capsule (lengths[i] = 0
// marks a state the pack kernel skipped).  kVerify = true: the first checks of
// Restore (state_capsule.cpp:481-494), status[i] = 0 when they all pass.
template <bool kVerify>
__global__ __launch_bounds__(kDigestThreads) void capsule_digest_kernel(DigestArgs a) {
  __shared__ __align__(16) uint4 ring[2][16][kDigestLanes];  // [slot][round / 4][lane]
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const uint32_t s = blockIdx.x * kDigestLanes + lane;

  // Per-capsule checks, evaluated identically by both wavefronts so that
  // their block counts (and so their barrier counts) agree.
  uint32_t status = GDN_STATE_CODEC_CAPSULE_OK;
  bool hash = false;
  uint8_t* base = nullptr;
  uint32_t content = 0;
  uint32_t recorded[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) recorded[i] = 0;
  if (s < a.states) {
    const uint64_t offset = a.offsets[s];
    const uint32_t length = a.lengths[s];
    hash = true;
    if constexpr (kVerify) {
      if ((offset & 7u) != 0 || offset > a.capacity || length > a.capacity - offset) {
        status = GDN_STATE_CODEC_CAPSULE_EXTENT;
        hash = false;
      } else if (length < kMinimumCapsule) {
        status = GDN_STATE_CODEC_CAPSULE_TRUNCATED;
        hash = false;
      }
    } else {
      hash = length != 0;
    }
    if (hash) {
      base = a.capsules + offset;
      content = length - kDigestChars;
      if constexpr (kVerify) {
        if (*reinterpret_cast<const uint64_t*>(base) != kMagicWord) {
          status = GDN_STATE_CODEC_CAPSULE_MAGIC;
          hash = false;
        } else {
          bool lowercase_hex = true;
#pragma unroll
          for (int i = 0; i < 64; ++i) {
            const uint32_t ch = base[content + i];
            lowercase_hex = lowercase_hex && (ch - '0' < 10u || ch - 'a' < 6u);
            recorded[i >> 2] |= ch << (8 * (i & 3));
          }
          if (!lowercase_hex) {
            status = GDN_STATE_CODEC_CAPSULE_DIGEST_ENCODING;
            hash = false;
          }
        }
      }
    }
  }
  const uint32_t blocks = hash ? message_blocks(content) : 0u;
  uint32_t wave_blocks = blocks;
#pragma unroll
  for (int mask = 32; mask >= 1; mask >>= 1) {
    const uint32_t other = __shfl_xor(wave_blocks, mask);
    wave_blocks = other > wave_blocks ? other : wave_blocks;
  }

  if (wave == 0) {
    // ---- producer: message schedule plus round constants ----
    const uint32_t full = content / 64;
    const uint64_t* src = reinterpret_cast<const uint64_t*>(base);
    uint64_t next[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) next[i] = 0;
    if (full > 0) {
#pragma unroll
      for (int i = 0; i < 8; ++i) next[i] = src[i];
    }
    for (uint32_t block = 0; block < wave_blocks; ++block) {
      if (block < blocks) {
        uint32_t w[16];
        message_block(base, content, block, next, w);
        // Issue the next block's loads before this block's schedule.
        if (block + 1 < full) {
#pragma unroll
          for (int i = 0; i < 8; ++i) next[i] = src[8 * (block + 1) + i];
        }
        uint4* slot = &ring[block & 1][0][0];
        uint32_t group[4];
#pragma unroll
        for (int t = 0; t < 64; ++t) {
          uint32_t wt;
          if (t < 16) {
            wt = w[t];
          } else {
            const uint32_t w15 = w[(t - 15) & 15];
            const uint32_t w2 = w[(t - 2) & 15];
            const uint32_t s0 = xor3(rotr(w15, 7), rotr(w15, 18), w15 >> 3);
            const uint32_t s1 = xor3(rotr(w2, 17), rotr(w2, 19), w2 >> 10);
            wt = w[t & 15] + s0 + w[(t - 7) & 15] + s1;
            w[t & 15] = wt;
          }
          group[t & 3] = kRound[t] + wt;
          if ((t & 3) == 3) {
            slot[(t >> 2) * kDigestLanes + lane] = make_uint4(group[0], group[1], group[2], group[3]);
          }
        }
      }
      __syncthreads();  // slot (block & 1) is ready
    }
    return;
  }

  // ---- consumer: the round chain ----
  uint32_t h[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = kInitial[i];
  for (uint32_t block = 0; block < wave_blocks; ++block) {
    __syncthreads();  // slot (block & 1) is ready
    if (block < blocks) {
      const uint4* slot = &ring[block & 1][0][0];
      uint32_t va = h[0], vb = h[1], vc = h[2], vd = h[3], ve = h[4], vf = h[5], vg = h[6],
               vh = h[7];
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const uint4 kw4 = slot[q * kDigestLanes + lane];
        const uint32_t kw[4] = {kw4.x, kw4.y, kw4.z, kw4.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t t1 = vh + xor3(rotr(ve, 6), rotr(ve, 11), rotr(ve, 25)) +
                              choose(ve, vf, vg) + kw[i];
          const uint32_t t2 = xor3(rotr(va, 2), rotr(va, 13), rotr(va, 22)) + majority(va, vb, vc);
          vh = vg;
          vg = vf;
          vf = ve;
          ve = vd + t1;
          vd = vc;
          vc = vb;
          vb = va;
          va = t1 + t2;
        }
      }
      h[0] += va;
      h[1] += vb;
      h[2] += vc;
      h[3] += vd;
      h[4] += ve;
      h[5] += vf;
      h[6] += vg;
      h[7] += vh;
    }
  }
  if (s >= a.states) return;
  if (!hash) {
    if constexpr (kVerify) a.status[s] = status;
    return;
  }
  uint32_t hex[16];
  digest_hex(h, hex);
  if constexpr (kVerify) {
    bool same = true;
#pragma unroll
    for (int i = 0; i < 16; ++i) same = same && recorded[i] == hex[i];
    a.status[s] = same ? GDN_STATE_CODEC_CAPSULE_OK : GDN_STATE_CODEC_CAPSULE_DIGEST_MISMATCH;
  } else {
    // Serialized content is a multiple of 8 bytes long.
    uint64_t* out = reinterpret_cast<uint64_t*>(base + content);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      out[i] = static_cast<uint64_t>(hex[2 * i]) | (static_cast<uint64_t>(hex[2 * i + 1]) << 32);
    }
  }
}

// ---- serialize: pack the content ------------------------------------------

struct PackArgs {
  const int8_t* residual;
  const float* smoothing;
  const float* scales;
  const uint16_t* comp_keys;
  const uint16_t* comp_values;
  const float* record_decay;
  const uint16_t* record_keys;
  const uint16_t* record_corrections;
  const uint32_t* positions;
  uint8_t* capsules;
  const uint64_t* offsets;
  uint64_t capacity;
  uint32_t* lengths;
  uint32_t layout;
  uint32_t states;
  Identity identity;
};

// Transpose staging: 128 rows of 128 code bytes at a 132-byte stride, so the
// column reads of 8 consecutive rows fall in different LDS banks.
constexpr int kTileStride = kDim + 4;

// Record floats of records 0..14 as float2 pairs, spread over the workgroup:
// pair u is handled by thread u % 256 in slot u / 256.  A wavefront's 64 pairs
// are one 128-float vector (decay, key or correction of one record), so every
// per-vector quantity is wave-uniform.
constexpr int kRecordPairSlots = ((kWindow - 1) * kRecordFloats / 2 + kThreads - 1) / kThreads;
static_assert(kRecordFloats / 2 % 64 == 0, "a record is whole wavefronts of pairs");

__device__ __forceinline__ uint32_t header_word(int t, uint32_t position, const Identity& id) {
  switch (t) {
    case 0: return static_cast<uint32_t>(kMagicWord);
    case 1: return static_cast<uint32_t>(kMagicWord >> 32);
    case 2: return 1;        // schema_version
    case 3: return kWindow;  // window_size
    case 4: return kRank;    // compensator_rank
    case 5: return 8;        // quant_bits
    case 6: return __float_as_uint(kSmoothingFloor);
    case 7: return static_cast<uint32_t>(id.generation);
    case 8: return static_cast<uint32_t>(id.generation >> 32);
    case 9: return static_cast<uint32_t>(id.epoch);
    case 10: return static_cast<uint32_t>(id.epoch >> 32);
    case 11: return kDim;  // key_dimension
    case 12: return kDim;  // value_dimension
    case 13: return position;
    default: return id.geometry[t - 14];
  }
}

__global__ __launch_bounds__(kThreads) void capsule_pack_kernel(PackArgs a) {
  __shared__ __align__(16) uint8_t tile[kDim * kTileStride];
  const uint32_t s = blockIdx.x;
  const int t = threadIdx.x;
  const uint32_t position = a.positions[static_cast<uint64_t>(s) * kPositionStride];
  const uint64_t offset = a.offsets[s];
  const uint64_t bytes = static_cast<uint64_t>(content_bytes(position)) + kDigestChars;
  if (position >= kWindow || (offset & 7u) != 0 || offset > a.capacity ||
      bytes > a.capacity - offset) {
    if (t == 0) a.lengths[s] = 0;
    return;
  }
  uint8_t* out = a.capsules + offset;

  // Every load first: smoothing then scales (one float per thread), the
  // compensators (two fp16 each), the records as 32-bit words (pair u of the
  // capsule's record floats: a gate, or two fp16 keys or corrections), then
  // the codes.
  const float value = t < kDim ? a.smoothing[static_cast<uint64_t>(s) * kDim + t]
                               : a.scales[static_cast<uint64_t>(s) * kDim + t - kDim];
  const uint64_t comp_base = static_cast<uint64_t>(s) * kDim * kRank;
  const uint32_t keys = reinterpret_cast<const uint32_t*>(a.comp_keys + comp_base)[t];
  const uint32_t values = reinterpret_cast<const uint32_t*>(a.comp_values + comp_base)[t];
  const uint64_t record_base = static_cast<uint64_t>(s) * kWindow;
  const uint32_t record_pairs = kRecordFloats / 2 * position;  // a multiple of 64
  uint32_t rec[kRecordPairSlots];
#pragma unroll
  for (int i = 0; i < kRecordPairSlots; ++i) {
    const uint32_t u = i * kThreads + t;
    rec[i] = 0;
    if (u < record_pairs) {  // uniform over the wavefront, as is the vector
      const uint32_t j = u / (kRecordFloats / 2), pair = u - j * (kRecordFloats / 2);
      if (pair < kDim / 2) {
        rec[i] = __float_as_uint(a.record_decay[record_base + j]);
      } else if (pair < kDim) {
        rec[i] = reinterpret_cast<const uint32_t*>(a.record_keys + (record_base + j) * kDim)[pair - kDim / 2];
      } else {
        rec[i] = reinterpret_cast<const uint32_t*>(a.record_corrections + (record_base + j) * kDim)[pair - kDim];
      }
    }
  }
  // Codes: [value][key] rows to transpose (thread = half a row), or
  // [key][value] words copied as they are.
  const int8_t* codes = a.residual + static_cast<uint64_t>(s) * kTile;
  uint4 row_part[4];
  uint64_t words[8];
  if (a.layout == kValueKey) {
    const uint4* src = reinterpret_cast<const uint4*>(codes + (t >> 1) * kDim + (t & 1) * 64);
#pragma unroll
    for (int i = 0; i < 4; ++i) row_part[i] = src[i];
  } else {
    const uint64_t* src = reinterpret_cast<const uint64_t*>(codes);
#pragma unroll
    for (int i = 0; i < 8; ++i) words[i] = src[i * kThreads + t];
  }
  // Keep the stores below from being scheduled between the loads.
  __builtin_amdgcn_sched_barrier(0);

  if (t < static_cast<int>(kHeaderWords)) {
    *reinterpret_cast<uint32_t*>(out + 4 * t) = header_word(t, position, a.identity);
  }
  *reinterpret_cast<float*>(out + kSmoothingOffset + 4 * t) = value;
  reinterpret_cast<float2*>(out + kCompKeysOffset)[t] =
      make_float2(half_bits_to_float(keys & 0xFFFFu), half_bits_to_float(keys >> 16));
  reinterpret_cast<float2*>(out + kCompValuesOffset)[t] =
      make_float2(half_bits_to_float(values & 0xFFFFu), half_bits_to_float(values >> 16));
  // Records 0..p-1: {gate repeated over the keys, key, correction}.
  float2* records = reinterpret_cast<float2*>(out + kRecordsOffset);
#pragma unroll
  for (int i = 0; i < kRecordPairSlots; ++i) {
    const uint32_t u = i * kThreads + t;
    if (u < record_pairs) {
      const bool gate = (u / 64) % 3 == 0;
      records[u] = gate ? make_float2(__uint_as_float(rec[i]), __uint_as_float(rec[i]))
                        : make_float2(half_bits_to_float(rec[i] & 0xFFFFu),
                                      half_bits_to_float(rec[i] >> 16));
    }
  }
  // Codes in [key][value] order: 2048 8-byte words, word w = 16 k + v / 8.
  uint64_t* residual_out = reinterpret_cast<uint64_t*>(out + kResidualOffset);
  if (a.layout == kValueKey) {
    const int row = t >> 1, half = t & 1;  // source row = value
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t* dst = reinterpret_cast<uint32_t*>(tile + row * kTileStride + half * 64 + 16 * i);
      dst[0] = row_part[i].x;
      dst[1] = row_part[i].y;
      dst[2] = row_part[i].z;
      dst[3] = row_part[i].w;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int w = i * kThreads + t;
      const int k = w >> 4, v0 = (w & 15) * 8;
      uint64_t word = 0;
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        word |= static_cast<uint64_t>(tile[(v0 + b) * kTileStride + k]) << (8 * b);
      }
      residual_out[w] = word;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) residual_out[i * kThreads + t] = words[i];
  }
  if (t == 0) a.lengths[s] = static_cast<uint32_t>(bytes);
}

// ---- restore: validate and unpack -----------------------------------------

struct UnpackArgs {
  const uint8_t* capsules;
  const uint64_t* offsets;
  const uint32_t* lengths;
  const uint32_t* expected_positions;
  int8_t* residual;
  float* smoothing;
  float* scales;
  uint16_t* comp_keys;
  uint16_t* comp_values;
  float* record_decay;
  uint16_t* record_keys;
  uint16_t* record_corrections;
  uint32_t* positions;
  uint32_t* status;
  uint32_t layout;
  uint32_t states;
  Identity identity;
};

__device__ __forceinline__ bool has_byte_0x80(uint64_t x) {
  // A byte equals 0x80 iff (byte ^ 0x80) == 0.
  const uint64_t y = x ^ 0x8080808080808080ull;
  return ((y - 0x0101010101010101ull) & ~y & 0x8080808080808080ull) != 0;
}

__device__ __forceinline__ bool half_exact(float x) {
  const uint32_t back = __float_as_uint(half_bits_to_float(float_to_half_bits(x)));
  return back == __float_as_uint(x);
}

// Maximum over the wavefront of non-negative float bits, in every lane.
__device__ __forceinline__ uint32_t wave_max_bits(uint32_t x) {
  // Row prefixes by DPP row shifts, then rows merged by row broadcasts: lane
  // 63 ends with the maximum.  A lane whose source is outside the row keeps
  // its own value (bound_ctrl off, old = x).
  x = max(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(x), static_cast<int>(x), 0x111, 0xF, 0xF, false)));
  x = max(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(x), static_cast<int>(x), 0x112, 0xF, 0xF, false)));
  x = max(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(x), static_cast<int>(x), 0x114, 0xF, 0xF, false)));
  x = max(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(x), static_cast<int>(x), 0x118, 0xF, 0xF, false)));
  x = max(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(x), static_cast<int>(x), 0x142, 0xA, 0xF, false)));
  x = max(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(x), static_cast<int>(x), 0x143, 0xC, 0xF, false)));
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x), 63));
}

__global__ __launch_bounds__(kThreads) void capsule_unpack_kernel(UnpackArgs a) {
  __shared__ uint32_t header[kHeaderWords];
  // |max| of smoothing, scales, ck, cv, then (decay, key, correction) of each
  // record, as float bits (non-negative floats order like their bits).
  __shared__ uint32_t maxima[4 + 3 * (kWindow - 1)];
  // flags[0]: bit 0 a code equals -128, bit 1 the boundary payload is invalid;
  // flags[1]: bit j record j holds a non-finite value.
  __shared__ uint32_t flags[2];
  __shared__ __align__(16) uint8_t tile[kDim * kTileStride];
  const uint32_t s = blockIdx.x;
  const int t = threadIdx.x;
  if (a.status[s] != GDN_STATE_CODEC_CAPSULE_OK) return;  // the digest kernel refused it
  const uint8_t* base = a.capsules + a.offsets[s];
  const uint32_t content = a.lengths[s] - kDigestChars;
  if (t < 2) flags[t] = 0u;
  if (t < 4 + 3 * (kWindow - 1)) maxima[t] = 0u;

  // Every load the checks and the slot writes need, issued together and held
  // in registers.  What is present depends only on the content length; which
  // of it counts is decided below.
  const bool has_header = content >= kResidualOffset;
  const bool has_codes = content >= kSmoothingOffset;
  const bool has_payload = content >= kRecordsOffset;
  const uint32_t whole = has_payload ? (content - kRecordsOffset) / kRecordBytes : 0u;
  const uint32_t loaded = whole < kWindow - 1 ? whole : kWindow - 1;
  const uint32_t loaded_pairs = kRecordFloats / 2 * loaded;  // a multiple of 64
  uint32_t header_bits = 0;
  if (has_header && t < static_cast<int>(kHeaderWords)) {
    header_bits = reinterpret_cast<const uint32_t*>(base)[t];
  }
  uint64_t codes[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) codes[i] = 0;
  if (has_codes) {
    const uint64_t* code_words = reinterpret_cast<const uint64_t*>(base + kResidualOffset);
#pragma unroll
    for (int i = 0; i < 8; ++i) codes[i] = code_words[i * kThreads + t];
  }
  // Thread t < 128 holds smoothing[t], the others scales[t - 128].
  float value = 0.0f;
  float2 key_pair = make_float2(0.0f, 0.0f), value_pair = make_float2(0.0f, 0.0f);
  float2 rec[kRecordPairSlots];
  if (has_payload) {
    value = *reinterpret_cast<const float*>(base + kSmoothingOffset + 4 * t);
    key_pair = reinterpret_cast<const float2*>(base + kCompKeysOffset)[t];
    value_pair = reinterpret_cast<const float2*>(base + kCompValuesOffset)[t];
  }
  const float2* record_pairs = reinterpret_cast<const float2*>(base + kRecordsOffset);
#pragma unroll
  for (int i = 0; i < kRecordPairSlots; ++i) {
    const uint32_t u = i * kThreads + t;
    rec[i] = u < loaded_pairs ? record_pairs[u] : make_float2(0.0f, 0.0f);
  }
  // Keep the checks below from being scheduled between the loads.
  __builtin_amdgcn_sched_barrier(0);

  if (has_header && t < static_cast<int>(kHeaderWords)) header[t] = header_bits;
  bool minus128 = false;
#pragma unroll
  for (int i = 0; i < 8; ++i) minus128 = minus128 || has_byte_0x80(codes[i]);
  bool payload_bad = false;
  const int lane = t & 63;
  __syncthreads();  // flags and maxima are clear
  // A wavefront's 64 magnitudes of one vector are reduced first, then merged
  // into the workgroup's slot by one atomic.
  const auto merge_max = [&](int slot, float magnitude) {
    const uint32_t m = wave_max_bits(__float_as_uint(magnitude));
    if (lane == 0) atomicMax(&maxima[slot], m);
  };
  if (has_payload) {
    payload_bad = t < kDim ? !(isfinite(value) && value > 0.0f) : !(isfinite(value) && value >= 0.0f);
    merge_max(t < kDim ? 0 : 1, fabsf(value));  // waves 0-1 smoothing, 2-3 scales
    payload_bad = payload_bad || !isfinite(key_pair.x) || !isfinite(key_pair.y) ||
                  !isfinite(value_pair.x) || !isfinite(value_pair.y);
    merge_max(2, fmaxf(fabsf(key_pair.x), fabsf(key_pair.y)));
    merge_max(3, fmaxf(fabsf(value_pair.x), fabsf(value_pair.y)));
#pragma unroll
    for (int i = 0; i < kRecordPairSlots; ++i) {
      const uint32_t u = i * kThreads + t;
      if (u < loaded_pairs) {  // uniform over the wavefront
        if (!isfinite(rec[i].x) || !isfinite(rec[i].y)) {
          atomicOr(&flags[1], 1u << (u / (kRecordFloats / 2)));
        }
        merge_max(4 + static_cast<int>(u / 64), fmaxf(fabsf(rec[i].x), fabsf(rec[i].y)));
      }
    }
  }
  if (minus128 || payload_bad) {
    atomicOr(&flags[0], (minus128 ? 1u : 0u) | (payload_bad ? 2u : 0u));
  }
  __syncthreads();

  // The checks of state_capsule.cpp:497-576 in their order; every value here
  // is uniform over the workgroup and the first failure names the outcome.
  uint32_t result = GDN_STATE_CODEC_CAPSULE_OK;
  uint32_t count = 0;
  if (!has_header) {
    result = GDN_STATE_CODEC_CAPSULE_TRUNCATED;  // geometry digest truncated (:509-511)
  } else {
    count = header[13];
    bool same = header[7] == static_cast<uint32_t>(a.identity.generation) &&
                header[8] == static_cast<uint32_t>(a.identity.generation >> 32) &&
                header[9] == static_cast<uint32_t>(a.identity.epoch) &&
                header[10] == static_cast<uint32_t>(a.identity.epoch >> 32) &&
                header[11] == kDim && header[12] == kDim;
#pragma unroll
    for (int i = 0; i < 16; ++i) same = same && header[14 + i] == a.identity.geometry[i];
    if (header[2] != 1 || header[3] != kWindow || header[4] != kRank || header[5] != 8 ||
        !(__uint_as_float(header[6]) == kSmoothingFloor)) {
      result = GDN_STATE_CODEC_CAPSULE_PARAMETERS;
    } else if (!same) {
      result = GDN_STATE_CODEC_CAPSULE_IDENTITY;
    } else if (count >= kWindow) {  // rank 4 <= min(128, 128) always holds
      result = GDN_STATE_CODEC_CAPSULE_POSITION;
    } else if (count != a.expected_positions[s]) {
      result = GDN_STATE_CODEC_CAPSULE_PHASE;
    } else if (!has_codes) {
      result = GDN_STATE_CODEC_CAPSULE_TRUNCATED;
    } else if (flags[0] & 1u) {
      result = GDN_STATE_CODEC_CAPSULE_RESIDUAL_DOMAIN;
    } else if (!has_payload) {
      result = GDN_STATE_CODEC_CAPSULE_TRUNCATED;
    } else if (flags[0] & 2u) {
      result = GDN_STATE_CODEC_CAPSULE_BOUNDARY_PAYLOAD;
    } else {
      // Records (:562-570): each is read whole, then checked; the first
      // record that runs past the content ends the restore as truncated.
      const uint32_t present = whole < count ? whole : count;
      if (flags[1] & ((1u << present) - 1u)) {
        result = GDN_STATE_CODEC_CAPSULE_RECORD_NONFINITE;
      } else if (present < count) {
        result = GDN_STATE_CODEC_CAPSULE_TRUNCATED;
      } else if (content != content_bytes(count)) {
        result = GDN_STATE_CODEC_CAPSULE_TRAILING;
      }
    }
  }
  if (result != GDN_STATE_CODEC_CAPSULE_OK) {
    if (t == 0) a.status[s] = result;
    return;
  }

  // DenseState (:337-352) must be finite.  A magnitude bound decides it for
  // almost every capsule: with B0 = max|s| max|scale| + 4 max|ck| max|cv| and
  // Bj = max|decay_j| B(j-1) + max|key_j| max|corr_j|, every value the
  // reference's fp32 evaluation forms after s*code is at most
  // B_p (1 + 2^-24)^40 in magnitude, so B_p and max|s| * 127 below
  // FLT_MAX (1 - 2^-10) prove the state finite.  Otherwise it is evaluated
  // exactly, in its own order, from the capsule's bytes: ((s*code)/127)*scale,
  // + ck.cv over the rank, then decay*x + key*corr per record (the build
  // disables contraction).
  const auto mx = [&](int slot) { return static_cast<double>(__uint_as_float(maxima[slot])); };
  double bound = mx(0) * mx(1) + 4.0 * mx(2) * mx(3);
  for (uint32_t j = 0; j < count; ++j) {
    bound = mx(4 + 3 * j) * bound + mx(5 + 3 * j) * mx(6 + 3 * j);
  }
  const double limit = static_cast<double>(FLT_MAX) * (1.0 - 1.0 / 1024.0);
  bool bad = false;
  if (!(bound < limit && mx(0) * 127.0 < limit)) {
    const float* sm = reinterpret_cast<const float*>(base + kSmoothingOffset);
    const float* sc = reinterpret_cast<const float*>(base + kScalesOffset);
    const float* ck = reinterpret_cast<const float*>(base + kCompKeysOffset);
    const float* cv = reinterpret_cast<const float*>(base + kCompValuesOffset);
    const float* records = reinterpret_cast<const float*>(base + kRecordsOffset);
    const int8_t* code_bytes = reinterpret_cast<const int8_t*>(base + kResidualOffset);
    // A rare path: one element at a time, in few registers.  Element b of
    // this thread's code word w is (key k, value v).
#pragma unroll 1
    for (int e = 0; e < 64; ++e) {
      const int w = (e >> 3) * kThreads + t, b = e & 7;
      const int k = w >> 4, v = (w & 15) * 8 + b;
      const float code = static_cast<float>(code_bytes[8 * w + b]);
      float x = sm[k] * code / 127.0f * sc[v];
#pragma unroll
      for (int r = 0; r < kRank; ++r) x += ck[k * kRank + r] * cv[v * kRank + r];
      for (uint32_t j = 0; j < count; ++j) {
        const float* r = records + j * kRecordFloats;
        x = r[k] * x + r[kDim + k] * r[2 * kDim + v];
      }
      bad = bad || !isfinite(x);
    }
    if (__syncthreads_or(bad)) {
      if (t == 0) a.status[s] = GDN_STATE_CODEC_CAPSULE_STATE_NONFINITE;
      return;
    }
  }
  // The slot's format: one gate per record, fp16 compensators and records.
  const uint32_t count_pairs = kRecordFloats / 2 * count;
  bad = !half_exact(key_pair.x) || !half_exact(key_pair.y) || !half_exact(value_pair.x) ||
        !half_exact(value_pair.y);
#pragma unroll
  for (int i = 0; i < kRecordPairSlots; ++i) {
    const uint32_t u = i * kThreads + t;
    if (u < count_pairs) {  // uniform over the wavefront, as is the vector
      if ((u / 64) % 3 == 0) {  // a decay vector: every value equals its first (lane 0's)
        const uint32_t first =
            static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(__float_as_uint(rec[i].x)), 0));
        bad = bad || __float_as_uint(rec[i].x) != first || __float_as_uint(rec[i].y) != first;
      } else {
        bad = bad || !half_exact(rec[i].x) || !half_exact(rec[i].y);
      }
    }
  }
  if (__syncthreads_or(bad)) {
    if (t == 0) a.status[s] = GDN_STATE_CODEC_CAPSULE_DEVICE_FORMAT;
    return;
  }
  // Admitted: write the slot.
  int8_t* residual = a.residual + static_cast<uint64_t>(s) * kTile;
  if (a.layout == kValueKey) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int w = i * kThreads + t;
      const int k = w >> 4, v0 = (w & 15) * 8;
      uint32_t* dst = reinterpret_cast<uint32_t*>(tile + k * kTileStride + v0);
      dst[0] = static_cast<uint32_t>(codes[i]);
      dst[1] = static_cast<uint32_t>(codes[i] >> 32);
    }
    __syncthreads();
    uint64_t* out = reinterpret_cast<uint64_t*>(residual);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int w = i * kThreads + t;
      const int v = w >> 4, k0 = (w & 15) * 8;
      uint64_t word = 0;
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        word |= static_cast<uint64_t>(tile[(k0 + b) * kTileStride + v]) << (8 * b);
      }
      out[w] = word;
    }
  } else {
    uint64_t* out = reinterpret_cast<uint64_t*>(residual);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i * kThreads + t] = codes[i];
  }
  if (t < kDim) {
    a.smoothing[static_cast<uint64_t>(s) * kDim + t] = value;
  } else {
    a.scales[static_cast<uint64_t>(s) * kDim + t - kDim] = value;
  }
  {
    const uint64_t comp_base = static_cast<uint64_t>(s) * kDim * kRank;
    reinterpret_cast<uint32_t*>(a.comp_keys + comp_base)[t] =
        float_to_half_bits(key_pair.x) | (float_to_half_bits(key_pair.y) << 16);
    reinterpret_cast<uint32_t*>(a.comp_values + comp_base)[t] =
        float_to_half_bits(value_pair.x) | (float_to_half_bits(value_pair.y) << 16);
  }
  // Records 0..p-1 from the registers: the gate once, keys and corrections
  // two fp16 values per 32-bit store.
  const uint64_t record_base = static_cast<uint64_t>(s) * kWindow;
#pragma unroll
  for (int i = 0; i < kRecordPairSlots; ++i) {
    const uint32_t u = i * kThreads + t;
    if (u < count_pairs) {
      const uint32_t j = u / (kRecordFloats / 2), pair = u - j * (kRecordFloats / 2);
      if (pair < kDim / 2) {
        if (pair == 0) a.record_decay[record_base + j] = rec[i].x;
      } else {
        const uint32_t bits = float_to_half_bits(rec[i].x) | (float_to_half_bits(rec[i].y) << 16);
        uint16_t* dst = pair < kDim ? a.record_keys + (record_base + j) * kDim + 2 * (pair - kDim / 2)
                                    : a.record_corrections + (record_base + j) * kDim +
                                          2 * (pair - kDim);
        *reinterpret_cast<uint32_t*>(dst) = bits;
      }
    }
  }
  if (t == 0) {
    a.positions[static_cast<uint64_t>(s) * kPositionStride] = count;
    a.status[s] = GDN_STATE_CODEC_CAPSULE_OK;
  }
}

// Host-side identity check (ValidateIdentity, state_capsule.cpp:40-48) and
// packing of the geometry digest into kernel-argument words.
bool make_identity(const char* geometry, uint64_t generation, uint64_t epoch, Identity* out) {
  if (geometry == nullptr || generation == 0 || epoch == 0) return false;
  for (int i = 0; i < 64; ++i) {
    const char c = geometry[i];
    if (!((c >= '0' && c <= '9') || (c >= 'a' && c <= 'f'))) return false;
  }
  memcpy(out->geometry, geometry, 64);
  out->generation = generation;
  out->epoch = epoch;
  return true;
}

uint32_t digest_blocks(uint32_t states) { return (states + kDigestLanes - 1) / kDigestLanes; }

}  // namespace
}  // namespace gdn

extern "C" uint64_t statecentric_gdn_state_codec_capsule_bytes_v1(uint32_t window_position) {
  return window_position < static_cast<uint32_t>(gdn::kWindow)
             ? static_cast<uint64_t>(gdn::content_bytes(window_position)) + gdn::kDigestChars
             : 0;
}

extern "C" int32_t statecentric_gdn_state_codec_capsule_serialize_launch_v1(
    void* stream, const int8_t* residual, const float* smoothing, const float* scales,
    const uint16_t* compensator_keys, const uint16_t* compensator_values,
    const float* record_decay, const uint16_t* record_keys,
    const uint16_t* record_corrections, const uint32_t* positions, uint32_t layout,
    const char* geometry_sha256, uint64_t generation, uint64_t epoch, uint8_t* capsules,
    const uint64_t* offsets, uint64_t capacity, uint32_t* lengths, uint32_t states) {
  gdn::PackArgs args{};
  if (!residual || !smoothing || !scales || !compensator_keys || !compensator_values ||
      !record_decay || !record_keys || !record_corrections || !positions || !capsules ||
      !offsets || !lengths || states == 0 || states > gdn::kMaxWindowStates ||
      (layout != gdn::kKeyValue && layout != gdn::kValueKey) ||
      !gdn::aligned16(residual, smoothing, scales, compensator_keys, compensator_values,
                      record_decay, record_keys, record_corrections, positions, capsules,
                      offsets, lengths) ||
      !gdn::make_identity(geometry_sha256, generation, epoch, &args.identity)) {
    return gdn::kStatusInvalidArgument;
  }
  args.residual = residual;
  args.smoothing = smoothing;
  args.scales = scales;
  args.comp_keys = compensator_keys;
  args.comp_values = compensator_values;
  args.record_decay = record_decay;
  args.record_keys = record_keys;
  args.record_corrections = record_corrections;
  args.positions = positions;
  args.capsules = capsules;
  args.offsets = offsets;
  args.capacity = capacity;
  args.lengths = lengths;
  args.layout = layout;
  args.states = states;
  int32_t status = gdn::launch(gdn::capsule_pack_kernel, dim3(states), dim3(gdn::kThreads),
                               stream, args);
  if (status != gdn::kStatusOk) return status;
  const gdn::DigestArgs digest{capsules, offsets, lengths, capacity, nullptr, states};
  return gdn::launch(gdn::capsule_digest_kernel<false>, dim3(gdn::digest_blocks(states)),
                     dim3(gdn::kDigestThreads), stream, digest);
}

extern "C" int32_t statecentric_gdn_state_codec_capsule_restore_launch_v1(
    void* stream, const uint8_t* capsules, const uint64_t* offsets, const uint32_t* lengths,
    uint64_t capacity, const char* geometry_sha256, uint64_t generation, uint64_t epoch,
    const uint32_t* expected_positions, uint32_t layout, int8_t* residual, float* smoothing,
    float* scales, uint16_t* compensator_keys, uint16_t* compensator_values,
    float* record_decay, uint16_t* record_keys, uint16_t* record_corrections,
    uint32_t* positions, uint32_t* status, uint32_t states) {
  gdn::UnpackArgs args{};
  if (!capsules || !offsets || !lengths || !expected_positions || !residual || !smoothing ||
      !scales || !compensator_keys || !compensator_values || !record_decay || !record_keys ||
      !record_corrections || !positions || !status || states == 0 ||
      states > gdn::kMaxWindowStates ||
      (layout != gdn::kKeyValue && layout != gdn::kValueKey) ||
      !gdn::aligned16(capsules, offsets, lengths, expected_positions, residual, smoothing,
                      scales, compensator_keys, compensator_values, record_decay, record_keys,
                      record_corrections, positions, status) ||
      !gdn::make_identity(geometry_sha256, generation, epoch, &args.identity)) {
    return gdn::kStatusInvalidArgument;
  }
  const gdn::DigestArgs digest{const_cast<uint8_t*>(capsules), offsets, lengths, capacity,
                               status, states};
  int32_t result = gdn::launch(gdn::capsule_digest_kernel<true>,
                               dim3(gdn::digest_blocks(states)), dim3(gdn::kDigestThreads),
                               stream, digest);
  if (result != gdn::kStatusOk) return result;
  args.capsules = capsules;
  args.offsets = offsets;
  args.lengths = lengths;
  args.expected_positions = expected_positions;
  args.residual = residual;
  args.smoothing = smoothing;
  args.scales = scales;
  args.comp_keys = compensator_keys;
  args.comp_values = compensator_values;
  args.record_decay = record_decay;
  args.record_keys = record_keys;
  args.record_corrections = record_corrections;
  args.positions = positions;
  args.status = status;
  args.layout = layout;
  args.states = states;
  return gdn::launch(gdn::capsule_unpack_kernel, dim3(states), dim3(gdn::kThreads), stream,
                     args);
}
