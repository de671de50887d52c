// Host build of gdn-state-codec_amd/csrc/codec_math.h, checked against IEEE
// division and std::lround (built and run by tests/test_codec_math.py).
//
//   codec_math_check div127          every float a with 2^-100 <= |a| <= 2^120
//                                    and a = +0: div_by_reciprocal(a, 127, RN(1/127))
//                                    == a / 127
//   codec_math_check divrandom N     N random divisors b in [2^-90, 2^90] x every
//                                    significand of a, exponents chosen so that
//                                    2^-120 <= |a/b| <= 2^120
//   codec_math_check refit           the quant-only refit's fast domain: divisors s
//                                    in [2^-20, 2^20] at its edges and around 1
//                                    (exponents -20, -19, -1, 0, 1, 19 with a
//                                    power-of-two, an all-ones and two random
//                                    significands, and s = 2^20) x every significand
//                                    of dividends at the domain's edges (|w| in
//                                    [2^-100, 2^-99) and [2^99, 2^100], both signs)
//   codec_math_check round           every float |x| <= 127: round_half_away_small(x)
//                                    == clamp(lroundf(x), -127, 127)
//   codec_math_check lift            the encoder's lifted codes: wherever
//                                    lift_fraction(code_lift(m, RN(127/scale))) >=
//                                    the margin, lifted_code (its floor) is
//                                    clamp(lround(RN(RN(m/scale)*127)), -127, 127);
//                                    every float m in [-scale, scale] for one
//                                    scale, random scales in [2^-90, 2^90] with
//                                    random m, and m within 200 ulps of every
//                                    tie (n + 0.5) * scale / 127.  The count of
//                                    values left to the exact path goes to stderr.
//   codec_math_check lift_refit      the same sweep against the refit re-encode's
//                                    rounding, trunc(RN(q +- 0.5)) clamped to +-127
//                                    (window_boundary.cpp:336-345)
//   codec_math_check wide_lift       the bf16 encoder's codes from the product
//                                    q0 = RN(r * RN(1/s)) of its input r: wherever
//                                    lift_fraction(wide_code_lift(q0,
//                                    RN(127/scale))) >= kWideLiftMargin, its floor
//                                    is clamp(lround(RN(RN(RN(r/s)/scale)*127)),
//                                    -127, 127); and r recovered from q0
//                                    (bf16_input_from_product) bit for bit, and
//                                    quotient_from_product(q0, r, ...) == RN(r/s);
//                                    16,384 random (s, scale) pairs over the fast
//                                    domains, scale the quotient of a random bf16
//                                    maximum, times every bf16 r with |RN(r/s)| <=
//                                    scale.  The count of values left to the exact
//                                    path goes to stderr.
//   codec_math_check order           xcd_contiguous_item (work_order.h) is a
//                                    bijection on 0 .. n-1 for every n up to
//                                    4096 and for the bench grids
// Prints "<checked> <failures>" and exits non-zero on any failure.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <cmath>
#include <thread>
#include <vector>

#include "codec_math.h"
#include "work_order.h"

namespace {

float from_bits(uint32_t u) {
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}
uint32_t to_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, sizeof u);
  return u;
}

std::atomic<uint64_t> checked{0}, failures{0};

template <typename Fn>
void parallel(uint64_t begin, uint64_t end, Fn fn) {
  const unsigned threads = std::max(1u, std::thread::hardware_concurrency());
  std::vector<std::thread> pool;
  for (unsigned t = 0; t < threads; ++t) {
    pool.emplace_back([=] {
      uint64_t local_checked = 0, local_failures = 0;
      for (uint64_t i = begin + t; i < end; i += threads) fn(i, local_checked, local_failures);
      checked += local_checked;
      failures += local_failures;
    });
  }
  for (auto& th : pool) th.join();
}

void check_div127() {
  const float b = 127.0f;
  const float y = 1.0f / b;
  // biased exponents 27 (2^-100) .. 247 (2^120), both signs, every significand.
  const uint64_t lo = static_cast<uint64_t>(27) << 23;
  const uint64_t hi = static_cast<uint64_t>(248) << 23;
  parallel(lo, hi, [&](uint64_t u, uint64_t& n, uint64_t& bad) {
    for (uint32_t sign = 0; sign < 2; ++sign) {
      const float a = from_bits(static_cast<uint32_t>(u) | (sign << 31));
      ++n;
      if (to_bits(gdn::div_by_reciprocal(a, b, y)) != to_bits(a / b)) ++bad;
    }
  });
  checked += 1;
  if (to_bits(gdn::div_by_reciprocal(0.0f, b, y)) != to_bits(0.0f / b)) ++failures;
}

// div_by_127 (the two-part reciprocal) against IEEE a / 127 over the same
// exponent range as check_div127, plus both zeros.
void check_div127_split() {
  const uint64_t lo = static_cast<uint64_t>(27) << 23;
  const uint64_t hi = static_cast<uint64_t>(248) << 23;
  parallel(lo, hi, [&](uint64_t u, uint64_t& n, uint64_t& bad) {
    for (uint32_t sign = 0; sign < 2; ++sign) {
      const float a = from_bits(static_cast<uint32_t>(u) | (sign << 31));
      ++n;
      if (to_bits(gdn::div_by_127(a)) != to_bits(a / 127.0f)) ++bad;
    }
  });
  for (const float a : {0.0f, -0.0f}) {
    ++checked;
    if (to_bits(gdn::div_by_127(a)) != to_bits(a / 127.0f)) ++failures;
  }
}

void check_div_random(int divisors) {
  srand(12345);
  for (int d = 0; d < divisors; ++d) {
    const uint32_t exponent = 127 - 90 + static_cast<uint32_t>(rand() % 181);
    const uint32_t mantissa = ((static_cast<uint32_t>(rand()) << 12) ^ rand()) & 0x7FFFFFu;
    const float b = from_bits((exponent << 23) | mantissa);
    const float y = 1.0f / b;
    // a exponent: pick one keeping |a| in [2^-100, 2^120] and |a/b| in range.
    const int eb = static_cast<int>(exponent) - 127;
    int ea = eb + (rand() % 61) - 30;
    if (ea < -100) ea = -100;
    if (ea > 119) ea = 119;
    const uint32_t abits = static_cast<uint32_t>(ea + 127) << 23;
    parallel(0, 1u << 23, [&](uint64_t m, uint64_t& n, uint64_t& bad) {
      for (uint32_t step = 0; step < 2; ++step) {
        const float a = from_bits(abits + (step << 23) + static_cast<uint32_t>(m));
        ++n;
        if (to_bits(gdn::div_by_reciprocal(a, b, y)) != to_bits(a / b)) ++bad;
      }
    });
  }
}

void check_refit_domain() {
  std::vector<float> divisors;
  srand(20261202);
  for (int e : {-20, -19, -1, 0, 1, 19}) {
    const uint32_t exponent = static_cast<uint32_t>(e + 127) << 23;
    for (uint32_t mantissa : {0u, 0x7FFFFFu,
                              ((static_cast<uint32_t>(rand()) << 12) ^ rand()) & 0x7FFFFFu,
                              ((static_cast<uint32_t>(rand()) << 12) ^ rand()) & 0x7FFFFFu}) {
      divisors.push_back(from_bits(exponent | mantissa));
    }
  }
  divisors.push_back(1048576.0f);  // s = 2^20, the top of the domain
  for (const float b : divisors) {
    const float y = 1.0f / b;
    // |w| in [2^-100, 2^-99) and [2^99, 2^100): every significand, both signs.
    for (const uint32_t biased : {27u, 226u}) {
      parallel(0, 1u << 23, [&](uint64_t m, uint64_t& n, uint64_t& bad) {
        for (uint32_t sign = 0; sign < 2; ++sign) {
          const float a = from_bits((sign << 31) | (biased << 23) | static_cast<uint32_t>(m));
          ++n;
          if (to_bits(gdn::div_by_reciprocal(a, b, y)) != to_bits(a / b)) ++bad;
        }
      });
    }
    for (const float a : {0x1p100f, -0x1p100f}) {  // the top edge itself
      ++checked;
      if (to_bits(gdn::div_by_reciprocal(a, b, y)) != to_bits(a / b)) ++failures;
    }
  }
}

void check_round() {
  const uint64_t end = static_cast<uint64_t>(to_bits(127.0f)) + 1;
  parallel(0, end, [&](uint64_t u, uint64_t& n, uint64_t& bad) {
    for (uint32_t sign = 0; sign < 2; ++sign) {
      const float x = from_bits(static_cast<uint32_t>(u) | (sign << 31));
      long expect = lroundf(x);
      if (expect < -127) expect = -127;
      if (expect > 127) expect = 127;
      ++n;
      if (gdn::round_half_away_small(x) != expect) ++bad;
    }
  });
}

std::atomic<uint64_t> lift_fallbacks{0};

// One lifted code against the reference expression; returns false on a
// mismatch (a value whose lift fraction is below the margin is not a mismatch:
// the kernel recomputes it exactly).
// The expected code: the codec's clamp(lround(q)) or, with refit_rounding,
// the refit re-encode's trunc(q +- 0.5) with the addition rounded to float
// (window_boundary.cpp:336-345), q = RN(RN(m / scale) * 127) in both.
bool refit_rounding = false;

bool lift_matches(float m, float scale, float factor, uint64_t& fallbacks) {
  const float u = gdn::code_lift(m, factor);
  if (!(gdn::lift_fraction(u) >= gdn::kCodeLiftMargin)) {
    ++fallbacks;
    return true;
  }
  const float scaled = scale == 0.0f ? 0.0f : m / scale * gdn::kQuantizedMaximum;
  long expect;
  if (refit_rounding) {
    volatile float q = scaled;
    q = q + (q >= 0.0f ? 0.5f : -0.5f);
    float r = q;
    r = r > 127.0f ? 127.0f : r;
    r = r < -127.0f ? -127.0f : r;
    expect = static_cast<long>(static_cast<int>(r));
  } else {
    expect = lroundf(scaled);
    if (expect < -127) expect = -127;
    if (expect > 127) expect = 127;
  }
  return gdn::lifted_code(u) == expect;
}

void check_lift_scale(float scale) {
  const float factor = gdn::kQuantizedMaximum / scale;
  const uint64_t end = static_cast<uint64_t>(to_bits(scale)) + 1;
  parallel(0, end, [&](uint64_t u, uint64_t& n, uint64_t& bad) {
    uint64_t fb = 0;
    for (uint32_t sign = 0; sign < 2; ++sign) {
      const float m = from_bits(static_cast<uint32_t>(u) | (sign << 31));
      ++n;
      if (!lift_matches(m, scale, factor, fb)) ++bad;
    }
    lift_fallbacks += fb;
  });
}

uint32_t random_u32(uint64_t& state) {  // xorshift64*
  state ^= state >> 12;
  state ^= state << 25;
  state ^= state >> 27;
  return static_cast<uint32_t>((state * 0x2545F4914F6CDD1DULL) >> 32);
}

void check_lift() {
  check_lift_scale(0.78539819f);
  // Random scales over the fast domain; random m by bit pattern and by value,
  // and m within 200 ulps of every tie point.
  parallel(0, 2048, [&](uint64_t d, uint64_t& n, uint64_t& bad) {
    uint64_t fb = 0;
    uint64_t state = 0x9E3779B97F4A7C15ULL * (d + 1);
    const uint32_t exponent = 127 - 90 + random_u32(state) % 181;
    const float scale = from_bits((exponent << 23) | (random_u32(state) & 0x7FFFFFu));
    const float factor = gdn::kQuantizedMaximum / scale;
    for (int i = 0; i < 200000; ++i) {
      const uint32_t bits = random_u32(state) % (to_bits(scale) + 1);
      const float by_bits = from_bits(bits | ((random_u32(state) & 1u) << 31));
      const float by_value = scale * (static_cast<float>(random_u32(state) >> 8) * 0x1p-24f) *
                             ((random_u32(state) & 1u) ? -1.0f : 1.0f);
      n += 2;
      if (!lift_matches(by_bits, scale, factor, fb)) ++bad;
      if (fabsf(by_value) <= scale && !lift_matches(by_value, scale, factor, fb)) ++bad;
    }
    for (int k = 0; k < 127; ++k) {
      const float tie = (static_cast<float>(k) + 0.5f) / gdn::kQuantizedMaximum * scale;
      for (int step = -200; step <= 200; ++step) {
        const float m = from_bits(static_cast<uint32_t>(static_cast<int64_t>(to_bits(tie)) + step));
        if (!(m <= scale)) continue;
        n += 2;
        if (!lift_matches(m, scale, factor, fb)) ++bad;
        if (!lift_matches(-m, scale, factor, fb)) ++bad;
      }
    }
    lift_fallbacks += fb;
  });
  // scale == 0: factor 0 and m == 0 give code 0.
  uint64_t fb = 0;
  checked += 2;
  if (!lift_matches(0.0f, 0.0f, 0.0f, fb)) ++failures;
  if (!lift_matches(-0.0f, 0.0f, 0.0f, fb)) ++failures;
  lift_fallbacks += fb;
  fprintf(stderr, "fallbacks %llu\n", static_cast<unsigned long long>(lift_fallbacks.load()));
}

// The bf16 encoder's direct lift (codec_math.h, wide_code_lift) against the
// reference chain on every bf16 input of random (s, scale) pairs, with the
// exact path's recovery of r and of m from the kept product.  s is drawn
// over [2^-14, 2^20] (the smoothing's fast-division domain; s >= sqrt(1e-8)),
// the scale is |RN(R / s)| for a random bf16 R chosen so that it lies in
// [2^-90, 2^90], and r runs over every finite bf16 with |r| >= 2^-100 or
// r = 0 and |RN(r / s)| <= scale, as in a tile whose maximum is R.
void check_wide_lift() {
  std::atomic<uint64_t> fallbacks{0};
  parallel(0, 16384, [&](uint64_t d, uint64_t& n, uint64_t& bad) {
    uint64_t state = 0xD1B54A32D192ED03ULL * (d + 7);
    const uint32_t s_exp = 127 - 14 + random_u32(state) % 35;
    const float s = from_bits((s_exp << 23) | (random_u32(state) & 0x7FFFFFu));
    const float y = 1.0f / s;
    float scale = 0.0f;
    while (!(scale >= 0x1p-90f && scale <= 0x1p90f)) {
      const uint32_t r_exp = 127 - 100 + random_u32(state) % 200;
      const float big = from_bits((r_exp << 23) | ((random_u32(state) & 0x7Fu) << 16));
      scale = fabsf(big / s);
    }
    const float factor = gdn::kQuantizedMaximum / scale;
    uint64_t fb = 0;
    for (uint32_t h = 0; h < 0x10000u; ++h) {
      const float r = from_bits(h << 16);
      if (!std::isfinite(r) || (r != 0.0f && fabsf(r) < 0x1p-100f)) continue;
      const float m = r / s;
      if (!(fabsf(m) <= scale)) continue;
      ++n;
      const float q0 = r * y;
      const float back = gdn::bf16_input_from_product(q0, s);
      if (memcmp(&back, &r, sizeof(r)) != 0) ++bad;
      if (!(gdn::quotient_from_product(q0, r, s, y) == m)) ++bad;
      const float u = gdn::wide_code_lift(q0, factor);
      if (!(gdn::lift_fraction(u) >= gdn::kWideLiftMargin)) {
        ++fb;
        continue;
      }
      const float q = m / scale;
      long expect = lroundf(q * gdn::kQuantizedMaximum);
      if (expect < -127) expect = -127;
      if (expect > 127) expect = 127;
      if (gdn::lifted_code(u) != expect) ++bad;
    }
    fallbacks += fb;
  });
  fprintf(stderr, "fallbacks %llu\n", static_cast<unsigned long long>(fallbacks.load()));
}

void check_order_grid(uint64_t blocks) {
  std::vector<uint8_t> seen(blocks, 0);
  bool ok = true;
  for (uint64_t b = 0; b < blocks; ++b) {
    const uint64_t item = gdn::xcd_contiguous_item(b, blocks);
    if (item >= blocks || seen[item]) {
      ok = false;
      break;
    }
    seen[item] = 1;
  }
  ++checked;
  if (!ok) ++failures;
}

void check_order() {
  for (uint64_t n = 1; n <= 4096; ++n) check_order_grid(n);
  // configs 2 and 5 (tiles), 3 and 4 (workgroups), odd sizes near them
  for (uint64_t n : {245760ull, 491520ull, 2048ull, 8192ull, 245759ull, 245761ull, 491527ull}) {
    check_order_grid(n);
  }
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) return 2;
  if (strcmp(argv[1], "div127") == 0) {
    check_div127();
  } else if (strcmp(argv[1], "div127split") == 0) {
    check_div127_split();
  } else if (strcmp(argv[1], "divrandom") == 0) {
    check_div_random(argc > 2 ? atoi(argv[2]) : 64);
  } else if (strcmp(argv[1], "refit") == 0) {
    check_refit_domain();
  } else if (strcmp(argv[1], "round") == 0) {
    check_round();
  } else if (strcmp(argv[1], "lift") == 0) {
    check_lift();
  } else if (strcmp(argv[1], "wide_lift") == 0) {
    check_wide_lift();
  } else if (strcmp(argv[1], "lift_refit") == 0) {
    refit_rounding = true;
    check_lift();
  } else if (strcmp(argv[1], "order") == 0) {
    check_order();
  } else {
    return 2;
  }
  printf("%llu %llu\n", static_cast<unsigned long long>(checked.load()),
         static_cast<unsigned long long>(failures.load()));
  return failures.load() == 0 ? 0 : 1;
}
