// TEST INFRASTRUCTURE. Oracle-side dtype conversions and threefry, written independently of
// the product's (kurumi_amd/csrc/ir/dtype.h, device prelude): bf16 from f32 follows the
// half crate's shift-and-round-bit formulation; f16/bf16 from f64 round once on the f64 bit
// pattern; e4m3/e5m2 pick the nearest representable code by search (ties to the even code).
//
// Reference semantics restated: kurumi_core/src/dtype/convert.rs:14-70 (every cast through
// f64), dtype/traits/elem.rs:31-45 (per-dtype from_f64: ints `as` = truncate + saturate,
// NaN -> 0; f8 = from_f32(x as f32)), rng.rs:10-31 (threefry2x32-20, uniform_f32).
#include <cmath>
#include <cstring>
#include <limits>

#include "oracle.h"

namespace kuo {

static uint32_t fbits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
static float bitsf(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }

uint16_t f32_to_bf16(float f) {
  uint32_t x = fbits(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((x >> 16) | 0x0040u);
  const uint32_t rb = 0x00008000u;
  uint16_t hi = static_cast<uint16_t>(x >> 16);
  if ((x & rb) != 0 && (x & (3 * rb - 1)) != 0) hi = static_cast<uint16_t>(hi + 1);
  return hi;
}
float bf16_to_f32(uint16_t h) { return bitsf(static_cast<uint32_t>(h) << 16); }

// Round a double to a binary format with `eb` exponent / `mb` mantissa bits (IEEE style,
// with infinities), nearest-even, on the f64 bit pattern.
static uint32_t round_f64_ieee(double x, int eb, int mb) {
  uint64_t u;
  std::memcpy(&u, &x, 8);
  uint32_t sign = static_cast<uint32_t>(u >> 63) << (eb + mb);
  int exp = static_cast<int>((u >> 52) & 0x7ff);
  uint64_t man = u & ((1ull << 52) - 1);
  uint32_t expall = (1u << eb) - 1;
  if (exp == 0x7ff) {
    // NaN: quiet bit set, the top mb mantissa bits kept (half 2.7.1 f64_to_f16_fallback)
    if (man) return sign | (expall << mb) | (1u << (mb - 1)) | static_cast<uint32_t>(man >> (52 - mb));
    return sign | (expall << mb);
  }
  if (exp == 0) return sign;  // f64 subnormals are far below every target's range
  int bias = (1 << (eb - 1)) - 1;
  int te = exp - 1023 + bias;
  if (te >= static_cast<int>(expall)) return sign | (expall << mb);
  uint64_t M = man | (1ull << 52);
  int shift = 52 - mb;
  uint32_t exp_field = static_cast<uint32_t>(te);
  if (te <= 0) {
    shift += 1 - te;
    exp_field = 0;
    if (shift > 60) return sign;
  }
  uint64_t q = M >> shift;
  uint64_t rem = M & ((1ull << shift) - 1);
  uint64_t half = 1ull << (shift - 1);
  if (rem > half || (rem == half && (q & 1))) q += 1;
  uint64_t r;
  if (exp_field == 0) r = q;  // subnormal (carry into the min normal works out)
  else r = (static_cast<uint64_t>(exp_field) << mb) + (q - (1ull << mb));
  if (r >= (static_cast<uint64_t>(expall) << mb)) return sign | (expall << mb);
  return sign | static_cast<uint32_t>(r);
}

static double decode_ieee(uint32_t b, int eb, int mb) {
  int bias = (1 << (eb - 1)) - 1;
  uint32_t expall = (1u << eb) - 1;
  bool neg = (b >> (eb + mb)) & 1u;
  uint32_t e = (b >> mb) & expall, m = b & ((1u << mb) - 1);
  double v;
  if (e == expall && m) {
    // NaN keeps sign and payload, quiet bit set (half 2.7.1 f16_to_f64_fallback)
    uint64_t bits = (static_cast<uint64_t>(neg) << 63) | 0x7ff8000000000000ull | (static_cast<uint64_t>(m) << (52 - mb));
    double d;
    std::memcpy(&d, &bits, 8);
    return d;
  }
  if (e == expall) v = INFINITY;
  else if (e == 0) v = std::ldexp(static_cast<double>(m), 1 - bias - mb);
  else v = std::ldexp(1.0 + static_cast<double>(m) / (1u << mb), static_cast<int>(e) - bias);
  return neg ? -v : v;
}

uint16_t f64_to_f16(double x) { return static_cast<uint16_t>(round_f64_ieee(x, 5, 10)); }
double f16_to_f64(uint16_t h) { return decode_ieee(h, 5, 10); }
uint16_t f64_to_bf16(double x) {
  if (std::isnan(x)) return f32_to_bf16(static_cast<float>(x));
  return static_cast<uint16_t>(round_f64_ieee(x, 8, 7));
}

// OCP OFP8: E4M3FN (bias 7, no inf, NaN = S.1111.111, max 448), E5M2 (IEEE-like).
double e4m3_to_f64(uint8_t b) {
  uint32_t e = (b >> 3) & 15u, m = b & 7u;
  double v;
  if (e == 15 && m == 7) v = std::numeric_limits<double>::quiet_NaN();
  else if (e == 0) v = std::ldexp(static_cast<double>(m), -9);
  else v = std::ldexp(1.0 + m / 8.0, static_cast<int>(e) - 7);
  return (b & 0x80) ? -v : v;
}
double e5m2_to_f64(uint8_t b) { return decode_ieee(b, 5, 2); }

// nearest code among ascending non-negative codes [0, top], ties to the even code
static uint8_t nearest_code(double a, int top, double (*dec)(uint8_t)) {
  int lo = 0, hi = top;
  while (hi - lo > 1) {
    int mid = (lo + hi) / 2;
    if (dec(static_cast<uint8_t>(mid)) <= a) lo = mid;
    else hi = mid;
  }
  double dl = a - dec(static_cast<uint8_t>(lo)), dh = dec(static_cast<uint8_t>(hi)) - a;
  if (dl < 0) return static_cast<uint8_t>(lo);
  if (dh < 0) return static_cast<uint8_t>(hi);
  if (dl < dh) return static_cast<uint8_t>(lo);
  if (dh < dl) return static_cast<uint8_t>(hi);
  return static_cast<uint8_t>((lo & 1) ? hi : lo);
}

uint8_t f32_to_e4m3(float x) {
  uint8_t s = std::signbit(x) ? 0x80 : 0;
  if (std::isnan(x)) return s | 0x7f;
  double a = std::fabs(static_cast<double>(x));
  if (a >= 448.0) return s | 0x7e;  // saturating (inf included)
  return s | nearest_code(a, 0x7e, e4m3_to_f64);
}
uint8_t f32_to_e5m2(float x) {
  uint8_t s = std::signbit(x) ? 0x80 : 0;
  if (std::isnan(x)) return s | 0x7e;
  double a = std::fabs(static_cast<double>(x));
  if (a >= 61440.0) return s | 0x7c;  // RNE overflow to inf
  return s | nearest_code(a, 0x7b, e5m2_to_f64);
}

uint64_t threefry2x32(uint64_t key, uint64_t counter) {
  static const uint32_t rot[8] = {13, 15, 26, 6, 17, 29, 16, 24};
  uint32_t ks[3] = {static_cast<uint32_t>(key), static_cast<uint32_t>(key >> 32), 0};
  ks[2] = 0x1BD11BDAu ^ ks[0] ^ ks[1];
  uint32_t x0 = static_cast<uint32_t>(counter) + ks[0];
  uint32_t x1 = static_cast<uint32_t>(counter >> 32) + ks[1];
  for (uint32_t r = 0; r < 20; ++r) {
    x0 += x1;
    uint32_t k = rot[r % 8];
    x1 = (x1 << k) | (x1 >> (32 - k));
    x1 ^= x0;
    if (r % 4 == 3) {
      uint32_t inj = r / 4 + 1;
      x0 += ks[inj % 3];
      x1 += ks[(inj + 1) % 3] + inj;
    }
  }
  return static_cast<uint64_t>(x0) | (static_cast<uint64_t>(x1) << 32);
}

float uniform_f32(uint64_t bits) {
  return static_cast<float>(static_cast<uint32_t>(bits) >> 8) / static_cast<float>(1u << 24);
}

}  // namespace kuo
