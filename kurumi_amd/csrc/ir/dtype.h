// Element dtypes of the kurumi IR and the host-side scalar conversions the graph
// builders need (a `scalar` constant is stored directly in the tensor's dtype).
//
// The tag order is the reference's `DType` declaration order
// (kurumi_core/src/dtype.rs:23-42), which is also the C ABI index (kurumi.h:29-34).
#pragma once
#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>

namespace ku {

enum class DType : uint32_t {
  BOOL = 0, U8, U16, U32, U64, I8, I16, I32, I64,
  F8E4M3, F8E5M2, F16, BF16, F32, F64, C64, C128,
};
constexpr uint32_t kNumDTypes = 17;

inline bool dt_is_float(DType d) {
  return d == DType::F8E4M3 || d == DType::F8E5M2 || d == DType::F16 || d == DType::BF16 ||
         d == DType::F32 || d == DType::F64;
}
inline bool dt_is_int(DType d) {
  return d >= DType::U8 && d <= DType::I64;
}
inline bool dt_is_complex(DType d) { return d == DType::C64 || d == DType::C128; }
inline bool dt_is_numeric(DType d) { return dt_is_int(d) || dt_is_float(d); }
inline bool dt_is_arith(DType d) { return dt_is_numeric(d) || dt_is_complex(d); }
inline bool dt_is_signed(DType d) {
  return dt_is_float(d) || d == DType::I8 || d == DType::I16 || d == DType::I32 || d == DType::I64;
}
inline bool dt_is_unsigned(DType d) { return d >= DType::U8 && d <= DType::U64; }
// f16/bf16/fp8: stored narrow, computed by upcasting to f32 and rounding back.
inline bool dt_is_lowp(DType d) {
  return d == DType::F8E4M3 || d == DType::F8E5M2 || d == DType::F16 || d == DType::BF16;
}

inline size_t dt_width(DType d) {
  switch (d) {
    case DType::BOOL: case DType::U8: case DType::I8: case DType::F8E4M3: case DType::F8E5M2: return 1;
    case DType::U16: case DType::I16: case DType::F16: case DType::BF16: return 2;
    case DType::U32: case DType::I32: case DType::F32: return 4;
    case DType::U64: case DType::I64: case DType::F64: case DType::C64: return 8;
    case DType::C128: return 16;
  }
  return 0;
}

inline const char* dt_name(DType d) {
  static const char* names[] = {"BOOL", "U8", "U16", "U32", "U64", "I8", "I16", "I32", "I64",
                                "F8E4M3", "F8E5M2", "F16", "BF16", "F32", "F64", "C64", "C128"};
  uint32_t i = static_cast<uint32_t>(d);
  return i < kNumDTypes ? names[i] : "?";
}

// ---- host scalar conversions (round-to-nearest-even, quiet NaN kept) ----

inline uint32_t f32_bits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
inline float bits_f32(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
inline uint64_t f64_bits(double f) { uint64_t u; std::memcpy(&u, &f, 8); return u; }
inline double bits_f64(uint64_t u) { double f; std::memcpy(&f, &u, 8); return f; }

inline uint16_t f32_to_bf16(float f) {
  uint32_t u = f32_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
inline float bf16_to_f32(uint16_t h) { return bits_f32(static_cast<uint32_t>(h) << 16); }

// Generic RNE encoder of a finite/inf/nan double into a small IEEE-like format with
// `eb` exponent bits and `mb` mantissa bits. `has_inf`: all-ones exponent is inf/nan
// (IEEE style); otherwise only S.1111.111 is NaN (OCP E4M3FN) and overflow saturates
// to the largest finite value. Returns the raw bit pattern (sign at bit eb+mb).
inline uint32_t encode_small_float(double x, int eb, int mb, bool has_inf) {
  const uint32_t sign = std::signbit(x) ? (1u << (eb + mb)) : 0u;
  const int bias = (1 << (eb - 1)) - 1;
  const uint32_t exp_all = (1u << eb) - 1;
  if (std::isnan(x)) {
    return has_inf ? (sign | (exp_all << mb) | (1u << (mb - 1))) : (sign | (exp_all << mb) | ((1u << mb) - 1));
  }
  double a = std::fabs(x);
  // largest finite
  double maxfin;
  if (has_inf) maxfin = std::ldexp(2.0 - std::ldexp(1.0, -mb), static_cast<int>(exp_all) - 1 - bias);
  else maxfin = std::ldexp(1.0 + (double)((1u << mb) - 2) / (double)(1u << mb), static_cast<int>(exp_all) - bias);
  if (std::isinf(a)) return has_inf ? (sign | (exp_all << mb)) : (sign | encode_small_float(maxfin, eb, mb, has_inf));
  if (a == 0.0) return sign;
  // quantum at this magnitude: normal if a >= 2^(1-bias)
  int e;
  std::frexp(a, &e);                 // a = m * 2^e, m in [0.5,1)
  int exp_unb = e - 1;               // a in [2^exp_unb, 2^(exp_unb+1))
  if (exp_unb < 1 - bias) exp_unb = 1 - bias;  // subnormal range shares the min quantum
  double q = std::ldexp(1.0, exp_unb - mb);
  double n = a / q;                  // exact (power-of-two scaling)
  double fl = std::floor(n);
  double rem = n - fl;
  if (rem > 0.5 || (rem == 0.5 && std::fmod(fl, 2.0) != 0.0)) fl += 1.0;
  double r = fl * q;
  if (r > maxfin) {
    if (has_inf) return sign | (exp_all << mb);
    r = maxfin;
  }
  // encode r exactly
  if (r < std::ldexp(1.0, 1 - bias)) {  // subnormal
    uint32_t mant = static_cast<uint32_t>(r / std::ldexp(1.0, 1 - bias - mb));
    return sign | mant;
  }
  int er;
  double mr = std::frexp(r, &er);    // r = mr * 2^er
  uint32_t biased = static_cast<uint32_t>(er - 1 + bias);
  uint32_t mant = static_cast<uint32_t>((mr * 2.0 - 1.0) * (double)(1u << mb));
  return sign | (biased << mb) | mant;
}

inline double decode_small_float(uint32_t b, int eb, int mb, bool has_inf) {
  const int bias = (1 << (eb - 1)) - 1;
  const uint32_t exp_all = (1u << eb) - 1;
  bool neg = (b >> (eb + mb)) & 1u;
  uint32_t ex = (b >> mb) & exp_all;
  uint32_t m = b & ((1u << mb) - 1);
  double v;
  if (has_inf && ex == exp_all) v = m ? NAN : INFINITY;
  else if (!has_inf && ex == exp_all && m == (1u << mb) - 1) v = NAN;
  else if (ex == 0) v = std::ldexp((double)m, 1 - bias - mb);
  else v = std::ldexp(1.0 + (double)m / (double)(1u << mb), (int)ex - bias);
  return neg ? -v : v;
}

inline uint16_t f64_to_f16(double x) { return static_cast<uint16_t>(encode_small_float(x, 5, 10, true)); }
inline double f16_to_f64(uint16_t h) { return decode_small_float(h, 5, 10, true); }
inline uint16_t f64_to_bf16(double x) {
  if (std::isnan(x)) return f32_to_bf16(static_cast<float>(x));
  return static_cast<uint16_t>(encode_small_float(x, 8, 7, true));
}
inline uint8_t f32_to_f8e4m3(float x) { return static_cast<uint8_t>(encode_small_float(x, 4, 3, false)); }
inline uint8_t f32_to_f8e5m2(float x) { return static_cast<uint8_t>(encode_small_float(x, 5, 2, true)); }
inline double f8e4m3_to_f64(uint8_t b) { return decode_small_float(b, 4, 3, false); }
inline double f8e5m2_to_f64(uint8_t b) { return decode_small_float(b, 5, 2, true); }

// Store a double into `dst` as dtype `d` with the reference's cast semantics
// (kurumi_core/src/dtype/convert.rs:14-70, dtype/traits/elem.rs:31-45): floats round
// to nearest even, floats -> ints truncate toward zero and saturate, NaN -> 0.
template <class I>
inline I sat_cast(double x) {
  if (std::isnan(x)) return 0;
  if (x <= (double)std::numeric_limits<I>::lowest()) return std::numeric_limits<I>::lowest();
  if (x >= (double)std::numeric_limits<I>::max()) return std::numeric_limits<I>::max();
  return static_cast<I>(x);
}

}  // namespace ku
