// Device-side helpers prepended to every generated region kernel (compiled by hipRTC
// for gfx950). Conversions follow the reference's cast semantics
// (kurumi_core/src/dtype/convert.rs:14-70, dtype/traits/elem.rs:31-45): round to nearest
// even, f64 sources rounded once (round-to-odd intermediate), e4m3 saturating to +-448,
// float -> int truncating and saturating with NaN -> 0. threefry2x32-20 is the reference
// RNG (kurumi_core/src/rng.rs:10-31).
#pragma once

namespace ku::hipbk {

inline const char* kDevicePrelude = R"KUPRELUDE(
#ifndef INFINITY
#define INFINITY __builtin_inff()
#endif
typedef unsigned char u8; typedef unsigned short u16; typedef unsigned int u32; typedef unsigned long long u64;
typedef signed char i8; typedef short i16; typedef int i32; typedef long long i64;
template <class T, int N> struct __attribute__((aligned(sizeof(T) * N))) VecT { T v[N]; };
#define KD __device__ __forceinline__
// non-temporal 16/8/4-byte vector accesses (streaming data that is touched once)
typedef u32 ku_u32x4 __attribute__((ext_vector_type(4)));
typedef u32 ku_u32x2 __attribute__((ext_vector_type(2)));
template <class V> KD V vld_nt(const V* p) {
  if constexpr (sizeof(V) == 16) return __builtin_bit_cast(V, __builtin_nontemporal_load((const ku_u32x4*)p));
  else if constexpr (sizeof(V) == 8) return __builtin_bit_cast(V, __builtin_nontemporal_load((const ku_u32x2*)p));
  else if constexpr (sizeof(V) == 4) return __builtin_bit_cast(V, __builtin_nontemporal_load((const u32*)p));
  else return *p;
}
template <class V> KD void vst_nt(V* p, const V& v) {
  if constexpr (sizeof(V) == 16) __builtin_nontemporal_store(__builtin_bit_cast(ku_u32x4, v), (ku_u32x4*)p);
  else if constexpr (sizeof(V) == 8) __builtin_nontemporal_store(__builtin_bit_cast(ku_u32x2, v), (ku_u32x2*)p);
  else if constexpr (sizeof(V) == 4) __builtin_nontemporal_store(__builtin_bit_cast(u32, v), (u32*)p);
  else *p = v;
}
KD float bf16_ld(u16 h) { return __uint_as_float(((u32)h) << 16); }
// v_cvt_pk_bf16_f32: round to nearest even, NaN quieted with its sign and top payload bits kept
// (the same result as the bit formula u + 0x7fff + lsb >> 16, NaN -> (u >> 16) | 0x40, for all
// 2^32 f32 inputs on gfx950)
KD u16 bf16_st(float f) { return __builtin_bit_cast(u16, (__bf16)f); }
typedef __bf16 ku_bf16x2 __attribute__((ext_vector_type(2)));
typedef float ku_f32x2 __attribute__((ext_vector_type(2)));
// f rounded to bf16, as an f32: v_cvt_pk_bf16_f32 with 0 as the low operand leaves bf16(f) in the
// high half over a zero low half, which is that value's f32 pattern (one instruction, no unpack)
KD float rbf16(float f) {
  return __uint_as_float(__builtin_bit_cast(u32, __builtin_convertvector((ku_f32x2){0.f, f}, ku_bf16x2)));
}
// two roundings: one instruction each (a shared v_cvt_pk_bf16_f32 would need two unpacks)
KD void rbf16x2(float& a, float& b) {
  a = rbf16(a);
  b = rbf16(b);
}
// bf16-exact floats (low 16 bits zero) -> two packed bf16 patterns
KD u32 pack_bf16_exact(float lo, float hi) { return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u); }
KD float quiet_nan(float f) { return f != f ? __uint_as_float(__float_as_uint(f) | 0x400000u) : f; }
KD float f16_ld(u16 h) { return (float)__builtin_bit_cast(_Float16, h); }
KD u16 f16_st(float f) { return __builtin_bit_cast(u16, (_Float16)f); }
KD float rf16(float f) { return (float)(_Float16)f; }
// f64 -> f32 rounded to odd: a later RNE to a narrower format then rounds exactly once
KD float f32_odd(double x) {
  float f = (float)x;
  if ((double)f != x && !(__float_as_uint(f) & 1u)) f = nextafterf(f, (double)f < x ? INFINITY : -INFINITY);
  return f;
}
KD float rbf16_d(double x) { return rbf16(f32_odd(x)); }
KD float rf16_d(double x) { return rf16(f32_odd(x)); }
// decodes: v_cvt_f32_fp8 / v_cvt_f32_bf8, NaN codes produced here (e4m3 S.1111.111 -> quiet NaN
// with the sign; e5m2 NaN keeps sign and payload, quiet bit set, like the half crate's f16 path)
KD float f8e4m3_ld(u8 b) {
  const float v = __builtin_amdgcn_cvt_f32_fp8((u32)b, 0);
  const float nan = __uint_as_float(((u32)(b & 0x80u) << 24) | 0x7fc00000u);
  return (b & 0x7fu) == 0x7fu ? nan : v;
}
// OCP e4m3: nearest even, saturating to +-448, NaN -> S.1111.111 (v_cvt_pk_fp8_f32 on the input
// clamped to +-448 gives the bit-level rounding's codes for all 2^32 f32 inputs on gfx950)
KD u8 f8e4m3_st(float x) {
  const u32 c = (u32)__builtin_amdgcn_cvt_pk_fp8_f32(__builtin_amdgcn_fmed3f(x, -448.f, 448.f), 0.f, 0, false) & 0xffu;
  const u32 nan = ((__float_as_uint(x) >> 24) & 0x80u) | 0x7fu;
  return (u8)(x != x ? nan : c);
}
KD float rf8e4m3(float x) { return f8e4m3_ld(f8e4m3_st(x)); }
KD float f8e5m2_ld(u8 b) {
  const float v = __builtin_amdgcn_cvt_f32_bf8((u32)b, 0);
  const float nan = __uint_as_float(((u32)(b & 0x80u) << 24) | 0x7fc00000u | ((u32)(b & 3u) << 21));
  return ((b & 0x7cu) == 0x7cu && (b & 3u)) ? nan : v;
}
// OCP e5m2: nearest even, overflow to inf, NaN -> S.11111.10 (v_cvt_pk_bf8_f32)
KD u8 f8e5m2_st(float x) {
  const u32 c = (u32)__builtin_amdgcn_cvt_pk_bf8_f32(x, 0.f, 0, false) & 0xffu;
  const u32 nan = ((__float_as_uint(x) >> 24) & 0x80u) | 0x7eu;
  return (u8)(x != x ? nan : c);
}
KD float rf8e5m2(float x) { return f8e5m2_ld(f8e5m2_st(x)); }
template <class I> KD I sat_int(double x);
#define KU_SAT(I, LO, HI) template <> KD I sat_int<I>(double x) { \
  if (x != x) return (I)0; if (x <= (double)(LO)) return (I)(LO); if (x >= (double)(HI)) return (I)(HI); return (I)x; }
KU_SAT(u8, 0, 255) KU_SAT(u16, 0, 65535) KU_SAT(u32, 0u, 4294967295u) KU_SAT(u64, 0ull, 18446744073709551615ull)
KU_SAT(i8, -128, 127) KU_SAT(i16, -32768, 32767) KU_SAT(i32, -2147483648ll, 2147483647ll)
KU_SAT(i64, (-9223372036854775807ll - 1), 9223372036854775807ll)
KD u32 rotl32(u32 x, u32 r) { return (x << r) | (x >> (32u - r)); }
KD u64 threefry2x32(u64 key, u64 ctr) {
  const u32 k0 = (u32)key, k1 = (u32)(key >> 32), k2 = 0x1BD11BDAu ^ k0 ^ k1;
  u32 x0 = (u32)ctr + k0, x1 = (u32)(ctr >> 32) + k1;
#define KU_TF(R) x0 += x1; x1 = rotl32(x1, R); x1 ^= x0;
#define KU_INJ(A, B, I) x0 += A; x1 += B + I;
  KU_TF(13) KU_TF(15) KU_TF(26) KU_TF(6) KU_INJ(k1, k2, 1u)
  KU_TF(17) KU_TF(29) KU_TF(16) KU_TF(24) KU_INJ(k2, k0, 2u)
  KU_TF(13) KU_TF(15) KU_TF(26) KU_TF(6) KU_INJ(k0, k1, 3u)
  KU_TF(17) KU_TF(29) KU_TF(16) KU_TF(24) KU_INJ(k1, k2, 4u)
  KU_TF(13) KU_TF(15) KU_TF(26) KU_TF(6) KU_INJ(k2, k0, 5u)
  return (u64)x0 | ((u64)x1 << 32);
}
KD float uniform_f32(u64 bits) { return (float)((u32)bits >> 8) / 16777216.f; }
KD float shx(float v, int m) { return __shfl_xor(v, m, 64); }
// wave64 reductions on DPP row shifts and row broadcasts (lane 63 ends with the total, which
// v_readlane hands to every lane): VALU latency instead of an LDS permute per step
template <int CTRL, int ROW_MASK> KD float dppf(float old, float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, v),
                                                                CTRL, ROW_MASK, 0xf, false));
}
KD float wave_sum(float v) {
  v += dppf<0x111, 0xf>(0.f, v);  // row_shr:1
  v += dppf<0x112, 0xf>(0.f, v);  // row_shr:2
  v += dppf<0x114, 0xf>(0.f, v);  // row_shr:4
  v += dppf<0x118, 0xf>(0.f, v);  // row_shr:8 -> lane 15 of each row holds the row
  v += dppf<0x142, 0xa>(0.f, v);  // row_bcast:15 into rows 1, 3
  v += dppf<0x143, 0xc>(0.f, v);  // row_bcast:31 into rows 2, 3
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
KD float wave_max(float v) {
  const float ni = -INFINITY;
  v = fmaxf(v, dppf<0x111, 0xf>(ni, v));
  v = fmaxf(v, dppf<0x112, 0xf>(ni, v));
  v = fmaxf(v, dppf<0x114, 0xf>(ni, v));
  v = fmaxf(v, dppf<0x118, 0xf>(ni, v));
  v = fmaxf(v, dppf<0x142, 0xa>(ni, v));
  v = fmaxf(v, dppf<0x143, 0xc>(ni, v));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
KD double shx(double v, int m) { return __shfl_xor(v, m, 64); }
KD i32 shx(i32 v, int m) { return __shfl_xor(v, m, 64); }
KD u32 shx(u32 v, int m) { return __shfl_xor((i32)v, m, 64); }
KD i64 shx(i64 v, int m) { return __shfl_xor((long long)v, m, 64); }
KD u64 shx(u64 v, int m) { return (u64)__shfl_xor((long long)v, m, 64); }
KD i8 shx(i8 v, int m) { return (i8)__shfl_xor((i32)v, m, 64); }
KD u8 shx(u8 v, int m) { return (u8)__shfl_xor((i32)v, m, 64); }
KD i16 shx(i16 v, int m) { return (i16)__shfl_xor((i32)v, m, 64); }
KD u16 shx(u16 v, int m) { return (u16)__shfl_xor((i32)v, m, 64); }
KD bool shx(bool v, int m) { return __shfl_xor((i32)v, m, 64) != 0; }
)KUPRELUDE";

}  // namespace ku::hipbk
