// Device element conversions shared by the precompiled kernels: the same rounding rules
// as the generated-kernel prelude (round to nearest even; e4m3 saturates to +-448).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

#include "kernels.h"

namespace ku::hipbk {

template <int V>
struct DTag { static constexpr int value = V; };

__device__ __forceinline__ float d_bf16_ld(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }
// v_cvt_pk_bf16_f32 (round to nearest even, NaN quieted keeping sign and top payload bits)
__device__ __forceinline__ uint16_t d_bf16_st(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
__device__ __forceinline__ float d_f16_ld(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t d_f16_st(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ __forceinline__ float d_e4m3_ld(uint8_t b) {
  uint32_t e = (b >> 3) & 15u, m = b & 7u;
  float v;
  if (e == 15u && m == 7u) v = __uint_as_float(0x7fc00000u);
  else if (e == 0u) v = (float)m * 0.001953125f;
  else v = __uint_as_float(((e + 120u) << 23) | (m << 20));
  return (b & 0x80u) ? -v : v;
}
__device__ __forceinline__ uint8_t d_e4m3_st(float x) {
  uint32_t u = __float_as_uint(x);
  uint32_t s = (u >> 24) & 0x80u;
  if (x != x) return (uint8_t)(s | 0x7fu);
  float a = fabsf(x);
  if (a > 448.f) return (uint8_t)(s | 0x7eu);
  if (a < 0.015625f) return (uint8_t)(s | (uint32_t)rintf(a * 512.f));
  int E = (int)((u >> 23) & 0xffu) - 127;
  float q = __uint_as_float((uint32_t)(E - 3 + 127) << 23);
  uint32_t n = (uint32_t)rintf(a / q);
  uint32_t r = ((uint32_t)(E + 7) << 3) + (n - 8u);
  if (r > 0x7eu) r = 0x7eu;
  return (uint8_t)(s | r);
}
__device__ __forceinline__ float d_e5m2_ld(uint8_t b) {
  uint32_t e = (b >> 2) & 31u, m = b & 3u;
  float v;
  if (e == 31u) v = m ? __uint_as_float(0x7fc00000u) : INFINITY;
  else if (e == 0u) v = (float)m * 1.52587890625e-05f;
  else v = __uint_as_float(((e + 112u) << 23) | (m << 21));
  return (b & 0x80u) ? -v : v;
}
__device__ __forceinline__ uint8_t d_e5m2_st(float x) {
  uint32_t u = __float_as_uint(x);
  uint32_t s = (u >> 24) & 0x80u;
  if (x != x) return (uint8_t)(s | 0x7eu);
  float a = fabsf(x);
  if (a >= 61440.f) return (uint8_t)(s | 0x7cu);
  if (a < 6.103515625e-05f) return (uint8_t)(s | (uint32_t)rintf(a * 65536.f));
  int E = (int)((u >> 23) & 0xffu) - 127;
  float q = __uint_as_float((uint32_t)(E - 2 + 127) << 23);
  uint32_t n = (uint32_t)rintf(a / q);
  return (uint8_t)(s | (((uint32_t)(E + 15) << 2) + (n - 4u)));
}

// storage element -> accumulation type
template <int DT, class TI, class TA>
__device__ __forceinline__ TA load_elem(TI x) {
  if constexpr (DT == GT_BF16) return d_bf16_ld(x);
  else if constexpr (DT == GT_F16) return d_f16_ld(x);
  else if constexpr (DT == GT_F8E4M3) return d_e4m3_ld(x);
  else if constexpr (DT == GT_F8E5M2) return d_e5m2_ld(x);
  else if constexpr (std::is_same_v<TA, uint64_t>) return (uint64_t)(int64_t)x;
  else return (TA)x;
}
// accumulator -> storage element of dtype OT
template <int OT, class TO, class TA>
__device__ __forceinline__ TO store_elem(TA v) {
  if constexpr (OT == GT_BF16) return d_bf16_st((float)v);
  else if constexpr (OT == GT_F16) return d_f16_st((float)v);
  else if constexpr (OT == GT_F8E4M3) return d_e4m3_st((float)v);
  else if constexpr (OT == GT_F8E5M2) return d_e5m2_st((float)v);
  else return (TO)v;
}
template <class TA>
__device__ __forceinline__ TA mac(TA acc, TA a, TA b) {
  if constexpr (std::is_same_v<TA, uint64_t>) return acc + a * b;
  else return fma(a, b, acc);
}

inline void throw_gemm_unsupported(const GemmArgs& a) {
  throw std::runtime_error("kurumi_hip: no GEMM kernel for in dtype " + std::to_string(a.in_type) + " -> out " +
                           std::to_string(a.out_type));
}

void launch_gemm_generic(const GemmArgs& a, hipStream_t s);

}  // namespace ku::hipbk
