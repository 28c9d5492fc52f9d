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
// v_cvt_f32_fp8, with the NaN code S.1111.111 decoded to a quiet NaN carrying the sign
__device__ __forceinline__ float d_e4m3_ld(uint8_t b) {
  if ((b & 0x7fu) == 0x7fu) return __uint_as_float(((uint32_t)(b & 0x80u) << 24) | 0x7fc00000u);
  return __builtin_amdgcn_cvt_f32_fp8((uint32_t)b, 0);
}
// OCP e4m3 (E4M3FN), round to nearest even, saturating to +-448, NaN -> S.1111.111:
// v_cvt_pk_fp8_f32 on the input clamped to +-448 (the same codes as the bit-level rounding for all
// 2^32 f32 inputs on gfx950)
__device__ __forceinline__ uint8_t d_e4m3_st(float x) {
  if (x != x) return (uint8_t)(((__float_as_uint(x) >> 24) & 0x80u) | 0x7fu);
  return (uint8_t)(__builtin_amdgcn_cvt_pk_fp8_f32(__builtin_amdgcn_fmed3f(x, -448.f, 448.f), 0.f, 0, false) & 0xffu);
}
// v_cvt_f32_bf8, NaN codes keeping sign and payload (quiet bit set)
__device__ __forceinline__ float d_e5m2_ld(uint8_t b) {
  if ((b & 0x7cu) == 0x7cu && (b & 3u))
    return __uint_as_float(((uint32_t)(b & 0x80u) << 24) | 0x7fc00000u | ((uint32_t)(b & 3u) << 21));
  return __builtin_amdgcn_cvt_f32_bf8((uint32_t)b, 0);
}
// OCP e5m2, round to nearest even, overflow to inf, NaN -> S.11111.10: v_cvt_pk_bf8_f32
__device__ __forceinline__ uint8_t d_e5m2_st(float x) {
  if (x != x) return (uint8_t)(((__float_as_uint(x) >> 24) & 0x80u) | 0x7eu);
  return (uint8_t)(__builtin_amdgcn_cvt_pk_bf8_f32(x, 0.f, 0, false) & 0xffu);
}

// round an f32 value to bf16 / f16 and back (a fused cast's source dtype); rt < 0: unchanged
__device__ __forceinline__ float d_round_through(int rt, float v) {
  if (rt == GT_BF16) return d_bf16_ld(d_bf16_st(v));
  if (rt == GT_F16) return d_f16_ld(d_f16_st(v));
  return v;
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
