// Generic batched GEMM for every dtype and stride pattern the contraction lowering can
// produce: C[b][m][n] = sum_k A[b][m][k] * B[b][k][n]. Low-precision floats accumulate in
// f32 and round once at the store; f64 accumulates in f64; integers wrap
// (kurumi_core/src/interp/contract.rs:26-64,101-144). The MFMA kernels (gemm_mfma.hip)
// take the bf16/f16/fp8 shapes that matter for speed; this one keeps every other case on
// the device.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.h"
#include "numeric.h"

namespace ku::hipbk {

namespace {

constexpr int TM = 64, TN = 64, TK = 16;

// accumulation type by dtype tag (not by storage type: bf16/f16 are stored as uint16_t)
template <int DT>
struct Acc { using T = uint64_t; };  // integers wrap in 64 bits, truncated at the store
template <> struct Acc<GT_BF16> { using T = float; };
template <> struct Acc<GT_F16> { using T = float; };
template <> struct Acc<GT_F8E4M3> { using T = float; };
template <> struct Acc<GT_F8E5M2> { using T = float; };
template <> struct Acc<GT_F32> { using T = float; };
template <> struct Acc<GT_F64> { using T = double; };

template <int DT, int OT, class TI, class TO, class TA>
__global__ void __launch_bounds__(256) gemm_generic_k(GemmArgs a) {
  __shared__ TA As[TK][TM + 1];
  __shared__ TA Bs[TK][TN + 1];
  const int64_t b = blockIdx.z;
  const int64_t m0 = (int64_t)blockIdx.y * TM, n0 = (int64_t)blockIdx.x * TN;
  const TI* A = static_cast<const TI*>(a.a) + b * a.sab;
  const TI* B = static_cast<const TI*>(a.b) + b * a.sbb;
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  TA acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (TA)0;
  for (int64_t k0 = 0; k0 < a.k; k0 += TK) {
    for (int e = threadIdx.x; e < TK * TM; e += 256) {
      int kk = e % TK, mm = e / TK;
      int64_t gm = m0 + mm, gk = k0 + kk;
      As[kk][mm] = (gm < a.m && gk < a.k) ? load_elem<DT, TI, TA>(A[gm * a.sam + gk * a.sak]) : (TA)0;
    }
    for (int e = threadIdx.x; e < TK * TN; e += 256) {
      int nn = e % TN, kk = e / TN;
      int64_t gn = n0 + nn, gk = k0 + kk;
      Bs[kk][nn] = (gn < a.n && gk < a.k) ? load_elem<DT, TI, TA>(B[gk * a.sbk + gn * a.sbn]) : (TA)0;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < TK; ++kk) {
      TA av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = As[kk][ty + 16 * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = Bs[kk][tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mac(acc[i][j], av[i], bv[j]);
    }
    __syncthreads();
  }
  TO* C = static_cast<TO*>(a.c) + b * a.m * a.n;
  const float alpha = a.alpha ? a.alpha[0] : 1.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int64_t gm = m0 + ty + 16 * i, gn = n0 + tx + 16 * j;
      if (gm < a.m && gn < a.n) {
        TA v = acc[i][j];
        if (a.alpha || a.col_scale) {
          float f = (float)v * alpha;
          if (a.col_scale) f *= a.col_scale[gn * a.col_scale_stride];
          v = (TA)f;
        }
        if constexpr (std::is_same_v<TA, float>) v = d_round_through(a.round_type, v);  // fused cast
        C[gm * a.n + gn] = store_elem<OT, TO, TA>(v);
      }
    }
}

template <int DT, class TI, int OT, class TO>
void launch_t(const GemmArgs& a, hipStream_t s) {
  using TA = typename Acc<DT>::T;
  dim3 grid((unsigned)((a.n + TN - 1) / TN), (unsigned)((a.m + TM - 1) / TM), (unsigned)a.batch);
  hipLaunchKernelGGL((gemm_generic_k<DT, OT, TI, TO, TA>), grid, dim3(256), 0, s, a);
}

}  // namespace

void launch_gemm_generic(const GemmArgs& a, hipStream_t s) {
  // out type follows the input unless an fp8 epilogue asks for bf16/f16/f32
  const int it = a.in_type, ot = a.out_type;
  auto float_out = [&](auto tag_in, auto dt_in) {
    using TI = decltype(tag_in);
    constexpr int DT = decltype(dt_in)::value;
    switch (ot) {
      case GT_BF16: launch_t<DT, TI, GT_BF16, uint16_t>(a, s); return;
      case GT_F16: launch_t<DT, TI, GT_F16, uint16_t>(a, s); return;
      case GT_F32: launch_t<DT, TI, GT_F32, float>(a, s); return;
      case GT_F8E4M3: launch_t<DT, TI, GT_F8E4M3, uint8_t>(a, s); return;
      case GT_F8E5M2: launch_t<DT, TI, GT_F8E5M2, uint8_t>(a, s); return;
      default: throw_gemm_unsupported(a);
    }
  };
  switch (it) {
    case GT_BF16: float_out(uint16_t{}, DTag<GT_BF16>{}); return;
    case GT_F16: float_out(uint16_t{}, DTag<GT_F16>{}); return;
    case GT_F8E4M3: float_out(uint8_t{}, DTag<GT_F8E4M3>{}); return;
    case GT_F8E5M2: float_out(uint8_t{}, DTag<GT_F8E5M2>{}); return;
    case GT_F32: float_out(float{}, DTag<GT_F32>{}); return;
    case GT_F64: launch_t<GT_F64, double, GT_F64, double>(a, s); return;
    case 1: launch_t<1, uint8_t, 1, uint8_t>(a, s); return;
    case 2: launch_t<2, uint16_t, 2, uint16_t>(a, s); return;
    case 3: launch_t<3, uint32_t, 3, uint32_t>(a, s); return;
    case 4: launch_t<4, uint64_t, 4, uint64_t>(a, s); return;
    case 5: launch_t<5, int8_t, 5, int8_t>(a, s); return;
    case 6: launch_t<6, int16_t, 6, int16_t>(a, s); return;
    case 7: launch_t<7, int32_t, 7, int32_t>(a, s); return;
    case 8: launch_t<8, int64_t, 8, int64_t>(a, s); return;
    default: throw_gemm_unsupported(a);
  }
}

}  // namespace ku::hipbk
