// Weight-only quantized matmul for gfx950 (kernel family 5):
// out[m][n] = sum_k act[m][k] * dequant(qweight)[n][k], the semantics of `Op::QuantMatmul`
// (kurumi_core/src/interp/contract.rs:69-99 over quant.rs:100-133): 2/4/8-bit fields packed
// row-major along K, low field first; one f16 scale per group of `group` K columns, plus an f16
// min when asymmetric (w = q * s + min) or a sign-extended field when symmetric (w = q * s);
// f32 products and accumulation, the result rounded once to act's dtype.
//
// quant_gemv_fast_k / quant_gemv_k (M <= 8, the decode shapes): the weight is read from HBM
// exactly once and dequantized in registers; GEMV_RW weight rows per work-group share each act
// value a thread loads, and their 16-byte chunks are all in flight at once. With bf16 / f16 act
// and 2- or 4-bit fields the products run on v_dot2 pairs (one v_bitop3 turns two fields into a
// 16-bit pair), which keeps the VALU work per weight byte below the HBM time.
// quant_mm_fused_k (int4, bf16 / f16 act, 9 <= M <= 64, groups a multiple of 128): the same
// register conversion feeds the MFMAs, both operands staged through LDS by whole-line DMA (a
// constant weight from its lane-ordered copy); quant_mm_k, after the act pass quant_act_prep_k,
// for the other groups.
// quant_dequant_k (everything else): the weight is expanded once into act's dtype (f32, bf16 or
// f16) for the MFMA / generic GEMM; bf16 / f16 round each dequantized weight once, the f32
// products then accumulate in f32 like the reference.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "kernels.h"
#include "lds_dma.h"
#include "numeric.h"

namespace ku::hipbk {

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int GEMV_RW = 4;  // weight rows per work-group (4 measured best for the decode shape)

__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

template <int AT>
__device__ __forceinline__ float act_ld(const void* p, int64_t i) {
  if constexpr (AT == GT_F32) return static_cast<const float*>(p)[i];
  else if constexpr (AT == GT_BF16) return __uint_as_float((uint32_t) static_cast<const uint16_t*>(p)[i] << 16);
  else return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
}

template <int AT>
__device__ __forceinline__ void act_st(void* p, int64_t i, float v) {
  if constexpr (AT == GT_F32) static_cast<float*>(p)[i] = v;
  else if constexpr (AT == GT_BF16) static_cast<uint16_t*>(p)[i] = d_bf16_st(v);
  else static_cast<uint16_t*>(p)[i] = d_f16_st(v);
}

// field i (0 .. 8/BITS - 1 per byte) of packed byte b, dequantized with scale s / min mn; the
// product is not fused with the min (the reference rounds q * s, then adds)
template <int BITS, bool SYM>
__device__ __forceinline__ float deq(uint32_t raw, float s, float mn) {
  if constexpr (SYM) {
    const int v = (int)(raw << (32 - BITS)) >> (32 - BITS);
    return __fmul_rn((float)v, s);
  } else {
    return __fadd_rn(__fmul_rn((float)raw, s), mn);
  }
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xf, false));
}

// sum over the wave, valid in every lane: DPP row shifts, then row broadcasts into lane 63
// (VALU latency per step, no LDS permutes)
__device__ __forceinline__ float wave_add(float v) {
  v += dpp_f<0x111, 0xf>(v);  // row_shr:1
  v += dpp_f<0x112, 0xf>(v);  // row_shr:2
  v += dpp_f<0x114, 0xf>(v);  // row_shr:4
  v += dpp_f<0x118, 0xf>(v);  // row_shr:8: lane 15 of each row of 16 holds the row's sum
  v += dpp_f<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp_f<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// acc + lo(x) * lo(y) + hi(x) * hi(y) on 16-bit pairs (bf16 or f16), f32 accumulate
template <int AT>
__device__ __forceinline__ float dot2(uint32_t x, uint32_t y, float acc) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
  if constexpr (AT == GT_BF16)
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x), __builtin_bit_cast(bf16x2, y), acc, false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, x), __builtin_bit_cast(f16x2, y), acc, false);
}

// V consecutive act values of one row as f32 (one or two 16-byte loads when V allows)
template <int AT, int V>
__device__ __forceinline__ void load_act(const void* act, int64_t idx, float (&av)[V]) {
  if constexpr (AT == GT_F32 && V % 4 == 0) {
    const float* p = static_cast<const float*>(act) + idx;
#pragma unroll
    for (int q = 0; q < V / 4; ++q) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(p + 4 * q);
#pragma unroll
      for (int i = 0; i < 4; ++i) av[4 * q + i] = __uint_as_float(v[i]);
    }
  } else if constexpr (AT != GT_F32 && V % 8 == 0) {
    const uint16_t* p = static_cast<const uint16_t*>(act) + idx;
#pragma unroll
    for (int q = 0; q < V / 8; ++q) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(p + 8 * q);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint16_t h = (uint16_t)(v[i >> 1] >> ((i & 1) * 16));
        av[8 * q + i] = AT == GT_BF16 ? __uint_as_float((uint32_t)h << 16) : f16_to_f32(h);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i) av[i] = act_ld<AT>(act, idx + i);
  }
}

// A work-group takes GEMV_RW weight rows; its threads stride over the K chunks of CB packed
// bytes (E values). Per chunk a thread issues the loads of all GEMV_RW rows first (they are in
// flight together), then walks the chunk V values at a time: each act value is loaded once for
// all weight rows. OG: a chunk lies inside one scale group (one scale / min per row and chunk);
// otherwise each value looks its group up. Partial dots are folded by a wave reduction and an
// LDS sum across waves.
template <int BITS, bool SYM, int AT, int MB, int CB, bool OG>
__global__ void __launch_bounds__(256) quant_gemv_k(QuantArgs a) {
  constexpr int PER = 8 / BITS, E = CB * PER;  // weight values per thread and chunk
  constexpr int V = E < 8 ? E : 8;             // act values loaded at a time
  __shared__ float red[4][GEMV_RW * MB];
  const int tid = threadIdx.x, nt = blockDim.x, lane = tid & 63, wave = tid >> 6, nwv = nt >> 6;
  const int64_t K = a.k, N = a.n, rb = K * BITS / 8, ng = K / a.group, nch = K / E;
  const int64_t row0 = (int64_t)blockIdx.x * GEMV_RW;
  int64_t rows[GEMV_RW];
#pragma unroll
  for (int r = 0; r < GEMV_RW; ++r) rows[r] = row0 + r < N ? row0 + r : N - 1;  // duplicates never stored
  float acc[GEMV_RW][MB];
#pragma unroll
  for (int r = 0; r < GEMV_RW; ++r)
#pragma unroll
    for (int m = 0; m < MB; ++m) acc[r][m] = 0.f;
  for (int64_t c = tid; c < nch; c += nt) {
    const int64_t k = c * E;
    uint32_t wb[GEMV_RW][(CB + 3) / 4];
#pragma unroll
    for (int r = 0; r < GEMV_RW; ++r) {
      const uint8_t* p = a.qw + rows[r] * rb + k / PER;
      if constexpr (CB == 16) {
        const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
#pragma unroll
        for (int j = 0; j < 4; ++j) wb[r][j] = w[j];
      } else if constexpr (CB == 8) {
        const u32x2 w = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
        wb[r][0] = w[0];
        wb[r][1] = w[1];
      } else {
        wb[r][0] = p[0];
      }
    }
    float s[GEMV_RW], mn[GEMV_RW];
    if constexpr (OG) {
#pragma unroll
      for (int r = 0; r < GEMV_RW; ++r) {
        const int64_t gi = rows[r] * ng + k / a.group;
        s[r] = f16_to_f32(a.scales[gi]);
        mn[r] = SYM ? 0.f : f16_to_f32(a.mins[gi]);
      }
    }
#pragma unroll
    for (int e0 = 0; e0 < E; e0 += V) {
      float av[MB][V];
#pragma unroll
      for (int m = 0; m < MB; ++m) {
        if (m < a.m) load_act<AT, V>(a.act, m * K + k + e0, av[m]);
        else {
#pragma unroll
          for (int e = 0; e < V; ++e) av[m][e] = 0.f;
        }
      }
#pragma unroll
      for (int r = 0; r < GEMV_RW; ++r)
#pragma unroll
        for (int e = 0; e < V; ++e) {
          const int ei = e0 + e;
          if constexpr (!OG) {
            const int64_t gi = rows[r] * ng + (k + ei) / a.group;
            s[r] = f16_to_f32(a.scales[gi]);
            mn[r] = SYM ? 0.f : f16_to_f32(a.mins[gi]);
          }
          const uint32_t raw = (wb[r][ei / (4 * PER)] >> ((ei % (4 * PER)) * BITS)) & ((1u << BITS) - 1);
          const float w = deq<BITS, SYM>(raw, s[r], mn[r]);
#pragma unroll
          for (int m = 0; m < MB; ++m) acc[r][m] = fmaf(av[m][e], w, acc[r][m]);
        }
    }
  }
#pragma unroll
  for (int r = 0; r < GEMV_RW; ++r)
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      const float v = wave_add(acc[r][m]);
      if (lane == 0) red[wave][r * MB + m] = v;
    }
  __syncthreads();
  if (tid < GEMV_RW * MB) {
    const int r = tid / MB, m = tid % MB;
    float v = red[0][tid];
    for (int w = 1; w < nwv; ++w) v += red[w][tid];
    const int64_t n = row0 + r;
    if (n < N && m < a.m) act_st<AT>(a.out, m * N + n, v);
  }
}

// Fast path of quant_gemv_k (chunks of 16 packed bytes, 8 for int2; each chunk inside one scale
// group). The fields are turned into floats a byte at a time with v_cvt_f32_ubyte{0..3} after one
// mask per word, and the per-value scale is factored out of the chunk's sum:
//   sum_e act[e] * w[e] = s * (sum_e act[e] * u[e] - off * sum_e act[e]) + min * sum_e act[e]
// with u the unsigned field (symmetric fields are offset by 2^(bits-1) with one xor per word,
// off = 2^(bits-1); asymmetric: off = 0). The act sums are shared by all rows of the work-group.
// This reassociates the f32 arithmetic of the reference's per-value dequantisation (a few f32
// ulps of the chunk sum), well inside the f32 tolerance.
template <int BITS, bool SYM, int AT, int MB>
__global__ void __launch_bounds__(256) quant_gemv_fast_k(QuantArgs a) {
  constexpr int CB = BITS == 2 ? 8 : 16, PER = 8 / BITS, E = CB * PER, NWD = CB / 4;
  constexpr int VW = 4 * PER;                 // values per 32-bit word
  constexpr int V = VW < 8 ? 8 : VW;          // act values loaded at a time (whole words)
  constexpr uint32_t FMASK = BITS == 8 ? 0xFFFFFFFFu : (BITS == 4 ? 0x0F0F0F0Fu : 0x03030303u);
  constexpr uint32_t XOR = SYM ? (BITS == 8 ? 0x80808080u : (BITS == 4 ? 0x88888888u : 0xAAAAAAAAu)) : 0u;
  constexpr float OFF = SYM ? (float)(1 << (BITS - 1)) : 0.f;
  // 16-bit act (bf16 / f16) with 2- or 4-bit fields: v_dot2 on pairs. A field u (< 16) OR-ed into
  // the mantissa of MAGICV (128 in bf16, 1024 in f16, both with ulp 1) is exactly MAGICV + u, and
  // the MAGICV * sum(act) this adds is taken off with the offset.
  constexpr bool DOT = BITS != 8 && AT != GT_F32;
  constexpr int H = VW / 2;
  constexpr uint32_t PMASK = BITS == 4 ? 0x000F000Fu : 0x00030003u;
  constexpr uint32_t MAGIC = AT == GT_BF16 ? 0x43004300u : 0x64006400u;
  constexpr float MAGICV = AT == GT_BF16 ? 128.f : 1024.f;
  constexpr uint32_t LXOR = DOT ? 0u : XOR;  // the dot path applies the offset in its v_bitop3
  constexpr uint32_t ONES = AT == GT_BF16 ? 0x3F803F80u : 0x3C003C00u;
  __shared__ float red[4][GEMV_RW * MB];
  const int tid = threadIdx.x, nt = blockDim.x, lane = tid & 63, wave = tid >> 6, nwv = nt >> 6;
  const int64_t K = a.k, N = a.n, rb = K * BITS / 8, ng = K / a.group, nch = K / E;
  const int64_t row0 = (int64_t)blockIdx.x * GEMV_RW;
  int64_t rows[GEMV_RW];
#pragma unroll
  for (int r = 0; r < GEMV_RW; ++r) rows[r] = row0 + r < N ? row0 + r : N - 1;  // duplicates never stored
  float acc[GEMV_RW][MB];
#pragma unroll
  for (int r = 0; r < GEMV_RW; ++r)
#pragma unroll
    for (int m = 0; m < MB; ++m) acc[r][m] = 0.f;
  for (int64_t c = tid; c < nch; c += nt) {
    const int64_t k = c * E;
    uint32_t wb[GEMV_RW][NWD];
#pragma unroll
    for (int r = 0; r < GEMV_RW; ++r) {
      const uint8_t* p = a.qw + rows[r] * rb + k / PER;
      if constexpr (CB == 16) {
        const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
#pragma unroll
        for (int j = 0; j < 4; ++j) wb[r][j] = w[j] ^ LXOR;
      } else {
        const u32x2 w = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
        wb[r][0] = w[0] ^ LXOR;
        wb[r][1] = w[1] ^ LXOR;
      }
    }
    float s[GEMV_RW], mn[GEMV_RW];
    const uint32_t kg = (uint32_t)k / (uint32_t)a.group;  // one 32-bit division per chunk
#pragma unroll
    for (int r = 0; r < GEMV_RW; ++r) {
      const uint32_t gi = (uint32_t)rows[r] * (uint32_t)ng + kg;
      s[r] = f16_to_f32(a.scales[gi]);
      mn[r] = SYM ? 0.f : f16_to_f32(a.mins[gi]);
    }
    float part[GEMV_RW][MB], asum[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      asum[m] = 0.f;
#pragma unroll
      for (int r = 0; r < GEMV_RW; ++r) part[r][m] = 0.f;
    }
    if constexpr (DOT) {
      // act as raw 16-bit pairs, VW / 2 words per weight word and act row: the whole chunk's act
      // loaded up front for M <= 4 (measured faster), one weight word's at a time for M = 8
      // (registers)
      constexpr int AWW = MB <= 4 ? NWD : 1;
      uint32_t awc[MB][AWW * VW / 2];
      auto load_aw = [&](int w0) {
#pragma unroll
        for (int m = 0; m < MB; ++m)
#pragma unroll
          for (int q = 0; q < AWW * VW / 8; ++q) {
            const u32x4 v = m < a.m ? *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.act) + m * K + k +
                                                                      w0 * VW + 8 * q)
                                    : u32x4{0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < 4; ++i) awc[m][4 * q + i] = v[i];
          }
#pragma unroll
        for (int m = 0; m < MB; ++m)
#pragma unroll
          for (int i = 0; i < AWW * VW / 2; ++i) asum[m] = dot2<AT>(awc[m][i], ONES, asum[m]);
      };
      if constexpr (AWW == NWD) load_aw(0);
#pragma unroll
      for (int wi = 0; wi < NWD; ++wi) {
        if constexpr (AWW == 1) load_aw(wi);
        const int wb0 = AWW == 1 ? 0 : wi * VW / 2;  // word wi's first act word in awc
        // pair p of word wi: fields p (low half) and p + H (high half), act values p and p + H
        uint32_t ap[MB][H];
#pragma unroll
        for (int m = 0; m < MB; ++m)
#pragma unroll
          for (int p = 0; p < H; ++p) {
            // p and p + H (H even) sit in the same half of their act words
            constexpr uint32_t SEL[2] = {0x05040100u, 0x07060302u};  // v_perm_b32: half h of src1 | half h of src0
            ap[m][p] = __builtin_amdgcn_perm(awc[m][wb0 + ((p + H) >> 1)], awc[m][wb0 + (p >> 1)], SEL[p & 1]);
          }
#pragma unroll
        for (int r = 0; r < GEMV_RW; ++r) {
          const uint32_t word = wb[r][wi];
#pragma unroll
          for (int p = 0; p < H; ++p) {
            // (MAGICV + u) as a 16-bit pair: C ^ (t & PMASK) with C = MAGIC | XOR in one v_bitop3
            // (0x6c: S1 ^ (S0 & S2)); the symmetric offset's xor rides along
            const uint32_t x = __builtin_amdgcn_bitop3_b32(word >> (BITS * p), MAGIC | (XOR & PMASK), PMASK, 0x6c);
#pragma unroll
            for (int m = 0; m < MB; ++m) part[r][m] = dot2<AT>(x, ap[m][p], part[r][m]);
          }
        }
      }
#pragma unroll
      for (int r = 0; r < GEMV_RW; ++r)
#pragma unroll
        for (int m = 0; m < MB; ++m) {
          const float q = fmaf(-(MAGICV + OFF), asum[m], part[r][m]);
          acc[r][m] = fmaf(s[r], q, acc[r][m]);
          if constexpr (!SYM) acc[r][m] = fmaf(mn[r], asum[m], acc[r][m]);
        }
      continue;
    }
#pragma unroll
    for (int e0 = 0; e0 < E; e0 += V) {
      float av[MB][V];
#pragma unroll
      for (int m = 0; m < MB; ++m) {
        if (m < a.m) load_act<AT, V>(a.act, m * K + k + e0, av[m]);
        else {
#pragma unroll
          for (int e = 0; e < V; ++e) av[m][e] = 0.f;
        }
#pragma unroll
        for (int e = 0; e < V; ++e) asum[m] += av[m][e];
      }
#pragma unroll
      for (int r = 0; r < GEMV_RW; ++r)
#pragma unroll
        for (int wi = 0; wi < V / VW; ++wi) {
          const uint32_t word = wb[r][e0 / VW + wi];
#pragma unroll
          for (int f = 0; f < PER; ++f) {
            const uint32_t fw = (word >> (f * BITS)) & FMASK;  // field f of each of the 4 bytes
#pragma unroll
            for (int bj = 0; bj < 4; ++bj) {
              const float u = (float)((fw >> (8 * bj)) & 0xFFu);  // v_cvt_f32_ubyte{bj}
              const int e = wi * VW + bj * PER + f;
#pragma unroll
              for (int m = 0; m < MB; ++m) part[r][m] = fmaf(av[m][e], u, part[r][m]);
            }
          }
        }
    }
#pragma unroll
    for (int r = 0; r < GEMV_RW; ++r)
#pragma unroll
      for (int m = 0; m < MB; ++m) {
        const float q = SYM ? fmaf(-OFF, asum[m], part[r][m]) : part[r][m];
        acc[r][m] = fmaf(s[r], q, acc[r][m]);
        if constexpr (!SYM) acc[r][m] = fmaf(mn[r], asum[m], acc[r][m]);
      }
  }
#pragma unroll
  for (int r = 0; r < GEMV_RW; ++r)
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      const float v = wave_add(acc[r][m]);
      if (lane == 0) red[wave][r * MB + m] = v;
    }
  __syncthreads();
  if (tid < GEMV_RW * MB) {
    const int r = tid / MB, m = tid % MB;
    float v = red[0][tid];
    for (int w = 1; w < nwv; ++w) v += red[w][tid];
    const int64_t n = row0 + r;
    if (n < N && m < a.m) act_st<AT>(a.out, m * N + n, v);
  }
}

// Fused dequant MFMA kernel (int4, bf16 / f16 act, 9 <= M <= 64: batched decode). Transposed
// like the attention kernel, C^T[n][m] = W[n][:] . act[m][:] with v_mfma_f32_32x32x16: the A
// operand is a 32-row tile of the weight, each lane converting the 8 fields of one packed word
// into 16-bit pairs (MAGICV + u) with v_bitop3 (pairs (p, p + 4) of the word), the B operand the
// act values of that word in the same order (v_perm), so no LDS staging is needed for either.
// Lane l owns act row m = l % 32 of each accumulator, which makes the act sum of the magic /
// offset correction a per-lane value. Per scale group the MFMA partial is folded as
//   acc += s[n][g] * (C_g - (MAGICV + off) * sum_k act) (+ min[n][g] * sum_k act).
// Every 64-value block of a row: lane half h reads bytes 16h..16h+15 (words 4h..4h+3) and k-step
// j of the MFMA takes word 4h + j in half h (a permutation of k shared by both operands). A
// work-group holds 32 * NT weight rows; its QMM_NW waves take the scale groups round-robin and
// add their partials through LDS at the end. The rows' scales (and mins) are staged in LDS
// transposed to [group][row] first. Act, the larger operand (every work-group reads all of it),
// comes from quant_act_prep_k in the order the lanes load it: one load instruction reads 1 KB of
// whole lines instead of 32 bytes from each of 32 rows.
constexpr int QMM_NW = 8;

// quant_mm_k's act operand, laid out for its loads. MP = 32 * MT rows (rows past M are zeros);
// sub-group sg is GB blocks of 64 values. For block bb of sub-group sg, load q (0..3), row m and
// lane half h, the 16 bytes at u32 index ((((sg * GB + bb) * 4 + q) * MP + m) * 2 + h) * 4 hold
// the MFMA B operand of k-step q: pairs (value p, value p + 4), p = 0..3, of the 8 values at
// k = 64 (sg GB + bb) + 32 h + 8 q. sums[(sg * MP + m) * 2 + h] is the v_dot2 chain of that
// half's 32 GB values over the sub-group (the kernel adds the two halves).
__host__ __device__ inline int64_t quant_act_rows(int64_t m) { return m <= 32 ? 32 : 64; }
__host__ __device__ inline size_t quant_actp_bytes(int64_t m, int64_t k) {
  return ((size_t)(quant_act_rows(m) * k * 2) + 255) & ~(size_t)255;
}
template <int AT, int GB>
__global__ void __launch_bounds__(64) quant_act_prep_k(const uint16_t* __restrict__ act, uint32_t* __restrict__ actp,
                                                       float* __restrict__ sums, int64_t m_rows, int64_t k) {
  constexpr uint32_t ONES = AT == GT_BF16 ? 0x3F803F80u : 0x3C003C00u;
  constexpr uint32_t SEL[2] = {0x05040100u, 0x07060302u};  // v_perm_b32: half p of src1 | half p of src0
  const int64_t mp = quant_act_rows(m_rows), nsg = k / (64 * GB);
  const int64_t idx = (int64_t)blockIdx.x * 64 + threadIdx.x;  // (sg, m, h), h fastest
  if (idx >= nsg * mp * 2) return;
  const int h = (int)(idx & 1);
  const int64_t m = (idx >> 1) % mp, sg = (idx >> 1) / mp;
  // all of this thread's loads in flight at once (the pass is one memory latency long)
  u32x4 v[GB][4];
#pragma unroll
  for (int bb = 0; bb < GB; ++bb)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      v[bb][q] = m < m_rows ? *reinterpret_cast<const u32x4*>(act + m * k + (sg * GB + bb) * 64 + 32 * h + 8 * q)
                            : u32x4{0, 0, 0, 0};
  float as = 0.f;
#pragma unroll
  for (int bb = 0; bb < GB; ++bb)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int i = 0; i < 4; ++i) as = dot2<AT>(v[bb][q][i], ONES, as);
      u32x4 o;
#pragma unroll
      for (int p = 0; p < 4; ++p) o[p] = __builtin_amdgcn_perm(v[bb][q][(p + 4) >> 1], v[bb][q][p >> 1], SEL[p & 1]);
      *reinterpret_cast<u32x4*>(actp + ((((sg * GB + bb) * 4 + q) * mp + m) * 2 + h) * 4) = o;
    }
  sums[idx] = as;
}

template <bool SYM, int AT, int NT, int MT, int GB>
__global__ void __launch_bounds__(QMM_NW * 64) quant_mm_k(QuantArgs a) {
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
  typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
  constexpr uint32_t PMASK = 0x000F000Fu;
  constexpr uint32_t MAGIC = AT == GT_BF16 ? 0x43004300u : 0x64006400u;
  constexpr float MAGICV = AT == GT_BF16 ? 128.f : 1024.f;
  constexpr uint32_t CX = MAGIC | (SYM ? 0x00080008u : 0u);  // bitop3 constant: magic + symmetric offset xor
  constexpr float OFF = SYM ? 8.f : 0.f;
  constexpr uint32_t ONES = AT == GT_BF16 ? 0x3F803F80u : 0x3C003C00u;
  constexpr int RW = 32 * NT;  // weight rows per work-group
  extern __shared__ __attribute__((aligned(16))) unsigned char qmm_lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, h = lane >> 5;
  const int64_t K = a.k, N = a.n, M = a.m, rb = K / 2, ng = K / a.group;
  const int64_t n0 = (int64_t)blockIdx.x * RW;
  uint16_t* ssc = reinterpret_cast<uint16_t*>(qmm_lds);  // [ng][RW]
  uint16_t* smn = ssc + ng * RW;
  for (int64_t i = tid; i < ng * RW; i += QMM_NW * 64) {
    const int64_t r = i / ng, g = i % ng;  // consecutive threads read along a row of the table
    const int64_t n = n0 + r < N ? n0 + r : N - 1;
    ssc[g * RW + r] = a.scales[n * ng + g];
    if constexpr (!SYM) smn[g * RW + r] = a.mins[n * ng + g];
  }
  __syncthreads();

  const uint8_t* wrow[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int64_t n = n0 + 32 * t + l32;
    wrow[t] = a.qw + (n < N ? n : N - 1) * rb + 16 * h;
  }
  // the prepared act (quant_act_prep_k): this lane's 16 bytes of load q of block bb of sub-group sg
  // at actp[(sg * GB + bb) * 4 + q][lane offset]; its sums at sums[sg][lane offset]
  constexpr int MP = 32 * MT;
  const uint32_t* actp = static_cast<const uint32_t*>(a.mm_scratch);
  const float* sums = reinterpret_cast<const float*>(static_cast<const unsigned char*>(a.mm_scratch) +
                                                     quant_actp_bytes(M, K));
  int aoff[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) aoff[mt] = (32 * mt + l32) * 2 + h;
  f32x16 acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[t][mt][v] = 0.f;
  // The wave's K range is a contiguous run of sub-groups of GB blocks of 64 values (GB * 64 divides
  // the scale group, so each sub-group has one scale per row and folds on its own). The loads of
  // sub-group i + 1 are issued before sub-group i is computed (two register sets that swap roles).
  const int nsg = (int)(K / (64 * GB));
  const int spw = (nsg + QMM_NW - 1) / QMM_NW, sbeg = wave * spw, send = min(nsg, sbeg + spw);
  const int sg_per_group = (int)(a.group / (64 * GB));
  auto load = [&](int sg, u32x4 (&w)[GB][NT], uint32_t (&aw)[GB][MT][16]) __attribute__((always_inline)) {
#pragma unroll
    for (int bb = 0; bb < GB; ++bb) {
      const int kb = (sg * GB + bb) * 64;  // first k of the block
#pragma unroll
      for (int t = 0; t < NT; ++t) w[bb][t] = *reinterpret_cast<const u32x4*>(wrow[t] + kb / 2);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const u32x4 v = *reinterpret_cast<const u32x4*>(actp + (((int64_t)(sg * GB + bb) * 4 + q) * MP * 2 + aoff[mt]) * 4);
#pragma unroll
          for (int i = 0; i < 4; ++i) aw[bb][mt][4 * q + i] = v[i];
        }
    }
  };
  auto step = [&](int sg, const u32x4 (&w)[GB][NT], const uint32_t (&aw)[GB][MT][16]) __attribute__((always_inline)) {
    f32x16 cg[NT][MT];
    float as[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) as[mt] = sums[(int64_t)sg * MP * 2 + aoff[mt]];
#pragma unroll
    for (int bb = 0; bb < GB; ++bb)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        // k-step jj of block bb: word 4h + jj of each row; act pairs (p, p + 4) of the same 8
        // values, prepared in that order
        u32x4 bf[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int p = 0; p < 4; ++p) bf[mt][p] = aw[bb][mt][4 * jj + p];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          u32x4 af;
#pragma unroll
          for (int p = 0; p < 4; ++p)
            // through the builtin, not inline asm: the compiler then keeps the wait states a VALU
            // result needs before an MFMA reads it
            af[p] = __builtin_amdgcn_bitop3_b32(w[bb][t][jj] >> (4 * p), CX, PMASK, 0x6c);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const f32x16 c = (bb == 0 && jj == 0) ? f32x16{} : cg[t][mt];  // the sub-group starts from zero
            if constexpr (AT == GT_BF16)
              cg[t][mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, af),
                                                                  __builtin_bit_cast(bf16x8, bf[mt]), c, 0, 0, 0);
            else
              cg[t][mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, af),
                                                                 __builtin_bit_cast(f16x8, bf[mt]), c, 0, 0, 0);
          }
        }
      }
    // the sub-group's act sum of this lane's row over both lane halves, then the fold
    const int g = sg / sg_per_group;
    float at[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(as[mt]), __float_as_uint(as[mt]), false, false);
      at[mt] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = 32 * t + 8 * (v >> 2) + 4 * h + (v & 3);  // C row = weight row of the tile
        const float sc = f16_to_f32(ssc[g * RW + r]);
        const float mn = SYM ? 0.f : f16_to_f32(smn[g * RW + r]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          acc[t][mt][v] = fmaf(sc, fmaf(-(MAGICV + OFF), at[mt], cg[t][mt][v]), acc[t][mt][v]);
          if constexpr (!SYM) acc[t][mt][v] = fmaf(mn, at[mt], acc[t][mt][v]);
        }
      }
  };
  u32x4 w0[GB][NT], w1[GB][NT];
  uint32_t a0[GB][MT][16], a1[GB][MT][16];
  if (sbeg < send) load(sbeg, w0, a0);
  for (int sg = sbeg; sg < send; sg += 2) {
    if (sg + 1 < send) load(sg + 1, w1, a1);
    step(sg, w0, a0);
    if (sg + 1 >= send) break;
    if (sg + 2 < send) load(sg + 2, w0, a0);
    step(sg + 1, w1, a1);
  }
  // partials of the waves through LDS (the scale table is no longer read)
  __syncthreads();
  float* red = reinterpret_cast<float*>(qmm_lds);  // [wave][t][mt][v][lane]
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 16; ++v) red[(((wave * NT + t) * MT + mt) * 16 + v) * 64 + lane] = acc[t][mt][v];
  __syncthreads();
  constexpr int PER = NT * MT * 16 * 64;  // elements of one wave's partial
  for (int e = tid; e < PER; e += QMM_NW * 64) {
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < QMM_NW; ++w) sum += red[w * PER + e];
    const int ln = e & 63, v = (e >> 6) & 15, mt = (e >> 10) % MT, t = (e >> 10) / MT;
    const int64_t m = 32 * mt + (ln & 31);
    const int64_t n = n0 + 32 * t + 8 * (v >> 2) + 4 * (ln >> 5) + (v & 3);
    if (m < M && n < N) act_st<AT>(a.out, m * N + n, sum);
  }
}

#define KU_LDS __attribute__((address_space(3)))

__device__ __forceinline__ __amdgpu_buffer_rsrc_t qrsrc(const void* p, uint32_t bytes) {
  // dword3 0x00020000: 32-bit data format, the raw-buffer setting for gfx9 parts
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// The fused MFMA kernel without the act pass (groups a multiple of 128, so every sub-group is two
// 64-value blocks; operands under 2 GiB). Same products, sums and folds in the same order as
// quant_mm_k, so the results are bit-identical; what changes is how the operands arrive. Each
// wave streams its run of blocks through two LDS stage buffers by DMA (buffer_load ... lds), the
// next block's DMAs in flight while the current block is computed:
//   act: the block's 32 * MT rows x 128 bytes, 8 rows per DMA, every DMA whole cache lines; lane
//        l of DMA i fetches row 8i + l / 8, chunk (l % 8) ^ (l / 8) into slot l % 8, so the 32
//        lanes that later read one chunk of 32 rows hit distinct bank groups 8 at a time;
//   weights: the 1 KB each row tile contributes to the block, lane l's 16 bytes at 16 l (the
//        bytes lane l reads back): whole lines when the weight is held lane-ordered (TW, the
//        planner's copy of a constant weight), 32 B from each of 32 rows otherwise;
//   scale (and min) rows: the work-group's [RW][ng] rows as they lie in the tables, once.
// Every operand arrives by DMA, so the kernel orders them with explicit vmcnt waits alone; a
// compiler-visible load among them would get the compiler's own wait, which does not count the
// DMAs and would wait for the next block's as well.
template <bool SYM, int AT, int NT, int MT, bool TW>
__global__ void __launch_bounds__(QMM_NW * 64) quant_mm_fused_k(QuantArgs a) {
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
  typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
  constexpr uint32_t PMASK = 0x000F000Fu;
  constexpr uint32_t MAGIC = AT == GT_BF16 ? 0x43004300u : 0x64006400u;
  constexpr float MAGICV = AT == GT_BF16 ? 128.f : 1024.f;
  constexpr uint32_t CX = MAGIC | (SYM ? 0x00080008u : 0u);
  constexpr float OFF = SYM ? 8.f : 0.f;
  constexpr uint32_t ONES = AT == GT_BF16 ? 0x3F803F80u : 0x3C003C00u;
  constexpr uint32_t SEL[2] = {0x05040100u, 0x07060302u};  // v_perm_b32: half p of src1 | half p of src0
  constexpr int RW = 32 * NT, MP = 32 * MT;
  constexpr int ABYTES = MP * 128, SBYTES = ABYTES + NT * 1024;  // one stage: act block + weight blocks
  constexpr int NDA = ABYTES / 1024, NDS = NDA + NT;               // act DMAs, all DMAs of a stage
  extern __shared__ __attribute__((aligned(1024))) unsigned char qmm_lds[];
  KU_LDS unsigned char* lds = (KU_LDS unsigned char*)qmm_lds;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, h = lane >> 5;
  const int64_t K = a.k, N = a.n, M = a.m, rb = K / 2, ng = K / a.group;
  const int64_t n0 = (int64_t)blockIdx.x * RW;
  // LDS: scale rows [RW][ng] f16, min rows after them (both 1 KB aligned), then two stage buffers
  // per wave; the wave partials of the end reuse it from the start
  const uint32_t tbl = (uint32_t)(RW * ng * 2), tblr = (tbl + 1023u) & ~1023u;
  KU_LDS unsigned char* st0 = lds + (SYM ? tblr : 2 * tblr) + wave * 2 * SBYTES;
  KU_LDS unsigned char* st1 = st0 + SBYTES;
  {
    // rows past N read 0. The byte count is rounded up to whole dwords: with an odd row count
    // and an odd ng the table's last f16 shares a dword with the next row's first, and a range
    // check made per dword would drop it. The rounding reads at most 2 bytes past the table, in
    // the same pool buffer (16-byte aligned operands, buffers whole multiples of 256 bytes).
    const uint32_t nrec = (uint32_t)(((N - n0 < RW ? N - n0 : RW) * ng * 2 + 3) & ~int64_t(3));
    const auto RS = qrsrc(a.scales + n0 * ng, nrec);
    for (uint32_t i = wave; i * 1024 < tbl; i += QMM_NW) lds_dma16(RS, i * 1024 + lane * 16, 0, lds + i * 1024);
    if constexpr (!SYM) {
      const auto RM = qrsrc(a.mins + n0 * ng, nrec);
      for (uint32_t i = wave; i * 1024 < tbl; i += QMM_NW)
        lds_dma16(RM, i * 1024 + lane * 16, 0, lds + tblr + i * 1024);
    }
  }
  const KU_LDS uint16_t* ssc = (const KU_LDS uint16_t*)lds;
  const KU_LDS uint16_t* smn = (const KU_LDS uint16_t*)(lds + tblr);
  const unsigned char* actb = static_cast<const unsigned char*>(a.act);
  const uint32_t abytes = (uint32_t)(M * K * 2);  // act rows past M read 0
  uint32_t aoff[NDA];
#pragma unroll
  for (int i = 0; i < NDA; ++i)
    aoff[i] = (uint32_t)((8 * i + (lane >> 3)) * K * 2) + (uint32_t)(((lane & 7) ^ (lane >> 3)) << 4);
  const int64_t ntiles = (N + 31) / 32, nblk = K / 64;
  const uint32_t wbytes = (uint32_t)(TW ? ntiles * nblk * 1024 : N * rb);  // tiles / rows past N read 0
  uint32_t woff[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
    woff[t] = TW ? (uint32_t)((n0 / 32 + t) * nblk * 1024 + lane * 16) : (uint32_t)((n0 + 32 * t + l32) * rb + 16 * h);
  auto issue = [&](int blk, KU_LDS unsigned char* st) __attribute__((always_inline)) {
    // the block offset moves the descriptors' bases: the range check does not see soffset
    const auto RA = qrsrc(actb + blk * 128, abytes - (uint32_t)blk * 128);
#pragma unroll
    for (int i = 0; i < NDA; ++i) lds_dma16(RA, aoff[i], 0, st + i * 1024);
    const uint32_t wo = TW ? (uint32_t)blk * 1024 : (uint32_t)blk * 32;
    const auto RW_ = qrsrc(a.qw + wo, wbytes - wo);
#pragma unroll
    for (int t = 0; t < NT; ++t) lds_dma16(RW_, woff[t], 0, st + ABYTES + t * 1024);
  };
  f32x16 acc[NT][MT], cg[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[t][mt][v] = 0.f;
  float as[MT];
  // block bb (0, 1) of a sub-group from a stage buffer: the act sums, then k-step jj of the MFMAs
  // takes word 4h + jj of each row and act pairs (p, p + 4) of the same 8 values
  auto block = [&](const KU_LDS unsigned char* st, int bb) __attribute__((always_inline)) {
    u32x4 v[MT][4], wv[NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        v[mt][q] = *(const KU_LDS u32x4*)(st + (32 * mt + l32) * 128 + (((4 * h + q) ^ (l32 & 7)) << 4));
#pragma unroll
    for (int t = 0; t < NT; ++t) wv[t] = *(const KU_LDS u32x4*)(st + ABYTES + t * 1024 + lane * 16);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if (bb == 0) as[mt] = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int i = 0; i < 4; ++i) as[mt] = dot2<AT>(v[mt][q][i], ONES, as[mt]);
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      u32x4 bf[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int p = 0; p < 4; ++p) bf[mt][p] = __builtin_amdgcn_perm(v[mt][jj][(p + 4) >> 1], v[mt][jj][p >> 1], SEL[p & 1]);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        u32x4 af;
#pragma unroll
        for (int p = 0; p < 4; ++p) af[p] = __builtin_amdgcn_bitop3_b32(wv[t][jj] >> (4 * p), CX, PMASK, 0x6c);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const f32x16 c = (bb == 0 && jj == 0) ? f32x16{} : cg[t][mt];  // the sub-group starts from zero
          if constexpr (AT == GT_BF16)
            cg[t][mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, af),
                                                                __builtin_bit_cast(bf16x8, bf[mt]), c, 0, 0, 0);
          else
            cg[t][mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, af),
                                                               __builtin_bit_cast(f16x8, bf[mt]), c, 0, 0, 0);
        }
      }
    }
  };
  // the sub-group's fold: act sum of this lane's row over both lane halves, then the scales
  auto fold = [&](int sg) __attribute__((always_inline)) {
    const int g = (int)((int64_t)sg * 128 / a.group);
    float at[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(as[mt]), __float_as_uint(as[mt]), false, false);
      at[mt] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = 32 * t + 8 * (v >> 2) + 4 * h + (v & 3);  // C row = weight row of the tile
        const float sc = f16_to_f32(ssc[r * ng + g]);
        const float mn = SYM ? 0.f : f16_to_f32(smn[r * ng + g]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          acc[t][mt][v] = fmaf(sc, fmaf(-(MAGICV + OFF), at[mt], cg[t][mt][v]), acc[t][mt][v]);
          if constexpr (!SYM) acc[t][mt][v] = fmaf(mn, at[mt], acc[t][mt][v]);
        }
      }
  };
  // each wave a contiguous run of sub-groups; block 2 sg in st0, block 2 sg + 1 in st1
  const int nsg = (int)(K / 128);
  const int spw = (nsg + QMM_NW - 1) / QMM_NW, sbeg = wave * spw, send = min(nsg, sbeg + spw);
  if (sbeg < send) {
    issue(2 * sbeg, st0);
    vm_wait<NDS>();  // this wave's scale-row DMAs, issued before the stage, have landed
  } else {
    vm_wait<0>();
  }
  __syncthreads();  // every wave's scale rows are in LDS
  for (int sg = sbeg; sg < send; ++sg) {
    issue(2 * sg + 1, st1);  // st1 was last read by the previous sub-group's second block
    vm_wait<NDS>();          // block 2 sg is in st0
    block(st0, 0);
    if (sg + 1 < send) {
      issue(2 * sg + 2, st0);
      vm_wait<NDS>();  // block 2 sg + 1 is in st1
    } else {
      vm_wait<0>();
    }
    block(st1, 1);
    fold(sg);
  }
  // partials of the waves through LDS (nothing reads the scale rows or the stages any more)
  __syncthreads();
  float* red = reinterpret_cast<float*>(qmm_lds);  // [wave][t][mt][v][lane]
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 16; ++v) red[(((wave * NT + t) * MT + mt) * 16 + v) * 64 + lane] = acc[t][mt][v];
  __syncthreads();
  constexpr int PER = NT * MT * 16 * 64;  // elements of one wave's partial
  for (int e = tid; e < PER; e += QMM_NW * 64) {
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < QMM_NW; ++w) sum += red[w * PER + e];
    const int ln = e & 63, v = (e >> 6) & 15, mt = (e >> 10) % MT, t = (e >> 10) / MT;
    const int64_t m = 32 * mt + (ln & 31);
    const int64_t n = n0 + 32 * t + 8 * (v >> 2) + 4 * (ln >> 5) + (v & 3);
    if (m < M && n < N) act_st<AT>(a.out, m * N + n, sum);
  }
}

// The lane-ordered weight of the fused kernel: wt[tile][blk][lane][16 B] = the 16 bytes lane l
// (row l % 32 of the 32-row tile, half l / 32 of the 64-value block) takes, rows past N repeating
// row N - 1 (their results are never stored). One thread per 16 bytes.
__global__ void __launch_bounds__(256) quant_tile_weights_k(const uint8_t* __restrict__ w, uint8_t* __restrict__ wt,
                                                             int64_t n, int64_t k) {
  const int64_t nblk = k / 64, ntiles = (n + 31) / 32, rb = k / 2;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (tile, blk, lane), lane fastest
  if (i >= ntiles * nblk * 64) return;
  const int lane = (int)(i & 63);
  const int64_t blk = (i >> 6) % nblk, tile = (i >> 6) / nblk;
  const int64_t row = tile * 32 + (lane & 31) < n ? tile * 32 + (lane & 31) : n - 1;
  *reinterpret_cast<u32x4*>(wt + i * 16) = *reinterpret_cast<const u32x4*>(w + row * rb + blk * 32 + 16 * (lane >> 5));
}

// LDS bytes of the fused kernel (its stages and scale rows; the wave partials fit inside)
static size_t quant_fused_lds(int64_t m, int64_t k, int64_t group, bool sym) {
  const int nt = m <= 32 ? 2 : 1, mt = m <= 32 ? 1 : 2;
  const size_t tblr = ((size_t)(32 * nt * (k / group) * 2) + 1023) & ~(size_t)1023;
  return (sym ? 1 : 2) * tblr + (size_t)QMM_NW * 2 * (32 * mt * 128 + nt * 1024);
}

template <bool SYM, int AT, int NT, int MT>
void launch_fused(const QuantArgs& a, hipStream_t s) {
  const size_t lds = quant_fused_lds(a.m, a.k, a.group, SYM);
  const dim3 grid((unsigned)((a.n + 32 * NT - 1) / (32 * NT)));
  if (a.qw_tiled) hipLaunchKernelGGL((quant_mm_fused_k<SYM, AT, NT, MT, true>), grid, dim3(QMM_NW * 64), lds, s, a);
  else hipLaunchKernelGGL((quant_mm_fused_k<SYM, AT, NT, MT, false>), grid, dim3(QMM_NW * 64), lds, s, a);
}

template <bool SYM, int AT, int NT, int MT>
void launch_mm(const QuantArgs& a, hipStream_t s) {
  const int64_t ng = a.k / a.group;
  {
    const int gb = a.group % 128 == 0 ? 2 : 1;
    const int64_t nthreads = a.k / (64 * gb) * quant_act_rows(a.m) * 2;
    const dim3 pg((unsigned)((nthreads + 63) / 64));
    const uint16_t* act = static_cast<const uint16_t*>(a.act);
    uint32_t* actp = static_cast<uint32_t*>(a.mm_scratch);
    float* sums = reinterpret_cast<float*>(static_cast<unsigned char*>(a.mm_scratch) + quant_actp_bytes(a.m, a.k));
    if (gb == 2) hipLaunchKernelGGL((quant_act_prep_k<AT, 2>), pg, dim3(64), 0, s, act, actp, sums, a.m, a.k);
    else hipLaunchKernelGGL((quant_act_prep_k<AT, 1>), pg, dim3(64), 0, s, act, actp, sums, a.m, a.k);
  }
  const size_t lds = std::max<size_t>((size_t)ng * 32 * NT * 2 * (SYM ? 1 : 2), (size_t)QMM_NW * NT * MT * 16 * 64 * 4);
  const dim3 grid((unsigned)((a.n + 32 * NT - 1) / (32 * NT)));
  // sub-groups of two 64-value blocks when the scale group allows
  if (a.group % 128 == 0) hipLaunchKernelGGL((quant_mm_k<SYM, AT, NT, MT, 2>), grid, dim3(QMM_NW * 64), lds, s, a);
  else hipLaunchKernelGGL((quant_mm_k<SYM, AT, NT, MT, 1>), grid, dim3(QMM_NW * 64), lds, s, a);
}

template <bool SYM, int AT>
void mm_at(const QuantArgs& a, hipStream_t s) {
  if (quant_mm_fused_ok(a)) {
    if (a.m <= 32) launch_fused<SYM, AT, 2, 1>(a, s);
    else launch_fused<SYM, AT, 1, 2>(a, s);
  } else if (a.m <= 32) {
    launch_mm<SYM, AT, 2, 1>(a, s);
  } else {
    launch_mm<SYM, AT, 1, 2>(a, s);
  }
}

// one thread per packed byte of the weight: its 8/BITS values into wdq [N, K] (dtype WT)
template <int BITS, bool SYM, int WT>
__global__ void __launch_bounds__(256) quant_dequant_k(QuantArgs a) {
  constexpr int PER = 8 / BITS;
  const int64_t rb = a.k * BITS / 8, ng = a.k / a.group;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.n * rb) return;
  const int64_t n = i / rb, k0 = (i % rb) * PER;
  const uint32_t b = a.qw[i];
#pragma unroll
  for (int f = 0; f < PER; ++f) {
    const int64_t gi = n * ng + (k0 + f) / a.group;
    const float s = f16_to_f32(a.scales[gi]);
    const float mn = SYM ? 0.f : f16_to_f32(a.mins[gi]);
    act_st<WT>(a.wdq, n * a.k + k0 + f, deq<BITS, SYM>((b >> (f * BITS)) & ((1u << BITS) - 1), s, mn));
  }
}

template <int BITS, bool SYM, int AT, int MB>
void gemv_mb(const QuantArgs& a, hipStream_t s) {
  // 16 packed bytes per thread and chunk (8 for int2: E = 32 values either way) when rows are
  // whole chunks and groups whole chunks; otherwise single bytes (one group per byte when the
  // group is a multiple of the fields per byte, else a group lookup per value)
  constexpr int CB = BITS == 2 ? 8 : 16, PER = 8 / BITS;
  const int64_t rb = a.k * BITS / 8;
  const int kind = (rb % CB == 0 && a.group % (CB * PER) == 0) ? 0 : (a.group % PER == 0 ? 1 : 2);
  const int64_t nch = kind == 0 ? rb / CB : rb;
  const int nwv = (int)std::min<int64_t>(4, std::max<int64_t>(1, (nch + 63) / 64));
  const dim3 grid((unsigned)((a.n + GEMV_RW - 1) / GEMV_RW)), block((unsigned)(nwv * 64));
  if (kind == 0) hipLaunchKernelGGL((quant_gemv_fast_k<BITS, SYM, AT, MB>), grid, block, 0, s, a);
  else if (kind == 1) hipLaunchKernelGGL((quant_gemv_k<BITS, SYM, AT, MB, 1, true>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((quant_gemv_k<BITS, SYM, AT, MB, 1, false>), grid, block, 0, s, a);
}

template <int BITS, bool SYM, int AT>
void gemv_at(const QuantArgs& a, hipStream_t s) {
  switch (a.m) {
    case 1: gemv_mb<BITS, SYM, AT, 1>(a, s); return;
    case 2: gemv_mb<BITS, SYM, AT, 2>(a, s); return;
    case 3:
    case 4: gemv_mb<BITS, SYM, AT, 4>(a, s); return;
    default: gemv_mb<BITS, SYM, AT, 8>(a, s); return;
  }
}

template <int BITS, bool SYM>
void gemv_bits(const QuantArgs& a, hipStream_t s) {
  switch (a.act_type) {
    case GT_F32: gemv_at<BITS, SYM, GT_F32>(a, s); return;
    case GT_BF16: gemv_at<BITS, SYM, GT_BF16>(a, s); return;
    default: gemv_at<BITS, SYM, GT_F16>(a, s); return;
  }
}

template <int BITS, bool SYM>
void dequant_bits(const QuantArgs& a, hipStream_t s) {
  const int64_t total = a.n * (a.k * BITS / 8);
  const dim3 grid((unsigned)((total + 255) / 256));
  switch (a.wdq_type) {
    case GT_F32: hipLaunchKernelGGL((quant_dequant_k<BITS, SYM, GT_F32>), grid, dim3(256), 0, s, a); return;
    case GT_BF16: hipLaunchKernelGGL((quant_dequant_k<BITS, SYM, GT_BF16>), grid, dim3(256), 0, s, a); return;
    default: hipLaunchKernelGGL((quant_dequant_k<BITS, SYM, GT_F16>), grid, dim3(256), 0, s, a); return;
  }
}

void check(const QuantArgs& a) {
  if (!(a.bits == 2 || a.bits == 4 || a.bits == 8)) throw std::runtime_error("quant: bits must be 2, 4 or 8");
  if (a.group <= 0 || a.k % a.group) throw std::runtime_error("quant: group must divide K");
  if (!(a.act_type == GT_F32 || a.act_type == GT_BF16 || a.act_type == GT_F16))
    throw std::runtime_error("quant: act must be f32, bf16 or f16");
  if (a.k * a.bits % 8) throw std::runtime_error("quant: K * bits must be whole bytes");
  if (!a.sym && !a.mins) throw std::runtime_error("quant: asymmetric weights need mins");
}

}  // namespace

bool quant_gemv_ok(const QuantArgs& a) { return a.m >= 1 && a.m <= 8; }

void launch_quant_gemv(const QuantArgs& a, hipStream_t s) {
  check(a);
  if (a.n * (a.k / a.group) >= (int64_t(1) << 31) || a.k >= (int64_t(1) << 31))
    throw std::runtime_error("quant: scale table or K too large for the GEMV kernel's 32-bit indices");
  if (!quant_gemv_ok(a)) throw std::runtime_error("quant: the GEMV kernel takes M <= 8");
  if (a.n == 0) return;
  if (reinterpret_cast<uintptr_t>(a.qw) & 15)
    throw std::runtime_error("quant: packed weight must be 16-byte aligned");
  switch (a.bits * 2 + (a.sym ? 1 : 0)) {
    case 5: gemv_bits<2, true>(a, s); return;
    case 4: gemv_bits<2, false>(a, s); return;
    case 9: gemv_bits<4, true>(a, s); return;
    case 8: gemv_bits<4, false>(a, s); return;
    case 17: gemv_bits<8, true>(a, s); return;
    default: gemv_bits<8, false>(a, s); return;
  }
}

// LDS bytes of the fused MFMA kernel: the staged scale (and min) table, or the wave partials
static size_t quant_mm_lds(const QuantArgs& a) {
  const int nt = a.m <= 32 ? 2 : 1, mt = a.m <= 32 ? 1 : 2;
  return std::max<size_t>((size_t)(a.k / a.group) * 32 * nt * 2 * (a.sym ? 1 : 2), (size_t)QMM_NW * nt * mt * 16 * 64 * 4);
}

bool quant_mm_ok(const QuantArgs& a) {
  if (const char* e = std::getenv("KURUMI_HIP_NO_MFMA"); e && *e && *e != '0') return false;
  return a.bits == 4 && (a.act_type == GT_BF16 || a.act_type == GT_F16) && a.m > 8 && a.m <= 64 && a.group > 0 &&
         a.group % 64 == 0 && a.k % a.group == 0 && a.k < (int64_t(1) << 31) && quant_mm_lds(a) <= 160 * 1024 &&
         (a.sym || a.mins);
}

bool quant_mm_fused_ok(const QuantArgs& a) {
  if (!quant_mm_ok(a) || a.group % 128 != 0) return false;
  // 32-bit buffer offsets and byte counts, including the rows / tiles a last work-group's lanes
  // address past N (64 rows at most)
  const int64_t lim = int64_t(1) << 31;
  return quant_act_rows(a.m) * a.k * 2 < lim && (a.n + 64) * (a.k / 2) < lim && a.n * (a.k / a.group) * 2 < lim &&
         quant_fused_lds(a.m, a.k, a.group, a.sym) <= 160 * 1024;
}

size_t quant_tiled_bytes(int64_t n, int64_t k) { return (size_t)((n + 31) / 32 * (k / 64) * 1024); }

void launch_quant_tile_weights(const uint8_t* qw, uint8_t* wt, int64_t n, int64_t k, hipStream_t s) {
  if (n <= 0 || k <= 0 || k % 64) throw std::runtime_error("quant: tiling needs n > 0 and k a multiple of 64");
  if ((reinterpret_cast<uintptr_t>(qw) & 15) || (reinterpret_cast<uintptr_t>(wt) & 15))
    throw std::runtime_error("quant: packed weight and its tiled copy must be 16-byte aligned");
  const int64_t threads = (int64_t)(quant_tiled_bytes(n, k) / 16);
  hipLaunchKernelGGL(quant_tile_weights_k, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, qw, wt, n, k);
}

size_t quant_mm_scratch_bytes(const QuantArgs& a) {
  if (quant_mm_fused_ok(a)) return 0;  // the fused kernel stages act itself
  const int64_t nsg = a.k / (64 * (a.group % 128 == 0 ? 2 : 1));
  return quant_actp_bytes(a.m, a.k) + (size_t)(nsg * quant_act_rows(a.m) * 2) * sizeof(float);
}

void launch_quant_mm(const QuantArgs& a, hipStream_t s) {
  check(a);
  if (!quant_mm_ok(a)) throw std::runtime_error("quant: shape not supported by the fused MFMA kernel");
  if (a.n == 0) return;
  const bool fused = quant_mm_fused_ok(a);
  if (a.qw_tiled && !fused) throw std::runtime_error("quant: a lane-ordered weight needs the fused MFMA kernel");
  if (!fused && (!a.mm_scratch || (reinterpret_cast<uintptr_t>(a.mm_scratch) & 15)))
    throw std::runtime_error("quant: the MFMA path needs a 16-byte aligned scratch of quant_mm_scratch_bytes()");
  if ((reinterpret_cast<uintptr_t>(a.qw) & 15) || (reinterpret_cast<uintptr_t>(a.act) & 15))
    throw std::runtime_error("quant: packed weight and act must be 16-byte aligned");
  if (a.sym) {
    if (a.act_type == GT_BF16) mm_at<true, GT_BF16>(a, s);
    else mm_at<true, GT_F16>(a, s);
  } else {
    if (a.act_type == GT_BF16) mm_at<false, GT_BF16>(a, s);
    else mm_at<false, GT_F16>(a, s);
  }
}

void launch_quant_dequant(const QuantArgs& a, hipStream_t s) {
  check(a);
  if (a.n == 0 || a.k == 0) return;
  switch (a.bits * 2 + (a.sym ? 1 : 0)) {
    case 5: dequant_bits<2, true>(a, s); return;
    case 4: dequant_bits<2, false>(a, s); return;
    case 9: dequant_bits<4, true>(a, s); return;
    case 8: dequant_bits<4, false>(a, s); return;
    case 17: dequant_bits<8, true>(a, s); return;
    default: dequant_bits<8, false>(a, s); return;
  }
}

}  // namespace ku::hipbk
