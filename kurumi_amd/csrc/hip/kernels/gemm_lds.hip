// MFMA GEMM with direct-to-LDS staging for gfx950 (kernel family 2):
// C[b][m][n] = alpha * colscale[n] * sum_k A[b][m][k] * B[b][k][n], f32 accumulation, one rounding.
//
// Stages of 128 K-bytes go from global memory straight into LDS with global_load_lds_dwordx4
// (lane l of a wave writes bytes 16l..16l+15 of the wave's 1 KB destination), double-buffered
// with one barrier per stage, so no registers or VALU work are spent on staging. Because the LDS
// position of every 16-byte chunk is fixed by the lane, the bank-conflict-avoiding layout is
// chosen on the global side: each lane fetches the chunk that belongs at its swizzled position.
//   A, and B when k-contiguous ("NT"): rows of 128 B, chunk c of row r stored at c ^ ((r / 2) % 8),
//     so any 16 consecutive rows read at one logical chunk hit 16 distinct 16-byte bank groups.
//   B when n-contiguous ("NN", [k][n] row-major): rows of BN*2 bytes kept n-major, 16-byte chunk c
//     of k-row r stored at c ^ 4(r % 4); fragments are read with ds_read_b64_tr_b16, which hands
//     each lane 4 consecutive k values of one column (two reads make the 8 a bf16 MFMA takes).
// The MFMAs produce C^T tiles (B fragment as the A operand) so that each lane ends up with runs
// of 4 consecutive output columns; the epilogue parks them in LDS and writes whole 128-byte row
// segments.
// bf16/f16 use v_mfma_f32_32x32x16_{bf16,f16}; OCP e4m3 uses v_mfma_f32_32x32x64_f8f6f4 (NT).
// Rows and columns past M and N are clamped on load (their results are never stored), so every
// load is in bounds. Work-groups are remapped so the tiles resident on one XCD share A rows and
// B columns in its L2. Semantics: kurumi_core/src/interp/contract.rs:26-64.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <string>
#include <type_traits>

#include "kernels.h"
#include "lds_dma.h"
#include "numeric.h"

namespace ku::hipbk {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((__vector_size__(4 * sizeof(short))));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
#define KU_LDS __attribute__((address_space(3)))

enum Elem : int { E_BF16 = 0, E_F16 = 1, E_FP8 = 2 };

constexpr int KB = 128;  // K bytes per stage (one row of an A/B^T stage)

template <int E>
struct Op;
template <>
struct Op<E_BF16> {
  static constexpr int KSTEP = 32;  // K bytes per MFMA (16 bf16)
  static constexpr int LV = 1;      // 16-byte pieces per lane per operand
  __device__ static void run(f32x16& c, const u32x4* a, const u32x4* b) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a[0]), __builtin_bit_cast(bf16x8, b[0]), c,
                                                0, 0, 0);
  }
};
template <>
struct Op<E_F16> {
  static constexpr int KSTEP = 32;
  static constexpr int LV = 1;
  __device__ static void run(f32x16& c, const u32x4* a, const u32x4* b) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a[0]), __builtin_bit_cast(f16x8, b[0]), c, 0,
                                               0, 0);
  }
};
template <>
struct Op<E_FP8> {
  static constexpr int KSTEP = 64;  // 64 e4m3 per MFMA
  static constexpr int LV = 2;
  __device__ static void run(f32x16& c, const u32x4* a, const u32x4* b) {
    i32x8 av, bv;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      av[i] = (int)a[0][i];
      av[4 + i] = (int)a[1][i];
      bv[i] = (int)b[0][i];
      bv[4 + i] = (int)b[1][i];
    }
    // format 0 = e4m3 for both operands; zero scales select the unscaled instruction
    c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, c, 0, 0, 0, 0, 0, 0);
  }
};

// two f32 -> one dword of two 16-bit floats, round to nearest even, in one packed conversion
// (v_cvt_pk_bf16_f32 / the f16 pair form) rather than a conversion, shift and or per value
template <int OT>
__device__ __forceinline__ uint32_t pack_out(float lo, float hi) {
  const f32x2 v = {lo, hi};
  if constexpr (OT == GT_BF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  else return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}

template <int OT>
__device__ __forceinline__ void store_out(void* c, int64_t idx, float v) {
  if constexpr (OT == GT_BF16) static_cast<uint16_t*>(c)[idx] = d_bf16_st(v);
  else if constexpr (OT == GT_F16) static_cast<uint16_t*>(c)[idx] = d_f16_st(v);
  else static_cast<float*>(c)[idx] = v;
}

// consecutive ids go to XCD id % 8: regroup them into contiguous ranges per XCD, then walk tiles
// in groups of GM tile-rows so the tiles running together reuse A rows and B columns
__device__ __forceinline__ void tile_of(int pid, int tm, int tn, int* im, int* in) {
  const int total = tm * tn;
  const int per = total / 8;
  if (pid < per * 8) pid = (pid % 8) * per + pid / 8;
  constexpr int GM = 8;
  const int group = pid / (GM * tn);
  const int first = group * GM;
  const int gs = min(tm - first, GM);
  const int r = pid % (GM * tn);
  *im = first + r % gs;
  *in = r / gs;
}

__device__ __forceinline__ void dma16(const void* g, KU_LDS unsigned char* l) { lds_dma16_g(g, (KU_LDS void*)l); }
// Buffer-resource form of the same DMA: a per-lane 32-bit offset that stays fixed across stages
// plus the stage's uniform offset in an SGPR (no 64-bit per-lane address arithmetic per stage;
// measured 9 % faster on the cfg 3 GEMM). Used when every operand byte lies within 2^31 of the
// batch's base.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t gemm_rsrc(const void* p) {
  // dword3 0x00020000: 32-bit data format, the raw-buffer setting for gfx9 parts
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ void bdma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, KU_LDS unsigned char* l) {
  lds_dma16(r, voff, soff, (KU_LDS void*)l);
}

template <int E, bool BNMAJ, int OT, int BM, int BN, int WM, int WN, bool BUF, int OCC>
__global__ void __launch_bounds__(WM* WN * 64)
    __attribute__((amdgpu_waves_per_eu(OCC, OCC))) gemm_lds_k(GemmArgs a) {
  constexpr int NW = WM * WN, NT = NW * 64;
  constexpr int EB = (E == E_FP8) ? 1 : 2;
  constexpr int KE = KB / EB;  // K elements per stage
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;
  constexpr int KSTEP = Op<E>::KSTEP, LV = Op<E>::LV, NKS = KB / KSTEP;
  constexpr int ABYTES = BM * KB, BBYTES = BN * KB;  // NN: KE rows of BN*2 bytes, the same size
  constexpr int AI = ABYTES / 1024 / NW;             // 1 KB DMA blocks per wave per stage
  constexpr int BI = BBYTES / 1024 / NW;
  constexpr int NROW = BN * 2;         // NN: bytes per k-row
  constexpr int NCH = NROW / 16;       // NN: 16-byte chunks per k-row
  constexpr int NRPB = 1024 / NROW;    // NN: k-rows per 1 KB block
  static_assert(AI * NW * 1024 == ABYTES && BI * NW * 1024 == BBYTES, "stage / wave mismatch");
  static_assert(!BNMAJ || (E != E_FP8 && NCH >= 16 && NRPB >= 1 && NRPB * NROW == 1024), "NN layout");
  __shared__ __attribute__((aligned(1024))) unsigned char lds_raw[2 * (ABYTES + BBYTES)];
  KU_LDS unsigned char* lds = (KU_LDS unsigned char*)lds_raw;

  // the wave index is uniform: kept in an SGPR, the DMA destinations (M0) need no VALU work
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), h = lane >> 5,
            l32 = lane & 31;
  const int wm = wave / WN, wn = wave % WN;
  const int tm = (int)((a.m + BM - 1) / BM), tn = (int)((a.n + BN - 1) / BN);
  int im, in;
  tile_of(blockIdx.x, tm, tn, &im, &in);
  const int64_t m0 = (int64_t)im * BM, n0 = (int64_t)in * BN;
  const int64_t bz = blockIdx.y;
  const unsigned char* A = static_cast<const unsigned char*>(a.a) + bz * a.sab * EB;
  const unsigned char* B = static_cast<const unsigned char*>(a.b) + bz * a.sbb * EB;
  const int KT = (int)(a.k / KE);

  // per-lane global sources of this lane's DMA chunks (stage 0; later stages add kt * stride)
  const unsigned char* asrc[AI];
#pragma unroll
  for (int i = 0; i < AI; ++i) {
    const int blk = i * NW + wave, r = blk * 8 + (lane >> 3), c = (lane & 7) ^ ((r >> 1) & 7);
    const int64_t gm = m0 + r < a.m ? m0 + r : a.m - 1;
    asrc[i] = A + gm * a.sam * EB + c * 16;
  }
  const unsigned char* bsrc[BI];
  int64_t bstep;  // bytes between consecutive stages
  if constexpr (!BNMAJ) {
#pragma unroll
    for (int i = 0; i < BI; ++i) {
      const int blk = i * NW + wave, r = blk * 8 + (lane >> 3), c = (lane & 7) ^ ((r >> 1) & 7);
      const int64_t gn = n0 + r < a.n ? n0 + r : a.n - 1;
      bsrc[i] = B + gn * a.sbn * EB + c * 16;
    }
    bstep = KB;
  } else {
#pragma unroll
    for (int i = 0; i < BI; ++i) {
      const int blk = i * NW + wave, r = blk * NRPB + lane / NCH, c = (lane % NCH) ^ (4 * (r & 3));
      const int64_t gn = n0 + c * 8 < a.n ? n0 + c * 8 : a.n - 8;
      bsrc[i] = B + ((int64_t)r * a.sbk + gn) * 2;
    }
    bstep = (int64_t)KE * a.sbk * 2;
  }
  [[maybe_unused]] __amdgpu_buffer_rsrc_t RA, RB;
  [[maybe_unused]] uint32_t aoff[AI], boff[BI];
  if constexpr (BUF) {
    RA = gemm_rsrc(A);
    RB = gemm_rsrc(B);
#pragma unroll
    for (int i = 0; i < AI; ++i) aoff[i] = (uint32_t)(asrc[i] - A);
#pragma unroll
    for (int i = 0; i < BI; ++i) boff[i] = (uint32_t)(bsrc[i] - B);
  }
  auto issue = [&](int kt, int buf) {
    KU_LDS unsigned char* L = lds + buf * (ABYTES + BBYTES);
    if constexpr (BUF) {
#pragma unroll
      for (int i = 0; i < AI; ++i) bdma16(RA, aoff[i], (uint32_t)(kt * KB), L + (i * NW + wave) * 1024);
#pragma unroll
      for (int i = 0; i < BI; ++i) bdma16(RB, boff[i], (uint32_t)(kt * bstep), L + ABYTES + (i * NW + wave) * 1024);
    } else {
#pragma unroll
      for (int i = 0; i < AI; ++i) dma16(asrc[i] + (int64_t)kt * KB, L + (i * NW + wave) * 1024);
#pragma unroll
      for (int i = 0; i < BI; ++i) dma16(bsrc[i] + (int64_t)kt * bstep, L + ABYTES + (i * NW + wave) * 1024);
    }
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // fragment reads from one stage
  auto afrags = [&](const KU_LDS unsigned char* L, int ks, u32x4 (&fa)[FM][LV]) {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int r = wm * TM + i * 32 + l32;
#pragma unroll
      for (int v = 0; v < LV; ++v) {
        const int c = ks * (KSTEP / 16) + h * LV + v;
        fa[i][v] = *(const KU_LDS u32x4*)(L + r * KB + ((c ^ ((r >> 1) & 7)) << 4));
      }
    }
  };
  auto bfrags_nt = [&](const KU_LDS unsigned char* L, int ks, u32x4 (&fb)[FN][LV]) {
    const KU_LDS unsigned char* LB = L + ABYTES;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int r = wn * TN + j * 32 + l32;
#pragma unroll
      for (int v = 0; v < LV; ++v) {
        const int c = ks * (KSTEP / 16) + h * LV + v;
        fb[j][v] = *(const KU_LDS u32x4*)(LB + r * KB + ((c ^ ((r >> 1) & 7)) << 4));
      }
    }
  };
  // NN: ds_read_b64_tr_b16 -- in each 16-lane group, input lane 4k'+q points at k-row k',
  // columns 4q..4q+3, and output lane i then holds rows 0..3 of column i
  auto bfrag_nn = [&](const KU_LDS unsigned char* L, int ks, int j) {
    const KU_LDS unsigned char* LB = L + ABYTES;
    const int g = lane >> 4, c16 = lane & 15;
    const int n = wn * TN + j * 32 + (g & 1) * 16 + (c16 & 3) * 4;
    u32x2 half[2];
#pragma unroll
    for (int r2 = 0; r2 < 2; ++r2) {
      const int k = ks * 16 + (g >> 1) * 8 + r2 * 4 + (c16 >> 2);
      const KU_LDS unsigned char* p = LB + k * NROW + (((n >> 3) ^ (4 * (k & 3))) << 4) + (n & 7) * 2;
      half[r2] = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((KU_LDS s16x4*)p));
    }
    return u32x4{half[0][0], half[0][1], half[1][0], half[1][1]};
  };

  if (KT > 0) issue(0, 0);
  vm_wait<0>();
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    const KU_LDS unsigned char* L = lds + cur * (ABYTES + BBYTES);
    if constexpr (BNMAJ) {
      // The transposing reads are not known to the compiler to miss the buffer the next stage's
      // DMA fills, so they all go ahead of that DMA (a later one would wait for it).
      u32x4 bst[NKS][FN];
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
        for (int j = 0; j < FN; ++j) bst[ks][j] = bfrag_nn(L, ks, j);
      if (kt + 1 < KT) issue(kt + 1, cur ^ 1);
      u32x4 af[2][FM][LV];
      afrags(L, 0, af[0]);
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        if (ks + 1 < NKS) afrags(L, ks + 1, af[(ks + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) Op<E>::run(acc[i][j], &bst[ks][j], af[ks & 1][i]);
      }
    } else {
      if (kt + 1 < KT) issue(kt + 1, cur ^ 1);
      // fragments double-buffered across k-steps: step ks+1's LDS reads run under step ks's MFMAs
      u32x4 af[2][FM][LV], bfr[2][FN][LV];
      afrags(L, 0, af[0]);
      bfrags_nt(L, 0, bfr[0]);
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        if (ks + 1 < NKS) {
          afrags(L, ks + 1, af[(ks + 1) & 1]);
          bfrags_nt(L, ks + 1, bfr[(ks + 1) & 1]);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) Op<E>::run(acc[i][j], bfr[ks & 1][j], af[ks & 1][i]);
      }
    }
    // this thread's DMA for stage kt+1 has landed; the barrier publishes it and retires stage kt
    vm_wait<0>();
    __syncthreads();
  }

  // Epilogue. The MFMAs computed C^T tiles (B fragment as the A operand): lane l32 owns row
  // i*32 + l32 of the wave's TM x TN block and, in register group g of tile j, the 4 columns
  // j*32 + 8g + 4h + 0..3. Scaled values are rounded, parked in LDS (the stage buffers are free
  // after the loop's last barrier) and written back row-contiguous, 16 bytes per lane and 128
  // bytes per row and instruction.
  const float alpha = a.alpha ? a.alpha[0] : 1.f;
  const int rt = a.round_type;  // a fused cast from the contraction's 16-bit dtype
  void* C = static_cast<unsigned char*>(a.c) + bz * a.m * a.n * (OT == GT_F32 ? 4 : 2);
  const int64_t rbase = m0 + wm * TM, cbase = n0 + wn * TN;
  float cs[FN][4][4];  // column scales of this lane's columns
  if (a.col_scale) {
    // one uniform branch around all loads, so they are issued back to back and waited for once
    // (a test per element put each load in its own block, waited for on its own)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t col = cbase + j * 32 + g * 8 + h * 4 + e;
          cs[j][g][e] = a.col_scale[(col < a.n ? col : a.n - 1) * a.col_scale_stride];
        }
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) cs[j][g][e] *= alpha;
  } else {
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) cs[j][g][e] = alpha;
  }
  if constexpr (OT != GT_F32) {
    constexpr int ROWB = TN * 2;          // bytes per staged row
    constexpr int UPR = ROWB / 8;         // 8-byte units per row
    static_assert(UPR == 16 && TM * ROWB * NW <= 2 * (ABYTES + BBYTES), "epilogue staging");
    KU_LDS unsigned char* EP = lds + wave * TM * ROWB;
    // unit u of row r sits at u ^ ((r / 2) % 16): the 32 rows one write touches cover all banks
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int r = i * 32 + l32;
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int u = j * 8 + g * 2 + h;
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * g + e] * cs[j][g][e];
          if (rt >= 0) {  // uniform branch
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = d_round_through(rt, v[e]);
          }
          u32x2 w;
          w[0] = pack_out<OT>(v[0], v[1]);
          w[1] = pack_out<OT>(v[2], v[3]);
          *(KU_LDS u32x2*)(EP + r * ROWB + ((u ^ ((r >> 1) & 15)) << 3)) = w;
        }
    }
    // each wave reads back only its own block: no barrier needed beyond the LDS wait
    const bool vec8 = (a.n & 7) == 0;
#pragma unroll
    for (int q = 0; q < TM / 8; ++q) {
      const int r = q * 8 + (lane >> 3), c = lane & 7;
      const int sw = (r >> 1) & 15;
      const u32x2 lo = *(const KU_LDS u32x2*)(EP + r * ROWB + (((2 * c) ^ sw) << 3));
      const u32x2 hi = *(const KU_LDS u32x2*)(EP + r * ROWB + (((2 * c + 1) ^ sw) << 3));
      const int64_t row = rbase + r, col = cbase + c * 8;
      if (row >= a.m || col >= a.n) continue;
      uint16_t* dst = static_cast<uint16_t*>(C) + row * a.n + col;
      if (vec8 && col + 8 <= a.n) {
        *reinterpret_cast<u32x4*>(dst) = u32x4{lo[0], lo[1], hi[0], hi[1]};
      } else {
        const uint32_t w4[4] = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (col + e < a.n) dst[e] = (uint16_t)(w4[e >> 1] >> ((e & 1) * 16));
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int64_t row = rbase + i * 32 + l32;
      if (row >= a.m) continue;
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int64_t col = cbase + j * 32 + g * 8 + h * 4;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (col + e < a.n)
              static_cast<float*>(C)[row * a.n + col + e] = d_round_through(rt, acc[i][j][4 * g + e] * cs[j][g][e]);
        }
    }
  }
}

// Persistent small-K GEMM (K of one or two 128-byte stages, e.g. the batched [8, 2048, 128] x
// [8, 128, 2048] product): C is the traffic (K = 128 writes 8x the bytes it reads), so the kernel
// is built to keep C stores streaming. One work-group of 8 waves per CU takes a contiguous run of
// 128 x 128 tiles in (batch, tile row, tile column) order, so consecutive tiles share their A
// rows: A is loaded once per tile row, B (all K stages) two tiles ahead into a ring of three LDS
// buffers. The waves specialise. Waves 0-3 ("loaders") issue every DMA and multiply (a 64 x 64
// block each); waves 4-7 ("storers") write C. A CU's vector memory requests are served in order,
// so under streaming stores a load takes microseconds: the two tiles of lead hide that, and since
// a wave's memory operations also retire in issue order, keeping the stores in other waves lets
// the loaders wait for their loads alone (the storers never wait). Per tile t, between two
// barriers the loaders park tile t - 1's results in a staging buffer, start B of tile t + 2 and
// wait for tile t's operands; after the second barrier they multiply tile t while the storers
// read tile t - 1 back from the staging buffer and store whole 128-byte row segments. Rows or
// columns past C go to an out-of-range buffer offset (dropped).
__device__ __forceinline__ void bar_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int E, bool BNMAJ, int OT, int KT>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) gemm_smallk_k(GemmArgs a) {
  constexpr int BM = 128, BN = 128, WM = 2, WN = 2, NL = WM * WN;  // NL loader waves, then NL storers
  constexpr int EB = 2, KE = KB / EB;
  constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
  constexpr int KSTEP = Op<E>::KSTEP, LV = Op<E>::LV, NKS = KB / KSTEP;
  constexpr int SA = BM * KB, SB = BN * KB;          // one stage of A, of B (16 KB each)
  constexpr int ABUF = KT * SA, BBUF = KT * SB;      // a tile's A, B (all stages)
  constexpr int NB = 3;                              // B ring: the current tile and two ahead
  constexpr int ROWB = TN * 2;                       // bytes of one staged row of a loader's block
  constexpr int BLK = TM * ROWB;                     // one loader's staged block
  constexpr int STG = NL * BLK;                      // the staging buffer: the whole C tile
  constexpr int AIL = SA / 1024 / NL, BIL = SB / 1024 / NL;  // 1 KB DMA blocks per loader wave
  constexpr int NROW = BN * 2, NCH = NROW / 16, NRPB = 1024 / NROW;
  constexpr int LB = KT * BIL;           // B DMA operations per loader wave per tile
  constexpr int SPB = BLK / 1024;        // store operations per storer per tile
  static_assert(E != E_FP8 && OT != GT_F32 && TM == 64 && TN == 64 && ROWB == 128, "small-K layout");
  static_assert(AIL * NL * 1024 == SA && BIL * NL * 1024 == SB && NRPB * NROW == 1024, "stage / wave mismatch");
  static_assert(2 * LB <= 63 && STG == BM * BN * 2, "counters / staging");
  __shared__ __attribute__((aligned(1024))) unsigned char lds_raw[ABUF + NB * BBUF + STG];
  KU_LDS unsigned char* lds = (KU_LDS unsigned char*)lds_raw;
  KU_LDS unsigned char* LA = lds;
  KU_LDS unsigned char* LS = lds + ABUF + NB * BBUF;
  auto bbuf = [&](int slot) { return lds + ABUF + slot * BBUF; };

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), h = lane >> 5,
            l32 = lane & 31;
  const bool loader = wave < NL;
  const int lw = loader ? wave : wave - NL;  // index within the role
  const int wm = lw / WN, wn = lw % WN;
  const int tm = (int)((a.m + BM - 1) / BM), tn = (int)((a.n + BN - 1) / BN);
  const int ntile = tm * tn * (int)a.batch;
  const int per = (ntile + (int)gridDim.x - 1) / (int)gridDim.x;
  const int t0 = (int)blockIdx.x * per, t1 = min(ntile, t0 + per);
  if (t0 >= t1) return;  // the whole work-group
  const auto RC = __builtin_amdgcn_make_buffer_rsrc(a.c, (short)0, (int)(a.batch * a.m * a.n * 2), 0x00020000);
  const int rt = a.round_type;

  // tile t: batch t / (tm tn), tile row (t / tn) % tm, tile column t % tn; its A depends on t / tn
  auto load_a = [&](int t) {  // loader waves
    const int bz = t / (tm * tn);
    const int64_t m0 = (int64_t)((t / tn) % tm) * BM;
    const auto RA = gemm_rsrc(static_cast<const unsigned char*>(a.a) + bz * a.sab * EB);
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int i = 0; i < AIL; ++i) {
        const int blk = i * NL + lw, r = blk * 8 + (lane >> 3), c = (lane & 7) ^ ((r >> 1) & 7);
        const int64_t gm = m0 + r < a.m ? m0 + r : a.m - 1;
        bdma16(RA, (uint32_t)(gm * a.sam * EB + c * 16 + kt * KB), 0, LA + kt * SA + blk * 1024);
      }
  };
  auto load_b = [&](int t, int slot) {  // loader waves
    const int bz = t / (tm * tn);
    const int64_t n0 = (int64_t)(t % tn) * BN;
    const auto RBs = gemm_rsrc(static_cast<const unsigned char*>(a.b) + bz * a.sbb * EB);
    KU_LDS unsigned char* base = bbuf(slot);
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int i = 0; i < BIL; ++i) {
        const int blk = i * NL + lw;
        uint32_t off;
        if constexpr (!BNMAJ) {
          const int r = blk * 8 + (lane >> 3), c = (lane & 7) ^ ((r >> 1) & 7);
          const int64_t gn = n0 + r < a.n ? n0 + r : a.n - 1;
          off = (uint32_t)(gn * a.sbn * EB + c * 16 + kt * KB);
        } else {
          const int r = blk * NRPB + lane / NCH, c = (lane % NCH) ^ (4 * (r & 3));
          const int64_t gn = n0 + c * 8 < a.n ? n0 + c * 8 : a.n - 8;
          off = (uint32_t)((((int64_t)kt * KE + r) * a.sbk + gn) * 2);
        }
        bdma16(RBs, off, 0, base + kt * SB + blk * 1024);
      }
  };

  f32x16 acc[FM][FN];
  // loader waves: the products of tile t into acc
  auto compute = [&](int slot) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
    const KU_LDS unsigned char* LB0 = bbuf(slot);
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        u32x4 fa[FM][LV], fb[FN][LV];
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const int r = wm * TM + i * 32 + l32;
#pragma unroll
          for (int v = 0; v < LV; ++v) {
            const int c = ks * (KSTEP / 16) + h * LV + v;
            fa[i][v] = *(const KU_LDS u32x4*)(LA + kt * SA + r * KB + ((c ^ ((r >> 1) & 7)) << 4));
          }
        }
        const KU_LDS unsigned char* Lb = LB0 + kt * SB;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          if constexpr (!BNMAJ) {
            const int r = wn * TN + j * 32 + l32;
#pragma unroll
            for (int v = 0; v < LV; ++v) {
              const int c = ks * (KSTEP / 16) + h * LV + v;
              fb[j][v] = *(const KU_LDS u32x4*)(Lb + r * KB + ((c ^ ((r >> 1) & 7)) << 4));
            }
          } else {
            const int g = lane >> 4, c16 = lane & 15;
            const int n = wn * TN + j * 32 + (g & 1) * 16 + (c16 & 3) * 4;
            u32x2 hv[2];
#pragma unroll
            for (int r2 = 0; r2 < 2; ++r2) {
              const int k = ks * 16 + (g >> 1) * 8 + r2 * 4 + (c16 >> 2);
              const KU_LDS unsigned char* p = Lb + k * NROW + (((n >> 3) ^ (4 * (k & 3))) << 4) + (n & 7) * 2;
              hv[r2] = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((KU_LDS s16x4*)p));
            }
            fb[j][0] = u32x4{hv[0][0], hv[0][1], hv[1][0], hv[1][1]};
          }
        }
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) Op<E>::run(acc[i][j], fb[j], fa[i]);
      }
  };
  // loader waves: acc into this wave's block of the staging buffer. C^T tiles: lane l32 owns row
  // i*32 + l32 and, in register group g of tile j, the 4 columns j*32 + 8g + 4h + 0..3; 8-byte
  // unit u of row r sits at u ^ ((r/2) % 16)
  auto stage = [&](auto round) __attribute__((always_inline)) {
    KU_LDS unsigned char* EP = LS + lw * BLK;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int r = i * 32 + l32;
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int u = j * 8 + g * 2 + h;
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            v[e] = decltype(round)::value ? d_round_through(rt, acc[i][j][4 * g + e]) : acc[i][j][4 * g + e];
          u32x2 w;
          w[0] = pack_out<OT>(v[0], v[1]);
          w[1] = pack_out<OT>(v[2], v[3]);
          *(KU_LDS u32x2*)(EP + r * ROWB + ((u ^ ((r >> 1) & 15)) << 3)) = w;
        }
    }
  };
  // storer waves: read back loader lw's block of tile t and store it
  auto store = [&](int t) {
    const int bz = t / (tm * tn);
    const int64_t rbase = (int64_t)((t / tn) % tm) * BM + wm * TM, cbase = (int64_t)(t % tn) * BN + wn * TN;
    const KU_LDS unsigned char* EP = LS + lw * BLK;
#pragma unroll
    for (int q = 0; q < SPB; ++q) {
      const int r = q * 8 + (lane >> 3), c = lane & 7, sw = (r >> 1) & 15;
      const u32x2 lo = *(const KU_LDS u32x2*)(EP + r * ROWB + (((2 * c) ^ sw) << 3));
      const u32x2 hi = *(const KU_LDS u32x2*)(EP + r * ROWB + (((2 * c + 1) ^ sw) << 3));
      const int64_t row = rbase + r, col = cbase + c * 8;
      // n % 8 == 0: a chunk is wholly inside or outside C
      const uint32_t off = row < a.m && col < a.n ? (uint32_t)((bz * a.m * a.n + row * a.n + col) * 2) : 0x80000000u;
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{lo[0], lo[1], hi[0], hi[1]}, RC, off, 0, 0);
    }
  };

  if (loader) {
    load_a(t0);
    load_b(t0, 0);
    if (t0 + 1 < t1) load_b(t0 + 1, 1);
  }
  for (int t = t0, slot = 0; t <= t1; ++t, slot = slot == NB - 1 ? 0 : slot + 1) {
    // tile t - 1 is multiplied (every loader) and tile t - 2 read back from staging (every storer)
    bar_lds();
    if (loader) {
      if (t > t0) {
        if (rt >= 0) stage(std::true_type{});
        else stage(std::false_type{});
      }
      if (t < t1) {
        if (t > t0 && t / tn != (t - 1) / tn) {
          // a new tile row: tile t - 1 no longer needs A; reload it and wait for everything
          load_a(t);
          vm_wait<0>();
        }
        // B of tile t + 2 goes where tile t - 1's B was
        if (t + 2 < t1) load_b(t + 2, slot == 0 ? 2 : slot - 1);
        // tile t's operands; at most the B loads of tiles t + 1 and t + 2 were issued after them
        if (t + 2 < t1) vm_wait<2 * LB>();
        else if (t + 1 < t1) vm_wait<LB>();
        else vm_wait<0>();
      }
    }
    // tile t's operands and tile t - 1's staged results are in place
    bar_lds();
    if (loader) {
      if (t < t1) compute(slot);
    } else if (t > t0) {
      store(t - 1);
    }
  }
}

// every byte the kernel reads of A and of B lies within 2^31 - 1 of its batch's base
bool spans_fit(const GemmArgs& a) {
  const int64_t eb = a.in_type == GT_F8E4M3 ? 1 : 2, lim = 0x7fffffffLL;
  const int64_t aspan = ((a.m - 1) * a.sam + (a.k - 1) * a.sak + 1) * eb;
  const int64_t bspan = ((a.n - 1) * a.sbn + (a.k - 1) * a.sbk + 1) * eb;
  return aspan + 16 <= lim && bspan + 16 <= lim;
}

template <int E, bool BNMAJ, int OT, int BM, int BN, int WM, int WN, int OCC = (WM * WN + 3) / 4>
void launch_tile(const GemmArgs& a, hipStream_t s) {
  const int tm = (int)((a.m + BM - 1) / BM), tn = (int)((a.n + BN - 1) / BN);
  dim3 grid((unsigned)(tm * tn), (unsigned)a.batch);
  if (spans_fit(a))
    hipLaunchKernelGGL((gemm_lds_k<E, BNMAJ, OT, BM, BN, WM, WN, true, OCC>), grid, dim3(WM * WN * 64), 0, s, a);
  else
    hipLaunchKernelGGL((gemm_lds_k<E, BNMAJ, OT, BM, BN, WM, WN, false, OCC>), grid, dim3(WM * WN * 64), 0, s, a);
}

// One work-group per CU at a time (the stages fill the LDS), so the tiles run in rounds of
// cu_count(). 192-row tiles win when they need no more rounds than 256-row ones by enough to
// outweigh their ~10 % lower efficiency (a 96 x 64 wave tile reads more LDS per MFMA): measured
// on the e4m3 [2048, 4096] x [11008, 4096]^T linear, 344 tiles of 256 x 256 (2 rounds, the second
// a third full) 101 us vs 473 tiles of 192 x 256 (2 full rounds) 90 us; the bf16
// [4096, 4096] x [4096, 11008] GEMM keeps 256 rows (359 vs 379 us).
bool rows192(const GemmArgs& a) {
  const int64_t ncu = cu_count(), tn = (a.n + 255) / 256;
  const int64_t r256 = ((a.m + 255) / 256 * tn * a.batch + ncu - 1) / ncu;
  const int64_t r192 = ((a.m + 191) / 192 * tn * a.batch + ncu - 1) / ncu;
  return (double)r192 * 192 * 1.1 < (double)r256 * 256;
}

// small K (one or two stages): 128 x 128 tiles of 4 waves, two work-groups per CU, so one
// group's epilogue stores run under the other's loads and MFMAs
// (measured on the batched [8, 2048, 128] x [8, 128, 2048] bf16 GEMM: 31.3 -> 27.5 us against
// 256 x 256 tiles; issuing both stages up front, or storing C non-temporally, changed nothing)
bool small_k(const GemmArgs& a) {
  const int64_t kbytes = a.k * (a.in_type == GT_F8E4M3 ? 1 : 2);
  return kbytes <= 2 * 128;
}

// the persistent small-K kernel: 16-bit operands and output, no scales, whole 16-byte output
// chunks, 32-bit offsets into every operand and into C
bool smallk_persistent(const GemmArgs& a) {
  if (!small_k(a) || a.in_type == GT_F8E4M3 || a.out_type == GT_F32 || a.alpha || a.col_scale) return false;
  if (a.n % 8 || !spans_fit(a) || a.batch * a.m * a.n * 2 >= (int64_t(1) << 31)) return false;
  return (a.m + 127) / 128 * ((a.n + 127) / 128) * a.batch < (int64_t(1) << 30);
}

template <int E, bool BNMAJ, int OT>
void launch_smallk(const GemmArgs& a, hipStream_t s) {
  const int64_t tiles = (a.m + 127) / 128 * ((a.n + 127) / 128) * a.batch;
  // one work-group per CU; KURUMI_HIP_SMALLK_GRID caps the grid (the tests use it to give every
  // work-group several tiles at small shapes)
  int64_t g = std::min<int64_t>(tiles, cu_count());
  if (const char* e = std::getenv("KURUMI_HIP_SMALLK_GRID"); e && *e && std::atoll(e) > 0) g = std::min<int64_t>(g, std::atoll(e));
  if (a.k * 2 <= 128) hipLaunchKernelGGL((gemm_smallk_k<E, BNMAJ, OT, 1>), dim3((unsigned)g), dim3(512), 0, s, a);
  else hipLaunchKernelGGL((gemm_smallk_k<E, BNMAJ, OT, 2>), dim3((unsigned)g), dim3(512), 0, s, a);
}

template <int E, bool BNMAJ, int OT>
void launch_cfg(const GemmArgs& a, hipStream_t s) {
  if constexpr (E != E_FP8 && OT != GT_F32) {
    if (smallk_persistent(a)) return launch_smallk<E, BNMAJ, OT>(a, s);
  }
  if (small_k(a)) launch_tile<E, BNMAJ, OT, 128, 128, 2, 2, 2>(a, s);
  else if (rows192(a)) launch_tile<E, BNMAJ, OT, 192, 256, 2, 4>(a, s);
  else launch_tile<E, BNMAJ, OT, 256, 256, 2, 4>(a, s);
}

template <int E, bool BNMAJ>
void launch_e(const GemmArgs& a, hipStream_t s) {
  switch (a.out_type) {
    case GT_BF16: launch_cfg<E, BNMAJ, GT_BF16>(a, s); return;
    case GT_F16: launch_cfg<E, BNMAJ, GT_F16>(a, s); return;
    default: launch_cfg<E, BNMAJ, GT_F32>(a, s); return;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

int cu_count() {
  static const int n = [] {
    int dev = 0, c = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0)
      c = 256;
    return c;
  }();
  return n;
}

bool gemm_lds_ok(const GemmArgs& a) {
  if (const char* e = std::getenv("KURUMI_HIP_NO_MFMA"); e && *e && *e != '0') return false;
  const bool fp8 = a.in_type == GT_F8E4M3;
  if (!(a.in_type == GT_BF16 || a.in_type == GT_F16 || fp8)) return false;
  if (!(a.out_type == GT_BF16 || a.out_type == GT_F16 || a.out_type == GT_F32)) return false;
  const int64_t ke = fp8 ? 128 : 64, eb = fp8 ? 1 : 2, vec = 16 / eb;
  if (a.k % ke != 0 || a.k == 0 || a.m == 0 || a.n == 0) return false;
  if (a.sak != 1 || (a.m > 1 && a.sam % vec) || a.sab % vec) return false;
  const bool nt = a.sbk == 1, nn = a.sbn == 1 && !fp8;
  if (nt) {
    if ((a.n > 1 && a.sbn % vec) || a.sbb % vec) return false;
  } else if (nn) {
    if (a.sbk % vec || a.n % 8 || a.sbb % vec) return false;
  } else {
    return false;
  }
  if (a.a && (!aligned16(a.a) || !aligned16(a.b))) return false;
  return a.batch <= 65535;
}

std::string gemm_lds_name(const GemmArgs& a) {
  std::string n = a.in_type == GT_F8E4M3 ? "gemm_mfma_e4m3" : a.in_type == GT_F16 ? "gemm_mfma_f16" : "gemm_mfma_bf16";
  n += a.sbk == 1 ? "_nt" : "_nn";
  n += smallk_persistent(a) ? "_128x128_persistent" : small_k(a) ? "_128x128" : rows192(a) ? "_192x256" : "_256x256";
  if (!spans_fit(a)) n += "_a64";
  return n;
}

void launch_gemm_lds(const GemmArgs& a, hipStream_t s) {
  const bool nt = a.sbk == 1;
  if (a.in_type == GT_F8E4M3) {
    launch_e<E_FP8, false>(a, s);
  } else if (a.in_type == GT_F16) {
    if (nt) launch_e<E_F16, false>(a, s);
    else launch_e<E_F16, true>(a, s);
  } else {
    if (nt) launch_e<E_BF16, false>(a, s);
    else launch_e<E_BF16, true>(a, s);
  }
}

}  // namespace ku::hipbk
