// MFMA GEMM for gfx950 (kernel family 2): C[b][m][n] = sum_k A[b][m][k] * B[b][k][n].
//
// One kernel template serves bf16/f16 (v_mfma_f32_32x32x16_{bf16,f16}) and OCP e4m3
// (v_mfma_f32_32x32x64_f8f6f4): a K stage is 128 bytes of every A row and B column, staged
// global -> registers -> LDS (padded rows, double-buffered, one barrier per stage) while the
// previous stage feeds the MFMAs. A is k-contiguous. B is either k-contiguous ("NT", the
// linear-layer weight [n][k]) or n-contiguous ("NN", [k][n]); NN tiles are transposed in
// registers on their way into LDS so both layouts share the compute loop. Work-groups are
// remapped so that the tiles resident on one XCD at a time share A rows and B columns in that
// XCD's L2. Accumulation is f32; the epilogue applies the optional per-tensor scale and
// per-column scale (the e4m3 linear's sx * sw[n]) and rounds once to the output dtype, the
// semantics of the reference contraction (kurumi_core/src/interp/contract.rs:26-64).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdlib>
#include <string>

#include "kernels.h"
#include "numeric.h"

namespace ku::hipbk {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

enum Elem : int { E_BF16 = 0, E_F16 = 1, E_FP8 = 2 };

constexpr int KB = 128;            // K bytes per stage
constexpr int LDS_ROW = KB + 16;   // padded LDS row (bytes): rows land on distinct 16-byte banks groups

template <int E>
struct Mfma;
template <>
struct Mfma<E_BF16> {
  static constexpr int KSTEP = 32;  // K bytes consumed per MFMA per row (16 bf16)
  static constexpr int LB = 16;     // bytes per lane per operand
  __device__ static void run(f32x16& c, const u32x4* a, const u32x4* b) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a[0]), __builtin_bit_cast(bf16x8, b[0]), c,
                                                0, 0, 0);
  }
};
template <>
struct Mfma<E_F16> {
  static constexpr int KSTEP = 32;
  static constexpr int LB = 16;
  __device__ static void run(f32x16& c, const u32x4* a, const u32x4* b) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a[0]), __builtin_bit_cast(f16x8, b[0]), c, 0,
                                               0, 0);
  }
};
template <>
struct Mfma<E_FP8> {
  static constexpr int KSTEP = 64;  // 64 e4m3 per row per MFMA
  static constexpr int LB = 32;
  __device__ static void run(f32x16& c, const u32x4* a, const u32x4* b) {
    i32x8 av, bv;
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

template <int OT>
__device__ __forceinline__ void store_out(void* c, int64_t idx, float v) {
  if constexpr (OT == GT_BF16) static_cast<uint16_t*>(c)[idx] = d_bf16_st(v);
  else if constexpr (OT == GT_F16) static_cast<uint16_t*>(c)[idx] = d_f16_st(v);
  else static_cast<float*>(c)[idx] = v;
}

// Tile mapping: first spread consecutive ids across the 8 XCDs back into contiguous ranges
// (dispatch places work-group i on XCD i % 8), then walk tiles in groups of GM tile-rows so
// concurrently running tiles reuse the same A rows / B columns.
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

template <int E, bool BNMAJ, int OT, int BM, int BN, int WM, int WN>
__global__ void __launch_bounds__(WM* WN * 64)
    __attribute__((amdgpu_waves_per_eu((WM * WN + 3) / 4, (WM * WN + 3) / 4))) gemm_mfma_k(GemmArgs a) {
  constexpr int NT = WM * WN * 64;
  constexpr int EB = (E == E_FP8) ? 1 : 2;
  constexpr int KE = KB / EB;  // K elements per stage
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;
  constexpr int KSTEP = Mfma<E>::KSTEP, LB = Mfma<E>::LB, NKS = KB / KSTEP, LV = LB / 16;
  constexpr int ACH = BM * (KB / 16) / NT;  // A chunks (16 B) per thread
  constexpr int BCH = BN * (KB / 16) / NT;  // B chunks per thread
  static_assert(ACH * NT == BM * (KB / 16) && BCH * NT == BN * (KB / 16), "tile/thread mismatch");
  // NN: each thread loads R consecutive k-rows of one 8-wide n chunk and writes them transposed
  constexpr int R = BNMAJ ? KE * (BN / 8) / NT : 1;
  static_assert(!BNMAJ || (E != E_FP8 && R >= 2 && R <= 8 && R * NT == KE * (BN / 8) && R <= BCH * 2),
                "NN transpose mapping");
  __shared__ __attribute__((aligned(16))) unsigned char lds[2][(BM + BN) * LDS_ROW];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int tm = (int)((a.m + BM - 1) / BM), tn = (int)((a.n + BN - 1) / BN);
  int im, in;
  tile_of(blockIdx.x, tm, tn, &im, &in);
  const int64_t m0 = (int64_t)im * BM, n0 = (int64_t)in * BN;
  const int64_t bz = blockIdx.y;
  const unsigned char* A = static_cast<const unsigned char*>(a.a) + bz * a.sab * EB;
  const unsigned char* B = static_cast<const unsigned char*>(a.b) + bz * a.sbb * EB;
  const int KT = (int)(a.k / KE);

  u32x4 ra[ACH], rb[BCH];
  auto load = [&](int kt) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + i * NT, row = c >> 3, col = c & 7;
      const int64_t gm = m0 + row;
      ra[i] = (gm < a.m) ? *reinterpret_cast<const u32x4*>(A + gm * a.sam * EB + (int64_t)kt * KB + col * 16)
                         : u32x4{0, 0, 0, 0};
    }
    if constexpr (!BNMAJ) {
#pragma unroll
      for (int i = 0; i < BCH; ++i) {
        const int c = tid + i * NT, row = c >> 3, col = c & 7;
        const int64_t gn = n0 + row;
        rb[i] = (gn < a.n) ? *reinterpret_cast<const u32x4*>(B + gn * a.sbn * EB + (int64_t)kt * KB + col * 16)
                           : u32x4{0, 0, 0, 0};
      }
    } else {
      const int kq = tid % (KE / R), nc = tid / (KE / R);
      const int64_t gn = n0 + nc * 8;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int64_t gk = (int64_t)kt * KE + kq * R + r;
        rb[r] = (gn < a.n) ? *reinterpret_cast<const u32x4*>(B + (gk * a.sbk + gn) * EB) : u32x4{0, 0, 0, 0};
      }
    }
  };
  auto store = [&](int buf) {
    unsigned char* L = lds[buf];
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + i * NT, row = c >> 3, col = c & 7;
      *reinterpret_cast<u32x4*>(L + row * LDS_ROW + col * 16) = ra[i];
    }
    unsigned char* LBp = L + BM * LDS_ROW;
    if constexpr (!BNMAJ) {
#pragma unroll
      for (int i = 0; i < BCH; ++i) {
        const int c = tid + i * NT, row = c >> 3, col = c & 7;
        *reinterpret_cast<u32x4*>(LBp + row * LDS_ROW + col * 16) = rb[i];
      }
    } else {
      // R k-rows x 8 n-columns of 16-bit values -> 8 n-rows x R k-values; consecutive lanes take
      // consecutive k groups of one n chunk, so the 16 lanes of a write cover 64 distinct banks
      const int kq = tid % (KE / R), nc = tid / (KE / R);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int w = j >> 1, hi = (j & 1) * 16;
        uint32_t o[R / 2];
#pragma unroll
        for (int d = 0; d < R / 2; ++d)
          o[d] = ((rb[2 * d][w] >> hi) & 0xffffu) | (((rb[2 * d + 1][w] >> hi) & 0xffffu) << 16);
        unsigned char* dst = LBp + (nc * 8 + j) * LDS_ROW + kq * R * 2;
        if constexpr (R == 8) *reinterpret_cast<u32x4*>(dst) = u32x4{o[0], o[1], o[2], o[3]};
        else if constexpr (R == 4) *reinterpret_cast<u32x2*>(dst) = u32x2{o[0], o[1]};
        else *reinterpret_cast<uint32_t*>(dst) = o[0];
      }
    }
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  if (KT > 0) {
    load(0);
    store(0);
  }
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) load(kt + 1);
    const unsigned char* L = lds[cur];
    // fragments double-buffered across k-steps: the LDS reads of step ks+1 are in flight while
    // the MFMAs of step ks run
    u32x4 af[2][FM][LV], bfr[2][FN][LV];
    auto frags = [&](int ks, u32x4 (&fa)[FM][LV], u32x4 (&fb)[FN][LV]) {
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const unsigned char* p = L + (wm * TM + i * 32 + (lane & 31)) * LDS_ROW + ks * KSTEP + (lane >> 5) * LB;
#pragma unroll
        for (int v = 0; v < LV; ++v) fa[i][v] = *reinterpret_cast<const u32x4*>(p + v * 16);
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const unsigned char* p =
            L + (BM + wn * TN + j * 32 + (lane & 31)) * LDS_ROW + ks * KSTEP + (lane >> 5) * LB;
#pragma unroll
        for (int v = 0; v < LV; ++v) fb[j][v] = *reinterpret_cast<const u32x4*>(p + v * 16);
      }
    };
    frags(0, af[0], bfr[0]);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      if (ks + 1 < NKS) frags(ks + 1, af[(ks + 1) & 1], bfr[(ks + 1) & 1]);
      // keep the next step's reads issued ahead of this step's MFMAs
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) Mfma<E>::run(acc[i][j], af[ks & 1][i], bfr[ks & 1][j]);
    }
    if (kt + 1 < KT) store(cur ^ 1);
    __syncthreads();
  }

  // epilogue: lane owns column (lane & 31) and rows 8*(v/4) + 4*(lane/32) + v%4 of each 32x32 tile
  const float alpha = a.alpha ? a.alpha[0] : 1.f;
  void* C = static_cast<unsigned char*>(a.c) + bz * a.m * a.n * (OT == GT_F32 ? 4 : 2);
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int64_t col = n0 + wn * TN + j * 32 + (lane & 31);
    if (col >= a.n) continue;
    const float cs = a.col_scale ? alpha * a.col_scale[col * a.col_scale_stride] : alpha;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t row = m0 + wm * TM + i * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
        if (row < a.m) store_out<OT>(C, row * a.n + col, d_round_through(a.round_type, acc[i][j][v] * cs));
      }
    }
  }
}

template <int E, bool BNMAJ, int OT, int BM, int BN, int WM, int WN>
void launch_tile(const GemmArgs& a, hipStream_t s) {
  const int tm = (int)((a.m + BM - 1) / BM), tn = (int)((a.n + BN - 1) / BN);
  dim3 grid((unsigned)(tm * tn), (unsigned)a.batch);
  hipLaunchKernelGGL((gemm_mfma_k<E, BNMAJ, OT, BM, BN, WM, WN>), grid, dim3(WM * WN * 64), 0, s, a);
}

// Tile shape: KURUMI_HIP_GEMM_TILE=256x256 (default) | 256x128 | 128x128 | 128x256
int tile_choice() {
  static const int t = [] {
    const char* e = std::getenv("KURUMI_HIP_GEMM_TILE");
    if (!e) return 1;
    std::string v(e);
    if (v == "256x128") return 0;
    if (v == "128x128") return 2;
    if (v == "128x256") return 3;
    if (v == "256x256w8") return 4;
    return 1;
  }();
  return t;
}

template <int E, bool BNMAJ, int OT>
void launch_cfg(const GemmArgs& a, hipStream_t s) {
  switch (tile_choice()) {
    case 1: launch_tile<E, BNMAJ, OT, 256, 256, 2, 2>(a, s); return;
    case 2: launch_tile<E, BNMAJ, OT, 128, 128, 2, 2>(a, s); return;
    case 3: launch_tile<E, BNMAJ, OT, 128, 256, 2, 2>(a, s); return;
    case 4: launch_tile<E, BNMAJ, OT, 256, 256, 2, 4>(a, s); return;
    default: launch_tile<E, BNMAJ, OT, 256, 128, 2, 2>(a, s); return;
  }
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

bool gemm_mfma_ok(const GemmArgs& a) {
  if (const char* e = std::getenv("KURUMI_HIP_NO_MFMA"); e && *e && *e != '0') return false;
  const bool fp8 = a.in_type == GT_F8E4M3;
  if (!(a.in_type == GT_BF16 || a.in_type == GT_F16 || fp8)) return false;
  if (!(a.out_type == GT_BF16 || a.out_type == GT_F16 || a.out_type == GT_F32)) return false;
  const int64_t ke = fp8 ? 128 : 64, eb = fp8 ? 1 : 2, vec = 16 / eb;
  if (a.k % ke != 0 || a.k == 0) return false;
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

const char* gemm_mfma_name(const GemmArgs& a) {
  if (a.in_type == GT_F8E4M3) return "gemm_mfma_e4m3_nt";
  if (a.sbk == 1) return a.in_type == GT_F16 ? "gemm_mfma_f16_nt" : "gemm_mfma_bf16_nt";
  return a.in_type == GT_F16 ? "gemm_mfma_f16_nn" : "gemm_mfma_bf16_nn";
}

void launch_gemm_mfma(const GemmArgs& a, hipStream_t s) {
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
