// Flash attention forward on MFMA for gfx950 (kernel family 4).
//
// out[h] = softmax(scale * q[h] k[h]^T [+ causal -inf above the diagonal]) v[h] for each of the
// bh heads of contiguous [bh, s, d] bf16/f16 tensors: the semantics of `Op::Sdpa`
// (kurumi_core/src/interp/nn.rs:125-172) and of the decomposed chain
// (graph/ops/nn/attention.rs:97-113), computed the flash way (scores never leave registers).
//
// Everything is computed transposed so that one lane owns one query: a wave holds 32 queries,
//   S^T[key][q] = K[key][:] . Q[q][:]        (A = K tile from LDS, B = Q fragment in registers)
//   O^T[d][q]  += V^T[d][key] . P^T[key][q]  (A = V^T tile from LDS, B = P straight from S^T)
// With v_mfma_f32_32x32x16 the accumulator of a 32x32 tile gives lane l column l % 32 (the
// query) and rows 8*(v/4) + 4*(l/32) + v%4 (keys of S^T, head dims of O^T). So the running max,
// the running sum and the rescale of O are per-lane scalars (one cross-half exchange per block
// for the max), and the probabilities are already laid out as the B operand of the second
// product once the key slots of every 16-key step are permuted: slot 8*h + i of lane half h
// holds key 8*(i/4) + 4*h + i%4, i.e. key k sits at slot swap(bit2, bit3)(k). V^T is written to
// LDS in that slot order, so both operands read 16 contiguous bytes per lane.
//
// Work-group: NW waves, 32*NW queries, blocks of BK = 64 keys staged global -> registers -> LDS
// (K row-major, V transposed), double-buffered with one barrier per block. Causal q-tiles are
// issued heaviest first, and every head's tiles land on one XCD so its K/V stay in that L2.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdlib>
#include <stdexcept>

#include "kernels.h"
#include "numeric.h"

namespace ku::hipbk {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int BK = 64;  // keys per block
constexpr float LOG2E = 1.4426950408889634f;

template <int DT>
__device__ __forceinline__ f32x16 mfma(const u32x4& a, const u32x4& b, const f32x16& c) {
  if constexpr (DT == GT_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
}

// two f32 -> one dword of two 16-bit values (round to nearest even)
template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (DT == GT_BF16) return (uint32_t)d_bf16_st(lo) | ((uint32_t)d_bf16_st(hi) << 16);
  else return (uint32_t)d_f16_st(lo) | ((uint32_t)d_f16_st(hi) << 16);
}

template <int DT>
__device__ __forceinline__ uint16_t st16(float v) {
  if constexpr (DT == GT_BF16) return d_bf16_st(v);
  else return d_f16_st(v);
}

__device__ __forceinline__ int key_slot(int k) { return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1); }

template <int D, int DT, int NW>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2, 2))) attn_mfma_k(AttnArgs a) {
  constexpr int NT = NW * 64, BQ = 32 * NW;
  constexpr int KROW = D * 2 + 16;   // LDS bytes per K row (padded)
  constexpr int VROW = BK * 2 + 16;  // LDS bytes per V^T row (padded)
  constexpr int KBYTES = BK * KROW, VBYTES = D * VROW;
  constexpr int KC = BK * D / 8 / NT;  // 16-byte K chunks per thread
  constexpr int R = BK * D / 8 / NT;   // consecutive keys per thread in the V transpose
  constexpr int DS = D / 16;           // k-steps of S^T
  constexpr int DTL = D / 32;          // 32-row tiles of O^T
  static_assert(KC >= 1 && KC * NT * 8 == BK * D, "K staging");
  static_assert(R >= 1 && R <= 4 && (R & (R - 1)) == 0 && R * NT * 8 == BK * D, "V staging");
  __shared__ __attribute__((aligned(16))) unsigned char lds[2][KBYTES + VBYTES];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, h = lane >> 5, qc = lane & 31;
  const int64_t S = a.s;
  const int nqt = (int)((S + BQ - 1) / BQ);
  // heaviest causal tiles first; tile ids with equal head stay on one XCD (bh % 8 == 0 case)
  const int id = blockIdx.x;
  const int head = id % (int)a.bh;
  const int qt = a.causal ? nqt - 1 - id / (int)a.bh : id / (int)a.bh;
  const int64_t q0 = (int64_t)qt * BQ;
  const int64_t qw = q0 + wave * 32;  // first query of this wave
  const int64_t qi = qw + qc;         // this lane's query
  const int64_t base = (int64_t)head * S * D;
  const uint16_t* Q = static_cast<const uint16_t*>(a.q) + base;
  const uint16_t* K = static_cast<const uint16_t*>(a.k) + base;
  const uint16_t* V = static_cast<const uint16_t*>(a.v) + base;

  // Q fragments (B operand of S^T): lane holds q = qi, dims 16*s + 8*h .. +7
  u32x4 qf[DS];
#pragma unroll
  for (int s = 0; s < DS; ++s)
    qf[s] = qi < S ? *reinterpret_cast<const u32x4*>(Q + qi * D + s * 16 + h * 8) : u32x4{0, 0, 0, 0};

  const int64_t kend = a.causal ? (q0 + BQ < S ? q0 + BQ : S) : S;  // keys this tile needs
  const int nkb = (int)((kend + BK - 1) / BK);

  u32x4 rk[KC], rv[R];
  auto load = [&](int kb) {
    const int64_t k0 = (int64_t)kb * BK;
#pragma unroll
    for (int i = 0; i < KC; ++i) {
      const int c = tid + i * NT, row = c / (D / 8), col = c % (D / 8);
      rk[i] = (k0 + row < S) ? *reinterpret_cast<const u32x4*>(K + (k0 + row) * D + col * 8) : u32x4{0, 0, 0, 0};
    }
    const int dc = tid % (D / 8), kq = tid / (D / 8);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t kk = k0 + kq * R + r;
      rv[r] = kk < S ? *reinterpret_cast<const u32x4*>(V + kk * D + dc * 8) : u32x4{0, 0, 0, 0};
    }
  };
  auto store = [&](int buf) {
    unsigned char* L = lds[buf];
#pragma unroll
    for (int i = 0; i < KC; ++i) {
      const int c = tid + i * NT, row = c / (D / 8), col = c % (D / 8);
      *reinterpret_cast<u32x4*>(L + row * KROW + col * 16) = rk[i];
    }
    // R keys x 8 dims -> 8 V^T rows x R key slots (R keys starting at a multiple of R stay
    // contiguous under the slot permutation because R <= 4)
    unsigned char* LV = L + KBYTES;
    const int dc = tid % (D / 8), kq = tid / (D / 8);
    const int slot = (kq * R & ~15) | key_slot((kq * R) & 15);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int w = j >> 1, sh = (j & 1) * 16;
      unsigned char* dst = LV + (dc * 8 + j) * VROW + slot * 2;
      if constexpr (R == 4) {
        uint32_t o0 = ((rv[0][w] >> sh) & 0xffffu) | (((rv[1][w] >> sh) & 0xffffu) << 16);
        uint32_t o1 = ((rv[2][w] >> sh) & 0xffffu) | (((rv[3][w] >> sh) & 0xffffu) << 16);
        *reinterpret_cast<u32x2*>(dst) = u32x2{o0, o1};
      } else if constexpr (R == 2) {
        *reinterpret_cast<uint32_t*>(dst) = ((rv[0][w] >> sh) & 0xffffu) | (((rv[1][w] >> sh) & 0xffffu) << 16);
      } else {
        *reinterpret_cast<uint16_t*>(dst) = (uint16_t)((rv[0][w] >> sh) & 0xffffu);
      }
    }
  };

  f32x16 o[DTL];
#pragma unroll
  for (int t = 0; t < DTL; ++t)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[t][v] = 0.f;
  float m = -INFINITY, l = 0.f;
  const float c = a.scale * LOG2E;

  load(0);
  store(0);
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    const int cur = kb & 1;
    if (kb + 1 < nkb) load(kb + 1);
    const int64_t k0 = (int64_t)kb * BK;
    // wave-uniform: skip blocks entirely above this wave's diagonal
    const bool active = !a.causal || k0 <= qw + 31;
    if (active && qw < S) {
      const unsigned char* L = lds[cur];
      f32x16 sc[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int v = 0; v < 16; ++v) sc[t][v] = 0.f;
#pragma unroll
        for (int s = 0; s < DS; ++s) {
          const u32x4 kf = *reinterpret_cast<const u32x4*>(L + (t * 32 + qc) * KROW + s * 32 + h * 16);
          sc[t] = mfma<DT>(kf, qf[s], sc[t]);
        }
      }
      // mask: keys past the sequence, and (causal) keys after the query
      const bool need_mask = (k0 + BK > S) || (a.causal && k0 + BK - 1 > qw);
      if (need_mask) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int64_t kk = k0 + t * 32 + (v >> 2) * 8 + h * 4 + (v & 3);
            if (kk >= S || (a.causal && kk > qi)) sc[t][v] = -INFINITY;
          }
      }
      float bm = sc[0][0];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) bm = fmaxf(bm, sc[t][v]);
      bm = fmaxf(bm, __shfl_xor(bm, 32));
      const float mn = fmaxf(m, bm);
      const float mb = mn == -INFINITY ? 0.f : mn * c;
      const float corr = __builtin_amdgcn_exp2f(m * c - mb);
      m = mn;
      float rs = 0.f;
      u32x4 pf[4];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int v2 = 0; v2 < 8; ++v2) {
          const float p0 = __builtin_amdgcn_exp2f(fmaf(sc[t][2 * v2], c, -mb));
          const float p1 = __builtin_amdgcn_exp2f(fmaf(sc[t][2 * v2 + 1], c, -mb));
          rs += p0 + p1;
          // step s = 2t + v2/4 takes v = 8*(s%2) .. +7 of tile t
          pf[2 * t + (v2 >> 2)][v2 & 3] = pack2<DT>(p0, p1);
        }
      l = l * corr + rs;
#pragma unroll
      for (int t = 0; t < DTL; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[t][v] *= corr;
      const unsigned char* LV = L + KBYTES;
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int t = 0; t < DTL; ++t) {
          const u32x4 vf = *reinterpret_cast<const u32x4*>(LV + (t * 32 + qc) * VROW + s * 32 + h * 16);
          o[t] = mfma<DT>(vf, pf[s], o[t]);
        }
    }
    if (kb + 1 < nkb) store(cur ^ 1);
    __syncthreads();
  }

  if (qi >= S) return;
  l += __shfl_xor(l, 32);
  const float inv = 1.f / l;
  uint16_t* O = static_cast<uint16_t*>(a.o) + base + qi * D;
#pragma unroll
  for (int t = 0; t < DTL; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = t * 32 + g * 8 + h * 4;
      u32x2 w;
      w[0] = pack2<DT>(o[t][4 * g] * inv, o[t][4 * g + 1] * inv);
      w[1] = pack2<DT>(o[t][4 * g + 2] * inv, o[t][4 * g + 3] * inv);
      *reinterpret_cast<u32x2*>(O + d0) = w;
    }
}

template <int D, int DT>
void launch_d(const AttnArgs& a, hipStream_t s) {
  constexpr int NW = 4;
  const int64_t nqt = (a.s + 32 * NW - 1) / (32 * NW);
  dim3 grid((unsigned)(nqt * a.bh));
  hipLaunchKernelGGL((attn_mfma_k<D, DT, NW>), grid, dim3(NW * 64), 0, s, a);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

bool attention_mfma_ok(const AttnArgs& a) {
  if (const char* e = std::getenv("KURUMI_HIP_NO_MFMA"); e && *e && *e != '0') return false;
  if (!(a.dtype == GT_BF16 || a.dtype == GT_F16)) return false;
  if (!(a.d == 64 || a.d == 128)) return false;
  if (a.s <= 0 || a.bh <= 0 || a.bh * ((a.s + 127) / 128) > 0x7fffffff) return false;
  if (a.q && (!aligned16(a.q) || !aligned16(a.k) || !aligned16(a.v) || !aligned16(a.o))) return false;
  return true;
}

void launch_attention_mfma(const AttnArgs& a, hipStream_t s) {
  if (!attention_mfma_ok(a)) throw std::runtime_error("kurumi_hip attention: shape not supported by the MFMA kernel");
  if (a.dtype == GT_BF16) {
    if (a.d == 128) launch_d<128, GT_BF16>(a, s);
    else launch_d<64, GT_BF16>(a, s);
  } else {
    if (a.d == 128) launch_d<128, GT_F16>(a, s);
    else launch_d<64, GT_F16>(a, s);
  }
}

}  // namespace ku::hipbk
