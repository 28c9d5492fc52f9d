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
// Work-group: NW waves of 32 queries each (a q-tile of 32*NW queries), blocks of BK = 64 keys
// staged global -> LDS by DMA, double-buffered with one barrier per block. The grid is persistent
// (two work-groups per CU), each work-group walking a fixed sequence of q-tiles with the pipeline
// running across tile boundaries; causal q-tiles are taken heaviest first, and every head's tiles
// land on one XCD so its K/V stay in that L2.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <stdexcept>
#include <type_traits>

#include "kernels.h"
#include "lds_dma.h"
#include "numeric.h"

namespace ku::hipbk {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((__vector_size__(4 * sizeof(short))));
#define KU_LDS __attribute__((address_space(3)))

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

// two f32 -> one dword of two 16-bit values, rounded to nearest even by v_cvt_pk_bf16_f32 /
// v_cvt_f16_f32 (the probabilities and outputs here are never NaN unless an input is)
template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  const f32x2 v = {lo, hi};
  if constexpr (DT == GT_BF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  else return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}

// c + lo + hi of a packed pair of 16-bit floats (v_dot2c_f32_{bf16,f16} against 1.0 pairs)
template <int DT>
__device__ __forceinline__ float sum2(uint32_t pair, float c) {
  if constexpr (DT == GT_BF16) {
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pair), one, c, false);
  } else {
    const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pair), one, c, false);
  }
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, uint32_t bytes) {
  // dword3 0x00020000: 32-bit data format, the raw-buffer setting for gfx9 parts
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 bload(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}


// Lazy rescaling: the running max m (kept pre-multiplied by scale*log2 e) only moves when a
// block's max exceeds it by more than RESCALE (log2 units), so most blocks skip the O rescale.
// Probabilities then reach at most 2^RESCALE before normalisation, far inside f32 and bf16 range;
// the result is the same softmax (numerator and denominator share the stale max).
constexpr float RESCALE = 8.f;


// One q-tile of one head, as the persistent loop below walks them. A tile past the last one has
// no key blocks and its queries start at the sequence end, so every load of it reads zeros.
// 32-bit fields: the scalar registers are the kernel's scarce resource (S < 2^24 here).
struct Tile {
  int head;  // q / k / v / o head
  int q0;    // first query
  int nkv;   // key blocks holding keys the tile needs
  int nkb;   // blocks the loop runs: nkv rounded up to even (the extra block is fully masked)
};

// Persistent work-groups (about two per CU): work-group b runs its tiles one after another (see
// tile_at), and the software pipeline runs straight across tile boundaries, so a tile's prologue
// (Q fragments, the first K / V blocks, the first S^T) and epilogue overlap the neighbouring
// tile's blocks instead of leaving the CU to the other work-group.
//
// Software pipeline per block kb (one barrier each): the S^T MFMAs of block kb+1 are independent
// of the softmax instructions of block kb, so the two interleave; then the P.V MFMAs of block kb
// run while K of block kb+2 and V of block kb+1 land in LDS. K and V have separate double
// buffers, K one block ahead of V. Past a tile's last block those are the next tile's blocks 0
// and 1: its Q fragments are loaded once the current tile's last S^T has been issued, and the
// last block's "next S^T" is the next tile's first, so every tile but a work-group's first
// starts with its K0, K1, V0 and first scores in place.
template <int D, int DT, int NW>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
attn_mfma_k(AttnArgs a) {
  constexpr int QT = 1;                  // 32-query tiles per wave
  constexpr int QW = 32 * QT, BQ = QW * NW;
  constexpr int RB = D * 2;              // bytes per K / V row in LDS (no padding: swizzled)
  constexpr int W = 256 / RB;            // rows per 256-byte bank window (64 banks)
  constexpr int CPR = RB / 16;           // 16-byte chunks per row
  constexpr int TBYTES = BK * RB;        // one K or V block
  constexpr int NBLK = TBYTES / 1024 / NW;  // 1 KB DMA blocks per wave per tile
  constexpr int DS = D / 16;             // k-steps of S^T
  constexpr int DTL = D / 32;            // 32-row tiles of O^T
  static_assert(W >= 1 && NBLK * NW * 1024 == TBYTES, "K / V staging");
  // every block a wave needs starts at or before the wave's first query, so a lane is never
  // fully masked in a block it needs
  static_assert(BK % 32 == 0 && (QW % BK == 0 || BK % QW == 0), "block / wave alignment");
  // K buffers 0, 1 then V buffers 0, 1; the last one doubles as the epilogue's staging area
  // (4 KB per wave), so it is at least that large
  constexpr int STAGE = NW * 4096;
  __shared__ __attribute__((aligned(1024))) unsigned char lds_raw[3 * TBYTES + (TBYTES > STAGE ? TBYTES : STAGE)];
  KU_LDS unsigned char* lds = (KU_LDS unsigned char*)lds_raw;

  // the wave index is uniform: kept in an SGPR, so the DMA destinations (M0) need no VALU work
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), h = lane >> 5,
            qc = lane & 31;
  const int S = (int)a.s;
  const int64_t HS = (int64_t)S * D;  // elements per head
  const int bh = (int)a.bh;
  const int nqt = (S + BQ - 1) / BQ;
  const int64_t ntiles = (int64_t)nqt * bh;
  const int64_t G = gridDim.x;
  const uint32_t hb = (uint32_t)(S * D * 2);  // bytes per head
  // Otherwise tile t is head t % bh, q-tile t / bh (causal: heaviest first). Work-group b takes
  // tile r*G + b in round r, and in odd rounds the tile at the mirrored position among the
  // work-groups of its XCD (b % 8 kept): the causal tiles' sizes even out over a work-group's
  // rounds, and with bh % 8 == 0 every tile of a head runs on one XCD.
  // Head-grouped order (when the shapes allow it): round r runs every q-tile of G / nqt heads,
  // each XCD (b % 8) G / nqt / 8 of them, so the q-tiles of a head start their walks over its
  // K / V blocks together and read them from one L2 (cfg 4: fetched bytes -28 %); in odd rounds
  // a work-group takes the mirrored q-tile, which evens out the causal tiles' sizes over two
  // rounds.
  const bool grouped = (G % (8 * (int64_t)nqt)) == 0 && bh % (G / nqt) == 0;
  auto tile_at = [&](int r) {
    const int64_t b = blockIdx.x;
    Tile T{0, S, 0, 0};
    int head = 0, qt = 0;
    bool valid;
    if (grouped) {
      const int64_t hpr = G / nqt, hpx = hpr / 8, x = b & 7, j = b >> 3, qs = j % nqt;
      valid = (int64_t)r * hpr < bh;
      head = (int)(r * hpr + x * hpx + j / nqt);
      qt = (int)((r & 1) ? nqt - 1 - qs : qs);
    } else {
      const bool mirror = (r & 1) && (G & 7) == 0;
      const int64_t t = (int64_t)r * G + (mirror ? (b & 7) + 8 * (G / 8 - 1 - (b >> 3)) : b);
      valid = t < ntiles;
      if (valid) {
        const int ti = (int)t;
        qt = a.causal ? nqt - 1 - ti / bh : ti / bh;
        head = ti % bh;
      }
    }
    if (valid) {
      T.head = head;
      T.q0 = qt * BQ;
      const int kend = a.causal ? (T.q0 + BQ < S ? T.q0 + BQ : S) : S;  // keys the tile needs
      T.nkv = (kend + BK - 1) / BK;
      T.nkb = (T.nkv + 1) & ~1;
    }
    return T;
  };

  // raw buffer loads: rows past the sequence read as zero, no branches
  // Q fragments (B operand of S^T): lane holds query qw + 32u + qc, dims 16*s + 8*h .. +7
  u32x4 qf[QT][DS];
  auto load_q = [&](const Tile& T) {
    const auto Q = rsrc(static_cast<const uint16_t*>(a.q) + T.head * HS, hb);
    const int qw = T.q0 + wave * QW;
#pragma unroll
    for (int u = 0; u < QT; ++u) {
      const int qi = qw + 32 * u + qc;
      const uint32_t off = qi < S ? (uint32_t)(qi * D * 2) + h * 16 : hb;
#pragma unroll
      for (int s = 0; s < DS; ++s) qf[u][s] = bload(Q, off + s * 32);
    }
  };

  // K and V blocks go global -> LDS by DMA (buffer_load ... lds: lane l of a wave writes bytes
  // 16l..16l+15 of the wave's 1 KB destination; offsets past the head read as zeros). The LDS
  // position of each chunk is fixed by the lane, so the swizzles are applied by choosing which
  // global chunk each lane fetches:
  //   K: chunk c of row r at c ^ ((r / W) % (16 / W)) -- the 16 rows one fragment read touches at
  //      one chunk land on 16 distinct bank groups;
  //   V: chunk c of row r at c ^ 4((r / W) % (4 / W)) -- the 4 rows x 4 chunks one transposing
  //      read touches do.
  auto kswz = [](int r) { return (r / W) % (16 / W); };
  auto vswz = [](int r) { return 4 * ((r / W) % (4 / W)); };
  // The block offset moves the descriptor's base (scalar work; the byte count shrinks with it, so
  // blocks past the tile's keys read zeros) and the per-lane offsets stay loop-invariant.
  const uint16_t* kp = static_cast<const uint16_t*>(a.k);
  const uint16_t* vp = static_cast<const uint16_t*>(a.v);
  auto dma = [&](const uint16_t* src, int head, int nkv, int kb, KU_LDS unsigned char* dst, bool isv) {
    const uint32_t k0b = kb < nkv ? (uint32_t)kb * BK * RB : hb;
    const auto R = rsrc(reinterpret_cast<const unsigned char*>(src + head * HS) + k0b, hb - k0b);
    // the wave's first destination, recomputed at every call (opaque to the optimiser): hoisted,
    // the M0 values of all DMAs would stay live in SGPRs across the loop and spill
    KU_LDS unsigned char* wd = dst + wave * 1024;
    asm volatile("" : "+s"(wd));
#pragma unroll
    for (int i = 0; i < NBLK; ++i) {
      const int blk = i * NW + wave, r = blk * (1024 / RB) + lane / CPR, pc = lane % CPR;
      const int cc = pc ^ (isv ? vswz(r) : kswz(r));
      lds_dma16(R, r * RB + cc * 16, 0, (KU_LDS void*)(wd + i * NW * 1024));
    }
  };
  auto kbuf = [&](int i) { return lds + i * TBYTES; };
  auto vbuf = [&](int i) { return lds + (2 + i) * TBYTES; };
  // S^T of one block from a K buffer: 2 key tiles x QT query tiles, DS k-steps
  auto s_mfma = [&](const KU_LDS unsigned char* L, f32x16 (&sc)[QT][2]) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int u = 0; u < QT; ++u)
#pragma unroll
        for (int v = 0; v < 16; ++v) sc[u][t][v] = 0.f;
#pragma unroll
    for (int s = 0; s < DS; ++s)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int r = t * 32 + qc;
        const u32x4 kf = *(const KU_LDS u32x4*)(L + r * RB + (((2 * s + h) ^ kswz(r)) << 4));
#pragma unroll
        for (int u = 0; u < QT; ++u) sc[u][t] = mfma<DT>(kf, qf[u][s], sc[u][t]);
      }
  };

  f32x16 o[QT][DTL];
  float mc[QT], l[QT];
  const float c = a.scale * LOG2E;
  int round = 0;
  Tile C = tile_at(0), N = tile_at(1);  // this work-group's current and next tile
  int qw = C.q0 + wave * QW;            // first query of this wave in the current tile

  // One block: softmax of sc (this block's S^T) and S^T of the next block into sn. The loop runs
  // two blocks per trip with the two score sets swapping roles, so no registers are copied.
  // The parity of kb is a compile-time constant, so every LDS address is a loop-invariant
  // per-lane value plus an immediate. Waves whose queries lie past the sequence run the same
  // instructions on zero queries (their results are never stored), so every wave computes the
  // next tile's first scores.
  auto block = [&](int kb, f32x16 (&sc)[QT][2], f32x16 (&sn)[QT][2], auto par) __attribute__((always_inline)) {
    constexpr int P = decltype(par)::value;
    // K of block kb+2 and V of block kb+1 into the buffers the previous block freed: this tile's
    // while it has them, then the next tile's first ones
    const bool kc = kb + 2 < C.nkb, vc = kb + 1 < C.nkb;
    dma(kp, kc ? C.head : N.head, kc ? C.nkv : N.nkv, kc ? kb + 2 : kb + 2 - C.nkb, kbuf(P), false);
    dma(vp, vc ? C.head : N.head, vc ? C.nkv : N.nkv, vc ? kb + 1 : kb + 1 - C.nkb, vbuf(P ^ 1), true);
    const int k0 = kb * BK;
    u32x4 pf[QT][4];
#pragma unroll
    for (int u = 0; u < QT; ++u) {
      // mask keys past the sequence and (causal) keys after the query: key k0 + off(t, v) + 4h
      // is dropped when off(t, v) > lim, off(t, v) = 32t + 8(v/4) + v%4 a constant per register
      if ((k0 + BK > S) || (a.causal && k0 + BK - 1 > qw + 32 * u)) {
        const int qi = qw + 32 * u + qc;
        const int last = a.causal && qi < S - 1 ? qi : S - 1;  // last visible key
        const int lim = last - k0 - 4 * h;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            if (t * 32 + (v >> 2) * 8 + (v & 3) > lim) sc[u][t][v] = -INFINITY;
      }
      float bm = sc[u][0][0];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) bm = fmaxf(bm, sc[u][t][v]);
      // the two halves of the wave hold the same queries: exchange without LDS
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(bm), __float_as_uint(bm), false, false);
      bm = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * c;
      // Each query decides for itself (both halves of the wave see the same bm and mc, so they
      // agree): a query that keeps its max multiplies by exactly 1. A query's result thus depends
      // on its own scores alone, never on a neighbour's rescale; the branch is skipped when no
      // query of the wave needs it.
      const bool need = bm > mc[u] + RESCALE;
      if (__builtin_amdgcn_ballot_w64(need) != 0) {
        const float mn = need ? fmaxf(mc[u], bm) : mc[u];
        const float corr = need ? __builtin_amdgcn_exp2f(mc[u] - mn) : 1.f;
        mc[u] = mn;
        l[u] *= corr;
#pragma unroll
        for (int t = 0; t < DTL; ++t)
#pragma unroll
          for (int v = 0; v < 16; ++v) o[u][t][v] *= corr;
      }
    }
    // S^T of the next block (its K is already in LDS) interleaved with the exponentials of block
    // kb. Wave priority: the section that interleaves the next S^T MFMAs with this block's softmax
    // goes first when both waves of a SIMD are ready (measured 3 % faster than equal priority)
    __builtin_amdgcn_s_setprio(1);
    {
      // The 2*DS S^T MFMAs of the next block (MFMA m: k-step m/2, key tile m%2) interleaved with
      // the 16 exponential pairs of this block (16 / (2*DS) pairs before each MFMA), each K
      // fragment read two MFMAs ahead; a scheduling barrier after each group keeps the compiler
      // from regrouping them (left to itself it ran the MFMAs back to back, each waiting for its
      // own LDS read, and the softmax after them).
      constexpr int NM = 2 * DS, PPM = 16 / NM;
      static_assert(NM * PPM == 16, "exponential pairs per MFMA");
      const KU_LDS unsigned char* LK = kbuf(P ^ 1);
      auto kread = [&](int m) {
        const int r = (m & 1) * 32 + qc;
        return *(const KU_LDS u32x4*)(LK + r * RB + (((2 * (m >> 1) + h) ^ kswz(r)) << 4));
      };
      // the row sum adds the rounded probabilities (the ones the P.V product uses), two at a
      // time with v_dot2 against (1, 1), in two chains
      float rs[2] = {0.f, 0.f};
      u32x4 kf[3];
      kf[0] = kread(0);
      kf[1] = kread(1);
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        if (m + 2 < NM) kf[(m + 2) % 3] = kread(m + 2);
#pragma unroll
        for (int e = 0; e < PPM; ++e) {
          const int i = m * PPM + e, te = i >> 3, v2 = i & 7;
          const float p0 = __builtin_amdgcn_exp2f(fmaf(sc[0][te][2 * v2], c, -mc[0]));
          const float p1 = __builtin_amdgcn_exp2f(fmaf(sc[0][te][2 * v2 + 1], c, -mc[0]));
          const uint32_t pp = pack2<DT>(p0, p1);
          rs[v2 & 1] = sum2<DT>(pp, rs[v2 & 1]);
          // step s = 2t + v2/4 takes v = 8*(s%2) .. +7 of tile t
          pf[0][2 * te + (v2 >> 2)][v2 & 3] = pp;
        }
        // the first k-step of each key tile starts from zero
        sn[0][m & 1] = mfma<DT>(kf[m % 3], qf[0][m >> 1], m < 2 ? f32x16{} : sn[0][m & 1]);
        __builtin_amdgcn_sched_barrier(0);
      }
      l[0] += rs[0] + rs[1];
    }
    // O^T += V^T . P^T for block kb. V^T fragments come straight from the row-major V block
    // with ds_read_b64_tr_b16: in each 16-lane group, input lane 4k'+q points at key row k',
    // dims 4q..4q+3, and output lane i receives keys 0..3 of dim i. Two reads fetch exactly the
    // key groups the probability registers hold: 16s + 4h + 0..3 and 16s + 8 + 4h + 0..3.
    __builtin_amdgcn_s_setprio(0);
    const KU_LDS unsigned char* LV = vbuf(P);
    const int g = lane >> 4, c16 = lane & 15;
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int t = 0; t < DTL; ++t) {
        const int d = t * 32 + (g & 1) * 16 + (c16 & 3) * 4;
        u32x2 half[2];
#pragma unroll
        for (int r2 = 0; r2 < 2; ++r2) {
          const int kr = 16 * s + 8 * r2 + 4 * h + (c16 >> 2);
          const KU_LDS unsigned char* p = LV + kr * RB + (((d >> 3) ^ vswz(kr)) << 4) + (d & 7) * 2;
          half[r2] = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((KU_LDS s16x4*)p));
        }
        const u32x4 vf = u32x4{half[0][0], half[0][1], half[1][0], half[1][1]};
#pragma unroll
        for (int u = 0; u < QT; ++u) o[u][t] = mfma<DT>(vf, pf[u][s], o[u][t]);
      }
    // the S^T just issued was this tile's last: the Q fragments now belong to the next tile
    if (kb + 2 == C.nkb) load_q(N);
    // this thread's loads for the next blocks have landed; the barrier publishes them
    vm_wait<0>();
    __syncthreads();
  };

  // the first tile's prologue: Q, K0, V0, K1 and the first scores
  f32x16 sa[QT][2], sb[QT][2];
  load_q(C);
  dma(kp, C.head, C.nkv, 0, kbuf(0), false);
  dma(vp, C.head, C.nkv, 0, vbuf(0), true);
  dma(kp, C.head, C.nkv, 1, kbuf(1), false);
  vm_wait<0>();
  __syncthreads();
  s_mfma(kbuf(0), sa);
  __syncthreads();  // block 0 refills K buffer 0: every wave has read it
  for (;;) {
#pragma unroll
    for (int u = 0; u < QT; ++u) {
      mc[u] = -INFINITY;
      l[u] = 0.f;
#pragma unroll
      for (int t = 0; t < DTL; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[u][t][v] = 0.f;
    }
    for (int kb = 0; kb < C.nkb; kb += 2) {
      block(kb, sa, sb, std::integral_constant<int, 0>{});
      block(kb + 1, sb, sa, std::integral_constant<int, 1>{});
    }
    // Epilogue: normalise, then stage through V buffer 1 (free between a tile's last block and
    // the next tile's first DMA; each wave owns 4 KB = 32 queries x 64 dims, 16-byte chunks
    // swizzled by row) so every store writes whole 128-byte lines: eight rows of 16 lanes x 16
    // bytes per instruction instead of 8-byte pieces of 32 rows, whose drain through the memory
    // pipeline stalled the next tile's first instructions.
    static_assert(QT == 1 && DTL % 2 == 0, "epilogue staging");
    {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l[0]), __float_as_uint(l[0]), false, false);
      const float inv = 1.f / (__uint_as_float(sw[0]) + __uint_as_float(sw[1]));
      KU_LDS unsigned char* R = vbuf(1) + wave * 4096;
      uint16_t* Oh = static_cast<uint16_t*>(a.o) + C.head * HS;
#pragma unroll
      for (int hf = 0; hf < DTL / 2; ++hf) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            // lane (qc, h) holds dims 32t + 8g + 4h .. +3 of query qc: chunk 4tt + g, bytes 8h..
            const f32x16& ot = o[0][2 * hf + tt];
            u32x2 w;
            w[0] = pack2<DT>(ot[4 * g] * inv, ot[4 * g + 1] * inv);
            w[1] = pack2<DT>(ot[4 * g + 2] * inv, ot[4 * g + 3] * inv);
            *(KU_LDS u32x2*)(R + qc * 128 + (((4 * tt + g) ^ (qc & 7)) << 4) + 8 * h) = w;
          }
        // one wave writes and reads its own region: its LDS operations complete in order
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int qr = (lane >> 3) + 8 * i, cc = lane & 7;
          const u32x4 val = *(const KU_LDS u32x4*)(R + qr * 128 + ((cc ^ (qr & 7)) << 4));
          if (qw + qr < S) *reinterpret_cast<u32x4*>(Oh + (int64_t)(qw + qr) * D + hf * 64 + cc * 8) = val;
        }
      }
      // every wave's staging reads are done before the next tile's first DMA refills V buffer 1
      // (a bare barrier: the stores need not have completed)
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    if (N.nkb == 0) break;
    C = N;
    N = tile_at(++round + 1);
    qw = C.q0 + wave * QW;
  }
}

template <int D, int DT>
void launch_d(const AttnArgs& a, hipStream_t s) {
  constexpr int NW = 4, BQ = 32 * NW;
  const int64_t ntiles = (a.s + BQ - 1) / BQ * a.bh;
  // two resident work-groups per CU; KURUMI_HIP_ATTN_GRID caps the grid (tests use it to give
  // every work-group several tiles at small shapes)
  int64_t g = std::min<int64_t>(ntiles, 2 * (int64_t)cu_count());
  if (const char* e = std::getenv("KURUMI_HIP_ATTN_GRID"); e && *e && std::atoll(e) > 0)
    g = std::min<int64_t>(g, std::atoll(e));
  if (g < ntiles) g = std::max<int64_t>(8, g & ~int64_t(7));  // mirrored rounds need whole XCD groups
  hipLaunchKernelGGL((attn_mfma_k<D, DT, NW>), dim3((unsigned)g), dim3(NW * 64), 0, s, a);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

bool attention_mfma_ok(const AttnArgs& a) {
  if (const char* e = std::getenv("KURUMI_HIP_NO_MFMA"); e && *e && *e != '0') return false;
  if (!(a.dtype == GT_BF16 || a.dtype == GT_F16)) return false;
  if (!(a.d == 64 || a.d == 128)) return false;
  if (a.s <= 0 || a.bh <= 0 || a.bh * ((a.s + 127) / 128) > 0x7fffffff) return false;
  if (a.s * a.d * 2 >= (int64_t(1) << 31)) return false;  // per-head buffer offsets are 32-bit
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
