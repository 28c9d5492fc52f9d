// The e4m3 linear on device buffers (the graph the e4m3 mixed-precision pass emits, as kernels):
//
//   amax = max_i |x_i|   (maxNum fold from -inf, so NaNs never win: f32::max of the reference
//                          interpreter, kurumi_core/src/dtype/traits/float.rs:36)
//   sx   = amax * f32(1/448),  inv = 1 / sx  (IEEE division, as Op::Recip; inv = 1 unless
//                                              sx > 0, so an all-zero x gives xq = 0 and y = 0)
//   xq   = e4m3(f32(x) * inv)                 (round to nearest even, saturating to +-448)
//   y    = round_out((xq @ wq^T) * sx * sw[n]) (the fp8 MFMA GEMM, scales in its epilogue)
//
// The activation quantisation runs in two passes with no atomics and nothing to clear: pass 1
// writes one absmax partial per work-group; pass 2 has every work-group fold all partials
// (a few KB from L2), derive sx and inv itself and quantise its part of x. Work-group 0 also
// stores sx for the GEMM epilogue. Scratch per call: the partials, sx and xq (M*K bytes).
//
// linear_e4m3 runs the whole layer with scratch the caller (a backend's workspace) provides; the
// planner runs the same activation kernels as one step before its fp8 GEMM step.
// linear_e4m3_noalloc runs it with scratch in a file-scope device array instead, for callers that
// cannot allocate (code under hipGraph capture, serving loops): no hipMalloc, hipFree or other
// allocating call. Every GPU holds its own copy of the array until the process ends; all calls on
// one GPU share it (each call's partials and sx are written before they are read, so nothing
// needs clearing), so calls that overlap on one GPU race.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>
#include <stdexcept>
#include <string>

#include "kernels.h"
#include "numeric.h"

namespace ku::hipbk {

namespace {

constexpr int kThreads = 256;
constexpr float kInv448 = 1.0f / 448.0f;  // correctly rounded, the pass's scalar constant

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// work-group maxNum of v (every thread gets the result)
__device__ __forceinline__ float block_max(float v, float* lds) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  if (l == 0) lds[w] = v;
  __syncthreads();
  float r = lds[0];
#pragma unroll
  for (int i = 1; i < kThreads / 64; ++i) r = fmaxf(r, lds[i]);
  __syncthreads();
  return r;
}

template <int XT>
struct XIn;
template <>
struct XIn<GT_BF16> {
  static constexpr int V = 8;
  __device__ static void load(const void* x, int64_t i, float* v) {
    const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + i);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = __uint_as_float(w[j] << 16);
      v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
  }
  __device__ static float load1(const void* x, int64_t i) { return d_bf16_ld(static_cast<const uint16_t*>(x)[i]); }
};
template <>
struct XIn<GT_F16> {
  static constexpr int V = 8;
  __device__ static void load(const void* x, int64_t i, float* v) {
    const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + i);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = d_f16_ld((uint16_t)(w[j] & 0xffffu));
      v[2 * j + 1] = d_f16_ld((uint16_t)(w[j] >> 16));
    }
  }
  __device__ static float load1(const void* x, int64_t i) { return d_f16_ld(static_cast<const uint16_t*>(x)[i]); }
};
template <>
struct XIn<GT_F32> {
  static constexpr int V = 4;
  __device__ static void load(const void* x, int64_t i, float* v) {
    const float4 q = *reinterpret_cast<const float4*>(static_cast<const float*>(x) + i);
    v[0] = q.x;
    v[1] = q.y;
    v[2] = q.z;
    v[3] = q.w;
  }
  __device__ static float load1(const void* x, int64_t i) { return static_cast<const float*>(x)[i]; }
};

// Each thread takes VPT vectors per trip, the loads of a trip all issued before any use (one
// memory latency per trip instead of one per vector); consecutive threads read consecutive
// vectors, so every load instruction of a wave is coalesced.
constexpr int kVptAbsmax = 4, kVptQuant = 2;

// pass 1: partials[g] = maxNum over the elements work-group g visits (-inf when none)
template <int XT>
__global__ __launch_bounds__(kThreads) void actq_absmax_k(const void* __restrict__ x, int64_t n,
                                                          float* __restrict__ partials) {
  __shared__ float lds[kThreads / 64];
  using In = XIn<XT>;
  constexpr int V = In::V, U = kVptAbsmax;
  float m = -__builtin_inff();
  const int64_t nv = n / V, trip = (int64_t)gridDim.x * kThreads * U;
  for (int64_t base = (int64_t)blockIdx.x * kThreads * U + threadIdx.x; base < nv; base += trip) {
    float v[U][V];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (base + u * kThreads < nv) In::load(x, (base + u * kThreads) * V, v[u]);
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (base + u * kThreads < nv)
#pragma unroll
        for (int j = 0; j < V; ++j) m = fmaxf(m, fabsf(v[u][j]));
  }
  for (int64_t i = nv * V + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
    m = fmaxf(m, fabsf(In::load1(x, i)));
  m = block_max(m, lds);
  if (threadIdx.x == 0) partials[blockIdx.x] = m;
}

template <int V>
__device__ __forceinline__ void store_e4m3(uint8_t* p, const float* v, float inv) {
  uint32_t q[V / 4];
#pragma unroll
  for (int j = 0; j < V / 4; ++j) {
    uint32_t w = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) w |= (uint32_t)d_e4m3_st(v[4 * j + e] * inv) << (8 * e);
    q[j] = w;
  }
  if constexpr (V == 8)
    *reinterpret_cast<uint2*>(p) = make_uint2(q[0], q[1]);
  else
    *reinterpret_cast<uint32_t*>(p) = q[0];
}

// pass 2: fold the partials, then xq = e4m3(x * (1 / (amax * (1/448)))) (1 / 1 when amax is 0);
// work-group 0 stores sx.
// The first trip's loads of x are issued before the partials are folded.
template <int XT>
__global__ __launch_bounds__(kThreads) void actq_quantise_k(const void* __restrict__ x, int64_t n,
                                                            const float* __restrict__ partials, int nparts,
                                                            uint8_t* __restrict__ xq, float* __restrict__ sx_out) {
  __shared__ float lds[kThreads / 64];
  using In = XIn<XT>;
  constexpr int V = In::V, U = kVptQuant;
  const int64_t nv = n / V, trip = (int64_t)gridDim.x * kThreads * U;
  int64_t base = (int64_t)blockIdx.x * kThreads * U + threadIdx.x;
  float v[U][V];
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (base + u * kThreads < nv) In::load(x, (base + u * kThreads) * V, v[u]);
  float m = -__builtin_inff();
  for (int i = threadIdx.x; i < nparts; i += kThreads) m = fmaxf(m, partials[i]);
  const float amax = block_max(m, lds);
  const float sx = amax * kInv448;
  const float inv = 1.0f / (sx > 0.f ? sx : 1.f);  // where(0 < sx, sx, 1) of the e4m3 pass
  if (blockIdx.x == 0 && threadIdx.x == 0) sx_out[0] = sx;
  while (base < nv) {
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (base + u * kThreads < nv) store_e4m3<V>(xq + (base + u * kThreads) * V, v[u], inv);
    base += trip;
    if (base >= nv) break;
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (base + u * kThreads < nv) In::load(x, (base + u * kThreads) * V, v[u]);
  }
  for (int64_t i = nv * V + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
    xq[i] = d_e4m3_st(In::load1(x, i) * inv);
}

int partial_count(int64_t n) {
  // about 16 KB of bf16 input per work-group for the absmax pass, at most kActqMaxPartials groups
  const int64_t g = (n + 8191) / 8192;
  return (int)std::max<int64_t>(1, std::min<int64_t>(g, kActqMaxPartials));
}

template <int XT>
void launch_actq_t(const ActQArgs& a, hipStream_t s) {
  const int np = partial_count(a.n);
  hipLaunchKernelGGL((actq_absmax_k<XT>), dim3(np), dim3(kThreads), 0, s, a.x, a.n, a.partials);
  constexpr int V = XIn<XT>::V;
  const int64_t per_group = (int64_t)kThreads * V * kVptQuant;
  const int64_t g = std::max<int64_t>(1, std::min<int64_t>((a.n + per_group - 1) / per_group, 1 << 20));
  hipLaunchKernelGGL((actq_quantise_k<XT>), dim3((unsigned)g), dim3(kThreads), 0, s, a.x, a.n, a.partials, np, a.xq,
                     a.sx);
}

}  // namespace

size_t actq_partials_bytes(int64_t n) { return (size_t)partial_count(n) * sizeof(float); }

void launch_actq(const ActQArgs& a, hipStream_t s) {
  if (a.n <= 0) throw std::runtime_error("kurumi_hip: e4m3 activation quantisation of an empty tensor");
  if ((reinterpret_cast<uintptr_t>(a.x) % 16) != 0)
    throw std::runtime_error("kurumi_hip: e4m3 activation input must be 16-byte aligned");
  switch (a.x_type) {
    case GT_BF16: launch_actq_t<GT_BF16>(a, s); break;
    case GT_F16: launch_actq_t<GT_F16>(a, s); break;
    case GT_F32: launch_actq_t<GT_F32>(a, s); break;
    default: throw std::runtime_error("kurumi_hip: e4m3 activation dtype must be bf16, f16 or f32");
  }
}

// ---------------- the e4m3 linear on device buffers ----------------

namespace {

void check_linear(const LinearE4m3Args& a) {
  if (!a.x || !a.wq || !a.sw || !a.y) throw std::runtime_error("null device pointer");
  if (a.m <= 0 || a.n <= 0 || a.k <= 0) throw std::runtime_error("m, n and k must be positive");
  if (a.k % 128 != 0) throw std::runtime_error("k must be a multiple of 128 (the e4m3 MFMA GEMM's K stage)");
  if (!(a.x_type == GT_BF16 || a.x_type == GT_F16 || a.x_type == GT_F32))
    throw std::runtime_error("x dtype must be KU_BF16, KU_F16 or KU_F32");
  if (!(a.y_type == GT_BF16 || a.y_type == GT_F16 || a.y_type == GT_F32))
    throw std::runtime_error("y dtype must be KU_BF16, KU_F16 or KU_F32");
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (!al(a.x) || !al(a.wq) || !al(a.y)) throw std::runtime_error("x, wq and y must be 16-byte aligned");
}

void run_linear(const LinearE4m3Args& a, uint8_t* xq, float* partials, float* sx, hipStream_t s) {
  ActQArgs q;
  q.x = a.x;
  q.x_type = a.x_type;
  q.n = a.m * a.k;
  q.xq = xq;
  q.partials = partials;
  q.sx = sx;
  launch_actq(q, s);
  GemmArgs g;
  g.a = xq;
  g.b = a.wq;
  g.c = a.y;
  g.sam = a.k; g.sak = 1; g.sab = 0;
  g.sbn = a.k; g.sbk = 1; g.sbb = 0;  // B[k][n] = wq[n][k]: the NT layout
  g.batch = 1; g.m = a.m; g.n = a.n; g.k = a.k;
  g.in_type = GT_F8E4M3;
  g.out_type = a.y_type;
  g.alpha = sx;
  g.col_scale = a.sw;
  g.col_scale_stride = 1;
  launch_gemm(g, s);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) throw std::runtime_error(std::string("launch failed: ") + hipGetErrorString(e));
}

// Scratch layout (both entry points): [0, 4 KiB) absmax partials, [4 KiB, 4 KiB + 256) sx,
// then xq (M*K bytes), every part 256-byte aligned.
constexpr size_t kPartialsOff = 0, kSxOff = 4096, kXqOff = 4096 + 256;
static_assert(kActqMaxPartials * sizeof(float) <= kSxOff, "partials overflow their scratch part");

// The no-allocation entry point's scratch. In host code `scratch` names a host-side stand-in,
// never the device memory: its device address on each GPU comes from hipGetSymbolAddress.
__device__ __align__(256) uint8_t scratch[kLinearE4m3ScratchBytes];

std::mutex g_scratch_mu;
constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};  // device address of `scratch` on each GPU, set once per GPU

// The current GPU's copy of `scratch` (looked up, with that GPU current, on its first use).
uint8_t* scratch_on_current_device() {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) throw std::runtime_error(std::string("hipGetDevice: ") + hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) throw std::runtime_error("device index out of range");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      throw std::runtime_error(std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  return static_cast<uint8_t*>(g_scratch_ptr[dev]);
}

}  // namespace

size_t linear_e4m3_scratch_bytes(int64_t m, int64_t k) { return kXqOff + (size_t)(m * k); }

void linear_e4m3(const LinearE4m3Args& a, void* scratch_buf, size_t scratch_bytes, hipStream_t s) {
  check_linear(a);
  if (!scratch_buf || scratch_bytes < linear_e4m3_scratch_bytes(a.m, a.k))
    throw std::runtime_error("scratch buffer too small");
  uint8_t* base = static_cast<uint8_t*>(scratch_buf);
  run_linear(a, base + kXqOff, reinterpret_cast<float*>(base + kPartialsOff), reinterpret_cast<float*>(base + kSxOff),
             s);
}

void linear_e4m3_noalloc(const LinearE4m3Args& a, hipStream_t s) {
  check_linear(a);
  if (linear_e4m3_scratch_bytes(a.m, a.k) > kLinearE4m3ScratchBytes)
    throw std::runtime_error("m * k = " + std::to_string(a.m * a.k) + " exceeds the " +
                             std::to_string(kLinearE4m3ScratchBytes - kXqOff) +
                             " bytes the static scratch holds for the quantised activation");
  uint8_t* base = scratch_on_current_device();
  run_linear(a, base + kXqOff, reinterpret_cast<float*>(base + kPartialsOff), reinterpret_cast<float*>(base + kSxOff),
             s);
}

void init_linear_e4m3_noalloc() { (void)scratch_on_current_device(); }

}  // namespace ku::hipbk
