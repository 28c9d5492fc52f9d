// Fused scaled-dot-product attention over [bh, s, d] (kernel family 4).
//
// Semantics: out = softmax(scale * q k^T [+ causal -inf above the diagonal]) v per head,
// the oracle of `Op::Sdpa` (kurumi_core/src/interp/nn.rs:125-172) and of the decomposed
// chain (graph/ops/nn/attention.rs:97-113). The kernel keeps scores and the running
// softmax in f32 (online softmax, never materialising [s, s]) and rounds the output once.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>

#include "kernels.h"
#include "numeric.h"

namespace ku::hipbk {

void launch_attention_mfma(const AttnArgs& a, hipStream_t s);
bool attention_mfma_ok(const AttnArgs& a);

namespace {

// Reference-grade fallback: one thread per query row, online softmax in registers.
template <int D, int DT, class T>
__global__ void __launch_bounds__(64) attn_rowwise_k(AttnArgs a) {
  const int64_t head = blockIdx.y;
  const int64_t qi = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (qi >= a.s) return;
  const T* Q = static_cast<const T*>(a.q) + head * a.s * D;
  const T* K = static_cast<const T*>(a.k) + head * a.s * D;
  const T* Vv = static_cast<const T*>(a.v) + head * a.s * D;
  float q[D], acc[D];
#pragma unroll
  for (int t = 0; t < D; ++t) {
    q[t] = load_elem<DT, T, float>(Q[qi * D + t]);
    acc[t] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  const int64_t kend = a.causal ? qi + 1 : a.s;
  for (int64_t j = 0; j < kend; ++j) {
    float sc = 0.f;
#pragma unroll
    for (int t = 0; t < D; ++t) sc = fmaf(q[t], load_elem<DT, T, float>(K[j * D + t]), sc);
    sc *= a.scale;
    float mn = fmaxf(m, sc);
    float corr = expf(m - mn);
    float p = expf(sc - mn);
    l = l * corr + p;
#pragma unroll
    for (int t = 0; t < D; ++t) acc[t] = acc[t] * corr + p * load_elem<DT, T, float>(Vv[j * D + t]);
    m = mn;
  }
  T* O = static_cast<T*>(a.o) + head * a.s * D;
  const float inv = 1.f / l;
#pragma unroll
  for (int t = 0; t < D; ++t) O[qi * D + t] = store_elem<DT, T, float>(acc[t] * inv);
}

template <int D>
void launch_rowwise(const AttnArgs& a, hipStream_t s) {
  dim3 grid((unsigned)((a.s + 63) / 64), (unsigned)a.bh);
  switch (a.dtype) {
    case GT_BF16: hipLaunchKernelGGL((attn_rowwise_k<D, GT_BF16, uint16_t>), grid, dim3(64), 0, s, a); return;
    case GT_F16: hipLaunchKernelGGL((attn_rowwise_k<D, GT_F16, uint16_t>), grid, dim3(64), 0, s, a); return;
    case GT_F32: hipLaunchKernelGGL((attn_rowwise_k<D, GT_F32, float>), grid, dim3(64), 0, s, a); return;
    default: throw std::runtime_error("kurumi_hip attention: unsupported dtype");
  }
}

}  // namespace

bool attn_supported(const AttnArgs& a) {
  bool dt = a.dtype == GT_BF16 || a.dtype == GT_F16 || a.dtype == GT_F32;
  bool d = a.d == 32 || a.d == 64 || a.d == 128;
  return dt && d && a.s > 0 && a.bh > 0;
}

const char* attn_variant(const AttnArgs& a) {
  if (attention_mfma_ok(a)) return "attn_mfma";
  return "attn_rowwise";
}

void launch_attention(const AttnArgs& a, hipStream_t s) {
  if (!attn_supported(a)) throw std::runtime_error("kurumi_hip attention: unsupported shape");
  if (attention_mfma_ok(a)) {
    launch_attention_mfma(a, s);
    return;
  }
  switch (a.d) {
    case 32: launch_rowwise<32>(a, s); return;
    case 64: launch_rowwise<64>(a, s); return;
    default: launch_rowwise<128>(a, s); return;
  }
}

}  // namespace ku::hipbk
