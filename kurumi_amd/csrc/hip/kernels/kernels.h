// Host-side launchers of the precompiled gfx950 kernels (GEMM and flash attention).
// Fused pointwise/reduce kernels are generated at run time (codegen.cpp) instead.
#pragma once
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <string>

namespace ku::hipbk {

// Element type tags for the GEMM launchers (match ku::DType values).
enum GemmType : int { GT_F8E4M3 = 9, GT_F8E5M2 = 10, GT_F16 = 11, GT_BF16 = 12, GT_F32 = 13, GT_F64 = 14, GT_I32 = 7, GT_I64 = 8 };

struct GemmArgs {
  const void* a = nullptr;
  const void* b = nullptr;
  void* c = nullptr;
  int64_t sab = 0, sam = 0, sak = 0;  // A[b][m][k] element strides
  int64_t sbb = 0, sbk = 0, sbn = 0;  // B[b][k][n] element strides
  int64_t batch = 1, m = 0, n = 0, k = 0;
  int in_type = GT_BF16;
  int out_type = GT_BF16;
  // optional epilogue: c = acc * alpha[0] * col_scale[n * col_scale_stride]
  const float* alpha = nullptr;
  const float* col_scale = nullptr;
  int64_t col_scale_stride = 1;
  // optional fused cast: the (scaled) f32 result is first rounded to this 16-bit float type (the
  // contraction's own dtype, GT_BF16 / GT_F16), then converted to out_type; -1: no extra rounding
  int round_type = -1;
};

// Compute units of the current device (cached on first use): sizes persistent grids and tile rounds.
int cu_count();

// Short name of the kernel variant that will run (for plan labels): the MFMA kernel's element
// type, layout and tile ("gemm_mfma_bf16_nn_256x256"; "_a64" when an operand spans 2^31 bytes or
// more and the 64-bit-address DMA form runs), or "gemm_generic".
std::string gemm_variant(const GemmArgs& a);
void launch_gemm(const GemmArgs& a, hipStream_t s);

struct AttnArgs {
  const void* q = nullptr;
  const void* k = nullptr;
  const void* v = nullptr;
  void* o = nullptr;
  int64_t bh = 0, s = 0, d = 0;  // [bh, s, d] contiguous
  float scale = 1.f;
  bool causal = false;
  int dtype = GT_BF16;
};
const char* attn_variant(const AttnArgs& a);
bool attn_supported(const AttnArgs& a);
void launch_attention(const AttnArgs& a, hipStream_t s);

// Weight-only quantized matmul (quant.hip): out[M, N] = act[M, K] x dequant(qw)[N, K]^T.
struct QuantArgs {
  const void* act = nullptr;          // [M, K] contiguous, act_type
  const uint8_t* qw = nullptr;        // [N, K * bits / 8] packed, low field first
  const uint16_t* scales = nullptr;   // f16 [N, K / group]
  const uint16_t* mins = nullptr;     // f16 [N, K / group], asymmetric only
  void* out = nullptr;                // [M, N] contiguous, act_type
  void* wdq = nullptr;                // dequantized weight [N, K] (wdq_type) for the GEMM path
  void* mm_scratch = nullptr;         // quant_mm_scratch_bytes() of device scratch for the MFMA path
  bool qw_tiled = false;              // qw in the fused MFMA kernel's lane order (launch_quant_tile_weights)
  int64_t m = 0, n = 0, k = 0, group = 0;
  int bits = 4;
  bool sym = true;
  int act_type = GT_BF16;
  int wdq_type = GT_BF16;
};
bool quant_gemv_ok(const QuantArgs& a);
void launch_quant_gemv(const QuantArgs& a, hipStream_t s);
void launch_quant_dequant(const QuantArgs& a, hipStream_t s);
// fused dequant MFMA kernel: int4, bf16 / f16 act, 9 <= M <= 64, group a multiple of 64
bool quant_mm_ok(const QuantArgs& a);
// scratch of the MFMA path when it runs the act pass (groups not a multiple of 128): act re-laid
// out in the order the kernel's lanes load it (whole lines per load instruction) and its
// per-sub-group sums, written by one small pass shared by every work-group; 0 for the fused kernel
size_t quant_mm_scratch_bytes(const QuantArgs& a);
// whether the MFMA path runs the fused kernel (groups a multiple of 128, operands under 2 GiB),
// which needs no scratch and can read a weight held in its lane order
bool quant_mm_fused_ok(const QuantArgs& a);
// the lane-ordered copy of a packed int4 weight [n, k / 2]: bytes, and the pass that writes it
size_t quant_tiled_bytes(int64_t n, int64_t k);
void launch_quant_tile_weights(const uint8_t* qw, uint8_t* wt, int64_t n, int64_t k, hipStream_t s);
void launch_quant_mm(const QuantArgs& a, hipStream_t s);

// Per-tensor e4m3 activation quantisation (linear_e4m3.hip): sx = max|x| * (1/448) and
// xq = e4m3(x * (1/sx)) over n contiguous elements, in two kernels (absmax partials, then fold
// + quantise). `partials` holds actq_partials_bytes(n) bytes of scratch.
constexpr int kActqMaxPartials = 1024;
struct ActQArgs {
  const void* x = nullptr;  // [n] bf16 / f16 / f32, 16-byte aligned
  int x_type = GT_BF16;
  int64_t n = 0;
  uint8_t* xq = nullptr;    // [n] e4m3
  float* sx = nullptr;      // [1]
  float* partials = nullptr;
};
size_t actq_partials_bytes(int64_t n);
void launch_actq(const ActQArgs& a, hipStream_t s);

// The e4m3 linear on device buffers: y[M, N] = round_y((e4m3(x / sx) @ wq^T) * sx * sw[n]) with
// sx = max|x| / 448 computed on the device (the graph ku_amp_fp8 emits for one linear layer).
struct LinearE4m3Args {
  const void* x = nullptr;     // [M, K] row-major, x_type
  int x_type = GT_BF16;
  const uint8_t* wq = nullptr; // [N, K] e4m3 row-major
  const float* sw = nullptr;   // [N] per-row weight scales
  void* y = nullptr;           // [M, N] row-major, y_type
  int y_type = GT_BF16;
  int64_t m = 0, n = 0, k = 0;
};
// bytes of scratch one call needs: absmax partials, sx and the quantised activation (M*K)
size_t linear_e4m3_scratch_bytes(int64_t m, int64_t k);
void linear_e4m3(const LinearE4m3Args& a, void* scratch, size_t scratch_bytes, hipStream_t s);
// The same with scratch in a static device array of kLinearE4m3ScratchBytes per GPU (no
// allocation): m * k <= kLinearE4m3ScratchBytes - 4352. init_ looks the array up on the current GPU.
constexpr size_t kLinearE4m3ScratchBytes = (size_t(16) << 20) + 4352;
void linear_e4m3_noalloc(const LinearE4m3Args& a, hipStream_t s);
void init_linear_e4m3_noalloc();

}  // namespace ku::hipbk
