// MFMA GEMM kernels for gfx950 (kernel family 2) — filled in by the tuned kernels.
#include <hip/hip_runtime.h>

#include "kernels.h"
#include "numeric.h"

namespace ku::hipbk {

bool gemm_mfma_ok(const GemmArgs&) { return false; }
const char* gemm_mfma_name(const GemmArgs&) { return "gemm_mfma"; }
void launch_gemm_mfma(const GemmArgs&, hipStream_t) {}

bool attention_mfma_ok(const AttnArgs&) { return false; }
void launch_attention_mfma(const AttnArgs&, hipStream_t) {}

}  // namespace ku::hipbk
