// GEMM dispatch: the direct-to-LDS MFMA kernel for the bf16/f16/fp8 layouts it covers, the
// register-staged MFMA kernel as the alternative (KURUMI_HIP_GEMM_V1), the generic tiled kernel
// for everything else.
#include <hip/hip_runtime.h>

#include "kernels.h"
#include "numeric.h"

namespace ku::hipbk {

bool gemm_lds_ok(const GemmArgs& a);
void launch_gemm_lds(const GemmArgs& a, hipStream_t s);
bool gemm_mfma_ok(const GemmArgs& a);
const char* gemm_mfma_name(const GemmArgs& a);
void launch_gemm_mfma(const GemmArgs& a, hipStream_t s);

const char* gemm_variant(const GemmArgs& a) {
  if (gemm_lds_ok(a) || gemm_mfma_ok(a)) return gemm_mfma_name(a);
  return "gemm_generic";
}

void launch_gemm(const GemmArgs& a, hipStream_t s) {
  if (a.batch * a.m * a.n == 0) return;
  if (gemm_lds_ok(a)) {
    launch_gemm_lds(a, s);
    return;
  }
  if (gemm_mfma_ok(a)) {
    launch_gemm_mfma(a, s);
    return;
  }
  launch_gemm_generic(a, s);
}

}  // namespace ku::hipbk
