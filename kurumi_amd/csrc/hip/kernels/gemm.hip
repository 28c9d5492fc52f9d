// GEMM dispatch: the direct-to-LDS MFMA kernel (gemm_lds.hip) for the bf16 / f16 / e4m3
// layouts it covers, the generic tiled kernel (gemm_generic.hip) for everything else.
#include <hip/hip_runtime.h>

#include "kernels.h"
#include "numeric.h"

namespace ku::hipbk {

bool gemm_lds_ok(const GemmArgs& a);
std::string gemm_lds_name(const GemmArgs& a);
void launch_gemm_lds(const GemmArgs& a, hipStream_t s);

std::string gemm_variant(const GemmArgs& a) {
  if (gemm_lds_ok(a)) return gemm_lds_name(a);
  return "gemm_generic";
}

void launch_gemm(const GemmArgs& a, hipStream_t s) {
  if (a.batch * a.m * a.n == 0) return;
  if (gemm_lds_ok(a)) {
    launch_gemm_lds(a, s);
    return;
  }
  launch_gemm_generic(a, s);
}

}  // namespace ku::hipbk
