// Instantiates the LDS-DMA GEMM kernel (gemm_dma.h) for f16 output: both
// input dtypes and the four operand layouts.
#include "gemm_dma.h"

namespace nova_hip {

int32_t launch_gemm_dma_f16out(const gemm::GemmArgs &a, int in_dt, bool akc, bool bkc,
                               hipStream_t s) {
  return dma::launch_out<NOVA_HIP_DT_F16>(a, in_dt, akc, bkc, s);
}

}  // namespace nova_hip
