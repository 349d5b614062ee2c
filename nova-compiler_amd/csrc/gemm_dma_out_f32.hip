// Instantiates the LDS-DMA GEMM kernels (gemm_dma.h, and its persistent form
// gemm_pers.h for problems of at least one full round of tiles, with or
// without a bias / GELU epilogue) for f32 output: both
// input dtypes and the four operand layouts.
#include "gemm_pers.h"

namespace nova_hip {

int32_t launch_gemm_dma_f32out(const gemm::GemmArgs &a, int in_dt, bool akc, bool bkc,
                               hipStream_t s) {
  if (pers::applicable(a)) return pers::launch_out<NOVA_HIP_DT_F32>(a, in_dt, akc, bkc, s);
  return dma::launch_out<NOVA_HIP_DT_F32>(a, in_dt, akc, bkc, s);
}

}  // namespace nova_hip
