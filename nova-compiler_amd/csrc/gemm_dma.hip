// Host side of the LDS-DMA GEMM (kernels in gemm_dma.h and gemm_pers.h):
// which problems it takes, the round size of its tile order, and dispatch
// to the per-output-dtype translation units gemm_dma_out_{f32,bf16,f16}.hip,
// each of which instantiates the kernels for its output dtype (compiled in
// parallel).
#include "gemm_common.h"

namespace nova_hip {

namespace {
constexpr int kBM = 256, kBN = 256, kBK = 64;  // the tile of gemm_dma.h
}  // namespace

bool gemm_dma_applicable(const gemm::GemmArgs &a, bool akc, bool bkc, bool vec) {
  (void)akc;
  (void)bkc;
  const int64_t tiles = (int64_t)a.batch * (a.M / kBM) * (a.N / kBN);
  // Full tiles only, and vector stores need 16-byte aligned output rows.
  const bool c_ok = (reinterpret_cast<uintptr_t>(a.C) & 15u) == 0 && a.scm % 8 == 0 &&
                    a.scb % 8 == 0;
  return vec && c_ok && a.M % kBM == 0 && a.N % kBN == 0 && a.K % kBK == 0 && a.K > 0 &&
         tiles >= 128 && tiles <= 0x7fffffff;
}

int32_t launch_gemm_dma(const gemm::GemmArgs &a_in, int in_dt, bool akc, bool bkc, hipStream_t s) {
  gemm::GemmArgs a = a_in;
  a.tiles_m = a.M / kBM;
  a.tiles_n = a.N / kBN;
  // The kernels' 128 KB (160 KB persistent) of LDS allow one workgroup per
  // CU: a round is one workgroup per CU of the current device (8 XCDs, so a
  // multiple of 8); the persistent kernel launches one round.
  const int cus = device_cu_count();
  a.round = (cus > 0 && cus % 8 == 0) ? cus : 0;
  if (a.out_dt == NOVA_HIP_DT_F32) return launch_gemm_dma_f32out(a, in_dt, akc, bkc, s);
  if (a.out_dt == NOVA_HIP_DT_BF16) return launch_gemm_dma_bf16out(a, in_dt, akc, bkc, s);
  return launch_gemm_dma_f16out(a, in_dt, akc, bkc, s);
}

}  // namespace nova_hip
