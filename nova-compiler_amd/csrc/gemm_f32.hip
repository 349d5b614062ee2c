// Exact GEMM: C[b,m,n] = init + sum_k A[b,m,k] * B[b,k,n], k ascending,
// every multiply and add separately rounded.  This is the arithmetic of
// Nova's CPU pipeline for f32 linalg.matmul / batch_matmul (no fast-math,
// no FMA contraction, sequential k: Pipeline.cpp:61-187), so the result is
// bit-identical to it, including the bias-initialised accumulator of
// FuseMatmulBias (FuseMatmulBias.cpp:184-188).
//
// The same kernel, instantiated for bf16 or f16, is linalg.matmul with a
// narrow outs operand: the upstream named-op body C += A * B runs in the
// outs element type, so every product and every partial sum is rounded to
// bf16 / f16 (NovaMatmulOpLowering creates such a matmul for an f16 x f16
// nova.matmul, whose result type is f16: NovaToLinalg.cpp:1027-1049,
// NovaOps.cpp:1198).  Each operation is done in f32 and rounded to the
// narrow type (RNE): a product of two narrow values is exact in f32, and
// a sum rounded first to f32 (24 bits) then to a p-bit type is the
// correctly rounded p-bit sum whenever 24 >= 2p + 2 (p = 8 for bf16, 11 for
// f16), so this is the narrow type's own IEEE arithmetic.  The reference's GPU path
// would have used tf32 mma.sync for f32 (SURVEY of
// NovaGPUNestedLayoutDistributionPatterns.cpp:2460); this kernel does not,
// because tf32 breaks 1e-4 parity.
//
// 64x64 output tile per 256-thread workgroup, 4x4 outputs per thread,
// K staged through LDS 16 at a time.  f32 GEMM is the plumbing path (bf16
// and f16 carry the throughput), so it is VALU-bound by design.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "nova_hip_internal.h"

namespace nova_hip {
namespace {

constexpr int kT = 64;   // output tile edge
constexpr int kKs = 16;  // k per LDS stage

struct F32Args {
  const void *A;
  const void *B;
  void *C;
  const void *bias;
  int64_t sab, sam, sak;
  int64_t sbb, sbk, sbn;
  int64_t scb, scm;
  int M, N, K;
  int tiles_m, tiles_n;
  int bias_dt, epi;
};

__device__ __forceinline__ float bias_value(const void *bias, int dt, int n) {
  if (dt == NOVA_HIP_DT_F32) return static_cast<const float *>(bias)[n];
  const uint16_t h = static_cast<const uint16_t *>(bias)[n];
  if (dt == NOVA_HIP_DT_BF16) return __uint_as_float(static_cast<uint32_t>(h) << 16);
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

__device__ __forceinline__ float gelu_ref(float x) {
#pragma clang fp contract(off)
  const float x2 = x * x;
  const float x3 = x2 * x;
  const float cubic = 4.471500e-02f * x3;
  const float inner = x + cubic;
  const float scaled = 0.7978845608028654f * inner;
  const float t = tanhf(scaled);
  return (0.5f * x) * (1.0f + t);
}

// Element DT of a (at element offset i) as f32 (exact).
template <int DT>
__device__ __forceinline__ float elem(const void *p, int64_t i) {
  if constexpr (DT == NOVA_HIP_DT_F32) return static_cast<const float *>(p)[i];
  const uint16_t h = static_cast<const uint16_t *>(p)[i];
  if constexpr (DT == NOVA_HIP_DT_BF16) return __uint_as_float(static_cast<uint32_t>(h) << 16);
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// Round an f32 value to DT (nearest even) and back: the accumulator's type.
template <int DT>
__device__ __forceinline__ float round_to(float x) {
  if constexpr (DT == NOVA_HIP_DT_BF16) return static_cast<float>(static_cast<__bf16>(x));
  else if constexpr (DT == NOVA_HIP_DT_F16) return static_cast<float>(static_cast<_Float16>(x));
  else return x;
}

template <int DT>
__global__ __launch_bounds__(256) void gemm_exact_kernel(F32Args a) {
#pragma clang fp contract(off)
  // Two LDS stages: stage s + 1's global loads are in registers while
  // stage s is multiplied, then written to the other buffer (one barrier
  // per stage).
  __shared__ float sa[2][kKs][kT + 4];
  __shared__ float sb[2][kKs][kT + 4];

  const int tiles = a.tiles_m * a.tiles_n;
  const int b = blockIdx.x / tiles;
  const int t = blockIdx.x - b * tiles;
  const int m0 = (t / a.tiles_n) * kT;
  const int n0 = (t % a.tiles_n) * kT;
  const int tid = threadIdx.x;
  const int tx = tid & 15, ty = tid >> 4;

  constexpr int kEsz = DT == NOVA_HIP_DT_F32 ? 4 : 2;
  const char *Ab = static_cast<const char *>(a.A) + (int64_t)b * a.sab * kEsz;
  const char *Bb = static_cast<const char *>(a.B) + (int64_t)b * a.sbb * kEsz;

  const bool has_bias = (a.epi == NOVA_HIP_EPI_BIAS || a.epi == NOVA_HIP_EPI_BIAS_GELU);
  const bool has_gelu = (a.epi == NOVA_HIP_EPI_BIAS_GELU || a.epi == NOVA_HIP_EPI_GELU);

  // 64x16 A tile and 16x64 B tile, 4 elements of each per thread, the
  // lanes along each operand's unit-stride dimension (coalesced loads).
  const bool a_kc = a.sak == 1, b_nc = a.sbn == 1;
  auto a_elem = [&](int e, int &r, int &kk) __attribute__((always_inline)) {
    const int q = tid + e * 256;
    if (a_kc) { kk = q & 15; r = q >> 4; } else { r = q & 63; kk = q >> 6; }
  };
  auto b_elem = [&](int e, int &c, int &kk) __attribute__((always_inline)) {
    const int q = tid + e * 256;
    if (b_nc) { c = q & 63; kk = q >> 6; } else { kk = q & 15; c = q >> 4; }
  };
  float ra[4], rb[4];
  auto load = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      int r, kk;
      a_elem(e, r, kk);
      const int gm = m0 + r, gk = k0 + kk;
      ra[e] = (gm < a.M && gk < a.K) ? elem<DT>(Ab, (int64_t)gm * a.sam + (int64_t)gk * a.sak)
                                     : 0.0f;
      int c, kb;
      b_elem(e, c, kb);
      const int gn = n0 + c, gkb = k0 + kb;
      rb[e] = (gn < a.N && gkb < a.K) ? elem<DT>(Bb, (int64_t)gkb * a.sbk + (int64_t)gn * a.sbn)
                                      : 0.0f;
    }
  };
  auto store = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      int r, kk;
      a_elem(e, r, kk);
      sa[buf][kk][r] = ra[e];
      int c, kb;
      b_elem(e, c, kb);
      sb[buf][kb][c] = rb[e];
    }
  };

  float acc[4][4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = n0 + tx * 4 + j;
    const float init = (has_bias && n < a.N) ? bias_value(a.bias, a.bias_dt, n) : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i][j] = init;
  }

  load(0);
  store(0);
  __syncthreads();
  int buf = 0;
  for (int k0 = 0; k0 < a.K; k0 += kKs) {
    const bool more = k0 + kKs < a.K;
    if (more) load(k0 + kKs);
    // Only the stage's real k: a padded k would add 0 * b, which turns a
    // -0 accumulator into +0 and an infinite b into NaN.
    const int kend = min(kKs, a.K - k0);
    for (int kk = 0; kk < kend; ++kk) {
      float av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = sa[buf][kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = sb[buf][kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float p = round_to<DT>(av[i] * bv[j]);
          acc[i][j] = round_to<DT>(acc[i][j] + p);
        }
    }
    if (more) store(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }

#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + ty * 4 + i;
    if (m >= a.M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + tx * 4 + j;
      if (n >= a.N) continue;
      float v = acc[i][j];
      const int64_t off = (int64_t)b * a.scb + (int64_t)m * a.scm + n;
      if constexpr (DT == NOVA_HIP_DT_F32) {
        if (has_gelu) v = gelu_ref(v);
        static_cast<float *>(a.C)[off] = v;
      } else if constexpr (DT == NOVA_HIP_DT_BF16) {
        static_cast<uint16_t *>(a.C)[off] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
      } else {
        static_cast<uint16_t *>(a.C)[off] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
      }
    }
  }
}

}  // namespace

int32_t launch_gemm_exact(const GemmProblem &p, hipStream_t s) {
  if (p.batch == 0 || p.M == 0 || p.N == 0) return NOVA_HIP_SUCCESS;
  if (p.M > 0x7fffffff || p.N > 0x7fffffff || p.K > 0x7fffffff)
    return fail(NOVA_HIP_ERANGE, "gemm_exact: dimension exceeds 2^31-1");
  if (p.out_dt != p.in_dt)
    return fail(NOVA_HIP_EDTYPE, "gemm_exact: the accumulator type must be the input type");
  if (p.in_dt != NOVA_HIP_DT_F32 &&
      (p.epi == NOVA_HIP_EPI_GELU || p.epi == NOVA_HIP_EPI_BIAS_GELU ||
       (p.epi == NOVA_HIP_EPI_BIAS && p.bias_dt != p.in_dt)))
    return fail(NOVA_HIP_EDTYPE,
                "gemm: a bf16 / f16 accumulator takes no GELU, and a bias of its own dtype only");
  F32Args a;
  a.A = p.A;
  a.B = p.B;
  a.C = p.C;
  a.bias = p.bias;
  a.sab = p.sab;
  a.sbb = p.sbb;
  // Expand the (contiguous dim, outer stride) description back to strides.
  a.sam = p.a_kcontig ? p.sa_outer : 1;
  a.sak = p.a_kcontig ? 1 : p.sa_outer;
  a.sbk = p.b_kcontig ? 1 : p.sb_outer;
  a.sbn = p.b_kcontig ? p.sb_outer : 1;
  a.scb = p.scb;
  a.scm = p.scm;
  a.M = (int)p.M;
  a.N = (int)p.N;
  a.K = (int)p.K;
  a.tiles_m = (int)((p.M + kT - 1) / kT);
  a.tiles_n = (int)((p.N + kT - 1) / kT);
  a.bias_dt = p.bias_dt;
  a.epi = p.epi;
  const int64_t total = p.batch * a.tiles_m * a.tiles_n;
  if (total > 0x7fffffff) return fail(NOVA_HIP_ERANGE, "gemm_exact: grid too large");
  if (p.in_dt == NOVA_HIP_DT_BF16)
    hipLaunchKernelGGL(gemm_exact_kernel<NOVA_HIP_DT_BF16>, dim3((unsigned)total), dim3(256), 0, s, a);
  else if (p.in_dt == NOVA_HIP_DT_F16)
    hipLaunchKernelGGL(gemm_exact_kernel<NOVA_HIP_DT_F16>, dim3((unsigned)total), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(gemm_exact_kernel<NOVA_HIP_DT_F32>, dim3((unsigned)total), dim3(256), 0, s, a);
  return check_hip(hipGetLastError(), "gemm_exact launch");
}

}  // namespace nova_hip
