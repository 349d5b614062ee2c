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
// Two forms, with the same per-output arithmetic (so the same bits):
//   * 64x64 output tile per 256-thread workgroup, 4x4 outputs per thread,
//     K staged through LDS 16 at a time, element loads: any strides, every
//     dtype, and problems of few tiles;
//   * f32 with 16-byte aligned operand rows and enough 128x128 tiles to give
//     every CU two workgroups: 8x8 outputs per thread, 16-byte global loads
//     along each operand's unit-stride dim, LDS stages [k][m] / [k][n] read
//     with 16-byte reads (half the LDS bytes per multiply-add of the 4x4
//     form, whose reads matched the VALU issue rate).
// Without contraction every multiply-add is two VALU operations, so the
// ceiling is half the f32 FMA rate.
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

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

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

// The 128x128 form (f32).  Thread (tx, ty) = (tid % 16, tid / 16) owns
// rows {ty*4 + i, 64 + ty*4 + i} and columns {tx*4 + j, 64 + tx*4 + j},
// i, j < 4, so its A and B values for one k are two 16-byte LDS reads each
// (A's broadcast within the 16 lanes of a row of threads, B's contiguous).
// Per stage each thread loads two float4 of A and two of B along the
// operands' unit-stride dims through buffer resources (rows past M / N or
// past the slice read zero or neighbouring data; their outputs are not
// stored, and k past K is never multiplied); a K-contiguous operand is
// transposed on its way into LDS.  The k loop is unrolled by 8, not 16:
// fully unrolled, the compiler hoisted the LDS reads of the whole stage
// (256 VGPRs, one wave per SIMD); unrolled by 8 the kernel needs 122, four
// waves per SIMD.
constexpr int kT2 = 128;
constexpr int kLd2 = kT2 + 4;  // LDS row pitch (floats)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t f32_rsrc(const float *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(p), (short)0, (int)bytes,
                                           0x00020000);
}

template <bool AKC, bool BKC>
__global__ __launch_bounds__(256) void gemm_exact128_kernel(F32Args a, uint32_t a_bytes,
                                                             uint32_t b_bytes) {
#pragma clang fp contract(off)
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  __shared__ __attribute__((aligned(16))) float sa[2][kKs][kLd2];
  __shared__ __attribute__((aligned(16))) float sb[2][kKs][kLd2];
  const int tiles = a.tiles_m * a.tiles_n;
  const int b = blockIdx.x / tiles;
  const int t = blockIdx.x - b * tiles;
  const int m0 = (t / a.tiles_n) * kT2, n0 = (t % a.tiles_n) * kT2;
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int64_t sa_outer = AKC ? a.sam : a.sak;
  const int64_t sb_outer = BKC ? a.sbn : a.sbk;
  const __amdgpu_buffer_rsrc_t ra = f32_rsrc(static_cast<const float *>(a.A) + b * a.sab, a_bytes);
  const __amdgpu_buffer_rsrc_t rb = f32_rsrc(static_cast<const float *>(a.B) + b * a.sbb, b_bytes);
  auto ld4 = [&](const __amdgpu_buffer_rsrc_t &r, int64_t e) __attribute__((always_inline)) {
    return __builtin_bit_cast(f32x4,
                              __builtin_amdgcn_raw_buffer_load_b128(r, (uint32_t)(e * 4), 0, 0));
  };
  // Element offset in the batch slice of the thread's float4 e of a stage.
  auto a_off = [&](int e, int k0) __attribute__((always_inline)) -> int64_t {
    const int q = tid + 256 * e;
    if (AKC) return (int64_t)(m0 + (q >> 2)) * sa_outer + k0 + (q & 3) * 4;
    return (int64_t)(k0 + (q >> 5)) * sa_outer + m0 + (q & 31) * 4;
  };
  auto b_off = [&](int e, int k0) __attribute__((always_inline)) -> int64_t {
    const int q = tid + 256 * e;
    if (BKC) return (int64_t)(n0 + (q >> 2)) * sb_outer + k0 + (q & 3) * 4;
    return (int64_t)(k0 + (q >> 5)) * sb_outer + n0 + (q & 31) * 4;
  };
  f32x4 ga[2], gb[2];
  auto gload = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      ga[e] = ld4(ra, a_off(e, k0));
      gb[e] = ld4(rb, b_off(e, k0));
    }
  };
  auto sstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int q = tid + 256 * e;
      if (AKC) {
#pragma unroll
        for (int u = 0; u < 4; ++u) sa[buf][(q & 3) * 4 + u][q >> 2] = ga[e][u];
      } else {
        *reinterpret_cast<f32x4 *>(&sa[buf][q >> 5][(q & 31) * 4]) = ga[e];
      }
      if (BKC) {
#pragma unroll
        for (int u = 0; u < 4; ++u) sb[buf][(q & 3) * 4 + u][q >> 2] = gb[e][u];
      } else {
        *reinterpret_cast<f32x4 *>(&sb[buf][q >> 5][(q & 31) * 4]) = gb[e];
      }
    }
  };
  const bool has_bias = (a.epi == NOVA_HIP_EPI_BIAS || a.epi == NOVA_HIP_EPI_BIAS_GELU);
  const bool has_gelu = (a.epi == NOVA_HIP_EPI_BIAS_GELU || a.epi == NOVA_HIP_EPI_GELU);
  float acc[8][8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int n = n0 + (j >> 2) * 64 + tx * 4 + (j & 3);
    const float init = (has_bias && n < a.N) ? bias_value(a.bias, a.bias_dt, n) : 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i][j] = init;
  }
  auto step = [&](int buf, int kk) __attribute__((always_inline)) {
    const f32x4 a0 = *reinterpret_cast<const f32x4 *>(&sa[buf][kk][ty * 4]);
    const f32x4 a1 = *reinterpret_cast<const f32x4 *>(&sa[buf][kk][64 + ty * 4]);
    const f32x4 b0 = *reinterpret_cast<const f32x4 *>(&sb[buf][kk][tx * 4]);
    const f32x4 b1 = *reinterpret_cast<const f32x4 *>(&sb[buf][kk][64 + tx * 4]);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float ai = i < 4 ? a0[i] : a1[i - 4];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float p = ai * (j < 4 ? b0[j] : b1[j - 4]);
        acc[i][j] = acc[i][j] + p;
      }
    }
  };
  gload(0);
  sstore(0);
  __syncthreads();
  int buf = 0;
  for (int k0 = 0; k0 < a.K; k0 += kKs) {
    const bool more = k0 + kKs < a.K;
    if (more) gload(k0 + kKs);
    // Only the stage's real k: a padded k would add 0 * b.
    const int kend = a.K - k0 < kKs ? a.K - k0 : kKs;
#pragma unroll 8
    for (int kk = 0; kk < kend; ++kk) step(buf, kk);
    if (more) sstore(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int m = m0 + (i >> 2) * 64 + ty * 4 + (i & 3);
    if (m >= a.M) continue;
    float *crow = static_cast<float *>(a.C) + (int64_t)b * a.scb + (int64_t)m * a.scm;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int n = n0 + (j >> 2) * 64 + tx * 4 + (j & 3);
      if (n >= a.N) continue;
      float v = acc[i][j];
      if (has_gelu) v = gelu_ref(v);
      crow[n] = v;
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
  // The 128x128 form: f32, 16-byte aligned operand rows (aligned bases, outer
  // and batch strides multiples of 4, 32-bit buffer offsets), and at least
  // two of its tiles per CU (with fewer it leaves CUs idle and the 64x64
  // form, with four times the tiles, is faster: on the GPT step's
  // [8192, 50304] x [50304, 384] it took 13.8 against 10.0 ms).
  if (p.in_dt == NOVA_HIP_DT_F32) {
    const int64_t t128 = p.batch * ((p.M + 127) / 128) * ((p.N + 127) / 128);
    const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
    const int64_t a_ext = p.a_kcontig ? (p.M - 1) * p.sa_outer + p.K : (p.K - 1) * p.sa_outer + p.M;
    const int64_t b_ext = p.b_kcontig ? (p.N - 1) * p.sb_outer + p.K : (p.K - 1) * p.sb_outer + p.N;
    const bool vec = aligned16(p.A) && aligned16(p.B) && p.sa_outer % 4 == 0 &&
                     p.sb_outer % 4 == 0 && p.sab % 4 == 0 && p.sbb % 4 == 0;
    if (vec && p.K > 0 && t128 >= 2 * (int64_t)cus && t128 <= 0x7fffffff &&
        a_ext * 4 <= 0x7fffffff && b_ext * 4 <= 0x7fffffff) {
      a.tiles_m = (int)((p.M + 127) / 128);
      a.tiles_n = (int)((p.N + 127) / 128);
      const uint32_t ab = (uint32_t)(a_ext * 4), bb = (uint32_t)(b_ext * 4);
      const dim3 g((unsigned)t128);
      if (p.a_kcontig && p.b_kcontig)
        hipLaunchKernelGGL((gemm_exact128_kernel<true, true>), g, dim3(256), 0, s, a, ab, bb);
      else if (p.a_kcontig)
        hipLaunchKernelGGL((gemm_exact128_kernel<true, false>), g, dim3(256), 0, s, a, ab, bb);
      else if (p.b_kcontig)
        hipLaunchKernelGGL((gemm_exact128_kernel<false, true>), g, dim3(256), 0, s, a, ab, bb);
      else
        hipLaunchKernelGGL((gemm_exact128_kernel<false, false>), g, dim3(256), 0, s, a, ab, bb);
      return check_hip(hipGetLastError(), "gemm_exact launch");
    }
  }
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
