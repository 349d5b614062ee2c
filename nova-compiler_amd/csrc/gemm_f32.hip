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
// would have used tf32 mma.sync for f32
// (NovaGPUNestedLayoutDistributionPatterns.cpp:2460); this kernel does not,
// because tf32 breaks 1e-4 parity.
//
// Three families, with the same per-output arithmetic (so the same bits):
//   * 64x64 output tile per 256-thread workgroup, 4x4 outputs per thread,
//     K staged through LDS 16 at a time, element loads: any strides, every
//     dtype;
//   * f32 with 16-byte aligned operand rows: 128x128, 64x128, 64x96, 64x64
//     and 64x32 tiles (8x8, 4x8, 4x6, 4x4 and 4x2 outputs per thread), 16-byte global
//     loads along each operand's unit-stride dim, LDS stages [k][m] / [k][n]
//     read with 16-byte reads; the tile is chosen per problem so that the
//     CUs stay busy;
//   * the same operands, problems too small for those tiles to fill the
//     CUs: 16x16 tiles, one output per thread.
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
  int acc_c;  // the accumulators start from C's own values (C += A . B)
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
  if (a.acc_c) {
    // linalg.matmul on data-holding outs: each sum starts from C's value.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = m0 + ty * 4 + i;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = n0 + tx * 4 + j;
        if (m < a.M && n < a.N)
          acc[i][j] = elem<DT>(a.C, (int64_t)b * a.scb + (int64_t)m * a.scm + n);
      }
    }
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

// The vector forms (f32, 16-byte aligned operand rows).  A workgroup of
// 16 x 16 threads computes a (16*RM) x (16*CN) tile.  Thread (tx, ty) =
// (tid % 16, tid / 16) owns rows g*64 + ty*4 + i (g < RM/4, i < 4) and
// columns tx*4 + j (j < 4) plus, for CN = 6 / 8, 64 + tx*(CN-4) + (j-4), so
// its A values for one k are RM/4 16-byte LDS reads (broadcast within the 16
// lanes of a row of threads) and its B values one 16-byte read and, for
// CN = 6 / 8, one 8- / 16-byte read.  Per stage of KS k the workgroup loads
// its A and B panels as float4 along each operand's unit-stride dim through
// buffer resources (rows past M / N or past the slice read neighbouring data
// or zero; their outputs are not stored, and k past K is never multiplied); a
// K-contiguous operand is transposed on its way into LDS.  Stage s + 1's
// loads are in registers while stage s is multiplied.  The k loop is unrolled
// by 8, not by the stage: fully unrolled, the compiler hoists the stage's LDS
// reads (256 VGPRs, one wave per SIMD).  With a grid of a multiple of 8
// workgroups, consecutive tiles (which share A rows) run on one XCD.
constexpr int kVt = 16;  // threads per workgroup row / column

__device__ __forceinline__ __amdgpu_buffer_rsrc_t f32_rsrc(const float *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(p), (short)0, (int)bytes,
                                           0x00020000);
}

template <int RM, int CN, int KS, bool AKC, bool BKC>
__global__ __launch_bounds__(256) void gemm_exact_vec_kernel(F32Args a, uint32_t a_bytes,
                                                              uint32_t b_bytes) {
#pragma clang fp contract(off)
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  static_assert(RM == 4 || RM == 8, "rows per thread");
  static_assert(CN == 2 || CN == 4 || CN == 6 || CN == 8, "columns per thread");
  constexpr int TM = kVt * RM, TN = kVt * CN;
  constexpr int A4 = TM * KS / 4, B4 = TN * KS / 4;  // float4 per stage
  constexpr int EA = (A4 + 255) / 256, EB = (B4 + 255) / 256;
  __shared__ __attribute__((aligned(16))) float sa[2][KS][TM + 4];
  __shared__ __attribute__((aligned(16))) float sb[2][KS][TN + 4];
  int bid = blockIdx.x;
  if ((gridDim.x & 7) == 0) bid = (bid & 7) * (gridDim.x >> 3) + (bid >> 3);
  const int tiles = a.tiles_m * a.tiles_n;
  const int b = bid / tiles;
  const int t = bid - b * tiles;
  const int m0 = (t / a.tiles_n) * TM, n0 = (t % a.tiles_n) * TN;
  const int tid = threadIdx.x, tx = tid % kVt, ty = tid / kVt;
  const int64_t sa_outer = AKC ? a.sam : a.sak;
  const int64_t sb_outer = BKC ? a.sbn : a.sbk;
  const __amdgpu_buffer_rsrc_t ra = f32_rsrc(static_cast<const float *>(a.A) + b * a.sab, a_bytes);
  const __amdgpu_buffer_rsrc_t rb = f32_rsrc(static_cast<const float *>(a.B) + b * a.sbb, b_bytes);
  auto ld4 = [&](const __amdgpu_buffer_rsrc_t &r, int64_t e) __attribute__((always_inline)) {
    return __builtin_bit_cast(f32x4,
                              __builtin_amdgcn_raw_buffer_load_b128(r, (uint32_t)(e * 4), 0, 0));
  };
  // Element offset in the batch slice of float4 q of a stage.
  auto a_off = [&](int q, int k0) __attribute__((always_inline)) -> int64_t {
    if (AKC) return (int64_t)(m0 + q / (KS / 4)) * sa_outer + k0 + (q % (KS / 4)) * 4;
    return (int64_t)(k0 + q / (TM / 4)) * sa_outer + m0 + (q % (TM / 4)) * 4;
  };
  auto b_off = [&](int q, int k0) __attribute__((always_inline)) -> int64_t {
    if (BKC) return (int64_t)(n0 + q / (KS / 4)) * sb_outer + k0 + (q % (KS / 4)) * 4;
    return (int64_t)(k0 + q / (TN / 4)) * sb_outer + n0 + (q % (TN / 4)) * 4;
  };
  f32x4 ga[EA], gb[EB];
  auto gload = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < EA; ++e) {
      const int q = tid + 256 * e;
      if (A4 % 256 == 0 || q < A4) ga[e] = ld4(ra, a_off(q, k0));
    }
#pragma unroll
    for (int e = 0; e < EB; ++e) {
      const int q = tid + 256 * e;
      if (B4 % 256 == 0 || q < B4) gb[e] = ld4(rb, b_off(q, k0));
    }
  };
  auto sstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < EA; ++e) {
      const int q = tid + 256 * e;
      if (A4 % 256 != 0 && q >= A4) continue;
      if (AKC) {
#pragma unroll
        for (int u = 0; u < 4; ++u) sa[buf][(q % (KS / 4)) * 4 + u][q / (KS / 4)] = ga[e][u];
      } else {
        *reinterpret_cast<f32x4 *>(&sa[buf][q / (TM / 4)][(q % (TM / 4)) * 4]) = ga[e];
      }
    }
#pragma unroll
    for (int e = 0; e < EB; ++e) {
      const int q = tid + 256 * e;
      if (B4 % 256 != 0 && q >= B4) continue;
      if (BKC) {
#pragma unroll
        for (int u = 0; u < 4; ++u) sb[buf][(q % (KS / 4)) * 4 + u][q / (KS / 4)] = gb[e][u];
      } else {
        *reinterpret_cast<f32x4 *>(&sb[buf][q / (TN / 4)][(q % (TN / 4)) * 4]) = gb[e];
      }
    }
  };
  auto col = [&](int j) __attribute__((always_inline)) {
    if (CN == 2) return tx * 2 + j;
    return j < 4 ? tx * 4 + j : 4 * kVt + tx * (CN - 4) + (j - 4);
  };
  const bool has_bias = (a.epi == NOVA_HIP_EPI_BIAS || a.epi == NOVA_HIP_EPI_BIAS_GELU);
  const bool has_gelu = (a.epi == NOVA_HIP_EPI_BIAS_GELU || a.epi == NOVA_HIP_EPI_GELU);
  float acc[RM][CN];
#pragma unroll
  for (int j = 0; j < CN; ++j) {
    const int n = n0 + col(j);
    const float init = (has_bias && n < a.N) ? bias_value(a.bias, a.bias_dt, n) : 0.0f;
#pragma unroll
    for (int i = 0; i < RM; ++i) acc[i][j] = init;
  }
  if (a.acc_c) {
    // linalg.matmul on data-holding outs: each sum starts from C's value.
#pragma unroll
    for (int i = 0; i < RM; ++i) {
      const int m = m0 + (i >> 2) * 4 * kVt + ty * 4 + (i & 3);
      const float *crow = static_cast<const float *>(a.C) + (int64_t)b * a.scb + (int64_t)m * a.scm;
#pragma unroll
      for (int j = 0; j < CN; ++j) {
        const int n = n0 + col(j);
        if (m < a.M && n < a.N) acc[i][j] = crow[n];
      }
    }
  }
  auto step = [&](int buf, int kk) __attribute__((always_inline)) {
    f32x4 av[RM / 4];
#pragma unroll
    for (int g = 0; g < RM / 4; ++g)
      av[g] = *reinterpret_cast<const f32x4 *>(&sa[buf][kk][g * 4 * kVt + ty * 4]);
    float bv[CN];
    if constexpr (CN == 2) {
      const f32x2 b0 = *reinterpret_cast<const f32x2 *>(&sb[buf][kk][tx * 2]);
      bv[0] = b0[0];
      bv[1] = b0[1];
    } else {
      const f32x4 b0 = *reinterpret_cast<const f32x4 *>(&sb[buf][kk][tx * 4]);
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = b0[j];
    }
    if constexpr (CN == 8) {
      const f32x4 b1 = *reinterpret_cast<const f32x4 *>(&sb[buf][kk][4 * kVt + tx * 4]);
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[4 + j] = b1[j];
    } else if constexpr (CN == 6) {
      const f32x2 b1 = *reinterpret_cast<const f32x2 *>(&sb[buf][kk][4 * kVt + tx * 2]);
      bv[4] = b1[0];
      bv[5] = b1[1];
    }
#pragma unroll
    for (int i = 0; i < RM; ++i) {
      const float ai = av[i >> 2][i & 3];
#pragma unroll
      for (int j = 0; j < CN; ++j) {
        const float p = ai * bv[j];
        acc[i][j] = acc[i][j] + p;
      }
    }
  };
  gload(0);
  sstore(0);
  __syncthreads();
  int buf = 0;
  for (int k0 = 0; k0 < a.K; k0 += KS) {
    const bool more = k0 + KS < a.K;
    if (more) gload(k0 + KS);
    // Only the stage's real k: a padded k would add 0 * b.
    const int kend = a.K - k0 < KS ? a.K - k0 : KS;
#pragma unroll 8
    for (int kk = 0; kk < kend; ++kk) step(buf, kk);
    if (more) sstore(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }
#pragma unroll
  for (int i = 0; i < RM; ++i) {
    const int m = m0 + (i >> 2) * 4 * kVt + ty * 4 + (i & 3);
    if (m >= a.M) continue;
    float *crow = static_cast<float *>(a.C) + (int64_t)b * a.scb + (int64_t)m * a.scm;
#pragma unroll
    for (int j = 0; j < CN; ++j) {
      const int n = n0 + col(j);
      if (n >= a.N) continue;
      float v = acc[i][j];
      if (has_gelu) v = gelu_ref(v);
      crow[n] = v;
    }
  }
}

// The tiny form, for problems whose vector-form tiles leave CUs idle (config
// 1, 256^3: the 64x32 form's 32 tiles occupy 32 of 256 CUs, each thread
// running eight 256-long chains): a 16x16 tile per 256-thread workgroup,
// one output per thread.  Per stage of KS k each thread loads KS / 64 float4
// of A and of B along their unit-stride dims; LDS holds A as [m][k] and B
// as [n][k] (KS + 4 floats apart: the 16 columns a wave reads fall on 64
// distinct banks), so a thread reads four k of its row and of its column
// with two 16-byte reads.  The arithmetic per output is the other forms'.
// Stages of 128 k (in-process A/B, us, stages of 64 / 128 / 256): 256^3
// 4.88 / 4.75 / 4.50, 512^3 12.84 / 12.42 / 13.95 (256-deep stages leave
// two workgroups per CU), 64x64x1024 13.4 / 12.1 / 11.2; the 64x32 form
// took 14.1, 25.7 and 47.9.
constexpr int kTinyKs = 128;

template <bool AKC, bool BKC>
__global__ __launch_bounds__(256) void gemm_exact_tiny_kernel(F32Args a, uint32_t a_bytes,
                                                               uint32_t b_bytes) {
#pragma clang fp contract(off)
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  constexpr int KS = kTinyKs, P = KS + 4;
  constexpr int E = KS / 64;  // float4 of each operand per thread per stage
  static_assert(KS % 64 == 0, "a stage is a whole number of float4 per thread");
  __shared__ __attribute__((aligned(16))) float sa[2][kVt * P];
  __shared__ __attribute__((aligned(16))) float sb[2][kVt * P];
  const int tiles = a.tiles_m * a.tiles_n;
  const int b = blockIdx.x / tiles;
  const int t = blockIdx.x - b * tiles;
  const int m0 = (t / a.tiles_n) * kVt, n0 = (t % a.tiles_n) * kVt;
  const int tid = threadIdx.x, tx = tid % kVt, ty = tid / kVt;
  const int64_t sa_outer = AKC ? a.sam : a.sak;
  const int64_t sb_outer = BKC ? a.sbn : a.sbk;
  const __amdgpu_buffer_rsrc_t ra = f32_rsrc(static_cast<const float *>(a.A) + b * a.sab, a_bytes);
  const __amdgpu_buffer_rsrc_t rb = f32_rsrc(static_cast<const float *>(a.B) + b * a.sbb, b_bytes);
  // float4 q = tid + 256 e of a stage: K-contiguous, row q / (KS / 4) and
  // k 4 (q % (KS / 4)); otherwise k q / 4 and rows 4 (q % 4) .. + 3.  Rows
  // past M / N read neighbouring data or zero (their outputs are not
  // stored); k past K is never multiplied.
  auto row_of = [&](int q) __attribute__((always_inline)) { return q / (KS / 4); };
  auto k4_of = [&](int q) __attribute__((always_inline)) { return (q % (KS / 4)) * 4; };
  auto ld4 = [&](const __amdgpu_buffer_rsrc_t &r, int64_t e) __attribute__((always_inline)) {
    return __builtin_bit_cast(f32x4,
                              __builtin_amdgcn_raw_buffer_load_b128(r, (uint32_t)(e * 4), 0, 0));
  };
  f32x4 ga[E], gb[E];
  auto gload = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int q = tid + 256 * e;
      ga[e] = ld4(ra, AKC ? (int64_t)(m0 + row_of(q)) * sa_outer + k0 + k4_of(q)
                          : (int64_t)(k0 + q / 4) * sa_outer + m0 + (q % 4) * 4);
      gb[e] = ld4(rb, BKC ? (int64_t)(n0 + row_of(q)) * sb_outer + k0 + k4_of(q)
                          : (int64_t)(k0 + q / 4) * sb_outer + n0 + (q % 4) * 4);
    }
  };
  auto sstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int q = tid + 256 * e;
      if (AKC) {
        *reinterpret_cast<f32x4 *>(&sa[buf][row_of(q) * P + k4_of(q)]) = ga[e];
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) sa[buf][((q % 4) * 4 + u) * P + q / 4] = ga[e][u];
      }
      if (BKC) {
        *reinterpret_cast<f32x4 *>(&sb[buf][row_of(q) * P + k4_of(q)]) = gb[e];
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) sb[buf][((q % 4) * 4 + u) * P + q / 4] = gb[e][u];
      }
    }
  };
  const int m = m0 + ty, n = n0 + tx;
  const bool has_bias = (a.epi == NOVA_HIP_EPI_BIAS || a.epi == NOVA_HIP_EPI_BIAS_GELU);
  const bool has_gelu = (a.epi == NOVA_HIP_EPI_BIAS_GELU || a.epi == NOVA_HIP_EPI_GELU);
  float acc = (has_bias && n < a.N) ? bias_value(a.bias, a.bias_dt, n) : 0.0f;
  // linalg.matmul on data-holding outs: the sum starts from C's value.
  if (a.acc_c && m < a.M && n < a.N)
    acc = static_cast<const float *>(a.C)[(int64_t)b * a.scb + (int64_t)m * a.scm + n];
  gload(0);
  sstore(0);
  __syncthreads();
  int buf = 0;
  for (int k0 = 0; k0 < a.K; k0 += KS) {
    const bool more = k0 + KS < a.K;
    if (more) gload(k0 + KS);
    const float *ar = &sa[buf][ty * P], *br = &sb[buf][tx * P];
    if (a.K - k0 >= KS) {
#pragma unroll 4
      for (int kq = 0; kq < KS / 4; ++kq) {
        const f32x4 av = *reinterpret_cast<const f32x4 *>(ar + 4 * kq);
        const f32x4 bv = *reinterpret_cast<const f32x4 *>(br + 4 * kq);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float p = av[u] * bv[u];
          acc = acc + p;
        }
      }
    } else {
      // The last, partial stage: only its real k (a padded k would add
      // 0 * b, which turns a -0 sum into +0 and an infinite b into NaN).
      for (int kk = 0; kk < a.K - k0; ++kk) {
        const float p = ar[kk] * br[kk];
        acc = acc + p;
      }
    }
    if (more) sstore(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }
  if (m < a.M && n < a.N) {
    float v = acc;
    if (has_gelu) v = gelu_ref(v);
    static_cast<float *>(a.C)[(int64_t)b * a.scb + (int64_t)m * a.scm + n] = v;
  }
}

// The vector forms: rows and columns per thread, k per stage, and the
// relative rate of one CU running two or more of its workgroups (measured on
// the GPT step's shapes: 55, 52, 51 and ~44 TFLOP/s when every CU holds
// several tiles; the 64x32 form's 0.6 keeps it to problems of few tiles,
// where its twice as many waves hide latency that the others cannot).
struct VecForm {
  int rm, cn, ks;
  double rate;
};
constexpr VecForm kVecForms[] = {{8, 8, 16, 1.0}, {4, 8, 16, 0.95}, {4, 6, 32, 0.93},
                                 {4, 4, 64, 0.8}, {4, 2, 64, 0.6}};
constexpr int kNumVecForms = sizeof(kVecForms) / sizeof(kVecForms[0]);
constexpr double kTinyRate = 0.5;

template <bool AKC, bool BKC>
void launch_tiny_t(const F32Args &a, uint32_t ab, uint32_t bb, unsigned grid, hipStream_t s) {
  hipLaunchKernelGGL((gemm_exact_tiny_kernel<AKC, BKC>), dim3(grid), dim3(256), 0, s, a, ab, bb);
}

void launch_tiny(const F32Args &a, bool akc, bool bkc, uint32_t ab, uint32_t bb, unsigned grid,
                 hipStream_t s) {
  if (akc && bkc) launch_tiny_t<true, true>(a, ab, bb, grid, s);
  else if (akc) launch_tiny_t<true, false>(a, ab, bb, grid, s);
  else if (bkc) launch_tiny_t<false, true>(a, ab, bb, grid, s);
  else launch_tiny_t<false, false>(a, ab, bb, grid, s);
}

template <int RM, int CN, int KS>
void launch_vec(const F32Args &a, bool akc, bool bkc, uint32_t ab, uint32_t bb, unsigned grid,
                hipStream_t s) {
  const dim3 g(grid), blk(256);
  if (akc && bkc)
    hipLaunchKernelGGL((gemm_exact_vec_kernel<RM, CN, KS, true, true>), g, blk, 0, s, a, ab, bb);
  else if (akc)
    hipLaunchKernelGGL((gemm_exact_vec_kernel<RM, CN, KS, true, false>), g, blk, 0, s, a, ab, bb);
  else if (bkc)
    hipLaunchKernelGGL((gemm_exact_vec_kernel<RM, CN, KS, false, true>), g, blk, 0, s, a, ab, bb);
  else
    hipLaunchKernelGGL((gemm_exact_vec_kernel<RM, CN, KS, false, false>), g, blk, 0, s, a, ab, bb);
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
  a.acc_c = p.acc_c ? 1 : 0;
  // The vector forms: f32 with 16-byte aligned operand rows (aligned bases,
  // outer and batch strides multiples of 4, 32-bit buffer offsets).  The
  // form is the one of least estimated time: the tiles run in waves of two
  // per CU, each wave taking the tile's area over the form's rate.  The
  // deep-stage 64x32 form wins where there are few tiles and long K (the
  // GPT step's MLP weight gradients [384, 8192] x [8192, 1536]: 288 tiles,
  // 0.59 -> 0.37 ms against the 64x64 form, whose one wave per SIMD cannot
  // hide its loads); the 64x96 form gives the LM-head input gradient
  // [8192, 50304] x [50304, 384] exactly two tiles per CU (6.9 ms against
  // 10.0 ms for the scalar 64x64 form).
  if (p.in_dt == NOVA_HIP_DT_F32) {
    const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
    const int64_t a_ext = p.a_kcontig ? (p.M - 1) * p.sa_outer + p.K : (p.K - 1) * p.sa_outer + p.M;
    const int64_t b_ext = p.b_kcontig ? (p.N - 1) * p.sb_outer + p.K : (p.K - 1) * p.sb_outer + p.N;
    const bool vec = aligned16(p.A) && aligned16(p.B) && p.sa_outer % 4 == 0 &&
                     p.sb_outer % 4 == 0 && p.sab % 4 == 0 && p.sbb % 4 == 0;
    if (vec && p.K > 0 && a_ext * 4 <= 0x7fffffff && b_ext * 4 <= 0x7fffffff) {
      int best = -1;
      double best_cost = 0.0;
      int64_t best_tiles = 0;
      for (int f = 0; f < kNumVecForms; ++f) {
        const VecForm &v = kVecForms[f];
        const int64_t tm = 16 * v.rm, tn = 16 * v.cn;
        const int64_t tiles = p.batch * ((p.M + tm - 1) / tm) * ((p.N + tn - 1) / tn);
        if (tiles > 0x7fffffff) continue;
        const int64_t waves = (tiles + 2 * (int64_t)cus - 1) / (2 * (int64_t)cus);
        const double cost = (double)waves * (double)(tm * tn) / v.rate;
        if (best < 0 || cost < best_cost) {
          best = f;
          best_cost = cost;
          best_tiles = tiles;
        }
      }
      // The tiny form, only where the smallest vector form's tiles leave
      // CUs idle; its tiles are costed like the others' at rate 0.5.
      const int64_t small_tiles = p.batch * ((p.M + 63) / 64) * ((p.N + 31) / 32);
      const int64_t tiny_tiles = p.batch * ((p.M + kVt - 1) / kVt) * ((p.N + kVt - 1) / kVt);
      if (small_tiles < cus && tiny_tiles <= 0x7fffffff) {
        const int64_t waves = (tiny_tiles + 2 * (int64_t)cus - 1) / (2 * (int64_t)cus);
        if ((double)waves * (kVt * kVt) / kTinyRate < best_cost) {
          a.tiles_m = (int)((p.M + kVt - 1) / kVt);
          a.tiles_n = (int)((p.N + kVt - 1) / kVt);
          launch_tiny(a, p.a_kcontig, p.b_kcontig, (uint32_t)(a_ext * 4), (uint32_t)(b_ext * 4),
                      (unsigned)tiny_tiles, s);
          return check_hip(hipGetLastError(), "gemm_exact launch");
        }
      }
      if (best >= 0) {
        const VecForm &v = kVecForms[best];
        a.tiles_m = (int)((p.M + 16 * v.rm - 1) / (16 * v.rm));
        a.tiles_n = (int)((p.N + 16 * v.cn - 1) / (16 * v.cn));
        const uint32_t ab = (uint32_t)(a_ext * 4), bb = (uint32_t)(b_ext * 4);
        const unsigned grid = (unsigned)best_tiles;
        const bool akc = p.a_kcontig, bkc = p.b_kcontig;
        switch (best) {
          case 0: launch_vec<8, 8, 16>(a, akc, bkc, ab, bb, grid, s); break;
          case 1: launch_vec<4, 8, 16>(a, akc, bkc, ab, bb, grid, s); break;
          case 2: launch_vec<4, 6, 32>(a, akc, bkc, ab, bb, grid, s); break;
          case 3: launch_vec<4, 4, 64>(a, akc, bkc, ab, bb, grid, s); break;
          default: launch_vec<4, 2, 64>(a, akc, bkc, ab, bb, grid, s); break;
        }
        return check_hip(hipGetLastError(), "gemm_exact launch");
      }
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
