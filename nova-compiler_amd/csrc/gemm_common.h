// Device-side pieces shared by the two MFMA GEMM kernels (register-staged,
// gemm_mfma.hip; LDS-DMA, gemm_dma.hip): argument block, MFMA wrapper,
// buffer resources, XCD-aware tile order and the bias / GELU / store
// epilogue.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "nova_hip_internal.h"

namespace nova_hip {
namespace gemm {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;          // four wave64s in a 2x2 grid
constexpr uint32_t kOOB = 0x80000000u;  // buffer offset beyond every range

struct GemmArgs {
  const uint16_t *A;
  const uint16_t *B;
  void *C;
  const void *bias;
  int64_t sab, sa_outer;
  int64_t sbb, sb_outer;
  int64_t scb, scm;
  uint32_t a_bytes, b_bytes;  // byte extent of one batch slice of A / B
  int M, N, K;
  int tiles_m, tiles_n, batch;
  int out_dt, bias_dt, epi;
  int round;  // workgroups resident at once (one per CU), or 0: see round_tile_of
};

template <int DT>
__device__ __forceinline__ f32x16 mfma_32x32x16(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (DT == NOVA_HIP_DT_BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(
        __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

// Raw buffer over `bytes` bytes at p: loads at offsets >= bytes return zero
// without touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const uint16_t *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(p), (short)0, (int)bytes,
                                           0x00020000);
}

__device__ __forceinline__ float bias_at(const void *bias, int dt, int n) {
  if (dt == NOVA_HIP_DT_F32) return static_cast<const float *>(bias)[n];
  const uint16_t h = static_cast<const uint16_t *>(bias)[n];
  if (dt == NOVA_HIP_DT_BF16) return __uint_as_float(static_cast<uint32_t>(h) << 16);
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// gelu(x) = 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), in the operation
// order of NovaGeluForwardPattern (NovaToLinalgGeneric.cpp:1310-1331).
__device__ __forceinline__ float gelu_tanh(float x) {
#pragma clang fp contract(off)
  const float x2 = x * x;
  const float x3 = x2 * x;
  const float cubic = 4.471500e-02f * x3;
  const float inner = x + cubic;
  const float scaled = 0.7978845608028654f * inner;
  const float t = tanhf(scaled);
  return (0.5f * x) * (1.0f + t);
}

// The same GELU (NovaToLinalgGeneric.cpp:1310-1331) for the GEMM epilogues,
// in the equivalent sigmoid form 0.5 x (1 + tanh s) = x / (1 + e^(-2s)),
// s = sqrt(2/pi) (x + 0.044715 x^3): -2s log2(e) = x (k1 + k2 x^2), then
// the hardware exp2 and reciprocal.  Five VALU operations and two
// transcendentals instead of twelve and two (the epilogue is where config 3
// spends its GELU time); limits: x / inf = -0 for x << 0, x for x >> 0.
// Against the f64 formula: abs error <= 5.2e-7, rel error <= 9e-7 where
// |gelu| > 1e-3 (x in [-12, 12]); bf16 rounding is 3.9e-3.
__device__ __forceinline__ float gelu_tanh_fast(float x) {
  constexpr float k1 = -2.3022082f;   // -2 sqrt(2/pi) log2(e)
  constexpr float k2 = -0.10294324f;  // k1 * 0.044715
  const float u = x * __builtin_fmaf(k2, x * x, k1);
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(u));
}

// f32 -> bf16 / f16, round to nearest even (NaN stays NaN), on gfx950's
// conversion instructions (v_cvt_pk_bf16_f32, v_cvt_pk_f16_f32): branch-free,
// and two values per instruction in the packed forms (a in the low half).
typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint16_t to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
__device__ __forceinline__ uint16_t to_f16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2v{a, b}, bf16x2v));
}
__device__ __forceinline__ uint32_t pack_f16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2v{a, b}, f16x2v));
}

// Map a linear tile index to (batch, tile_m, tile_n), wave-uniform: within
// a batch, consecutive indices sweep a band of 4 tile-rows column by column.
__device__ __forceinline__ void band_tile(int t, const GemmArgs &a, int &b, int &tm, int &tn) {
  const int per_batch = a.tiles_m * a.tiles_n;
  b = t / per_batch;
  t -= b * per_batch;
  constexpr int G = 4;
  const int band = t / (G * a.tiles_n);
  const int first = band * G;
  const int gsz = min(a.tiles_m - first, G);
  const int in_band = t - band * G * a.tiles_n;
  tm = first + in_band % gsz;
  tn = in_band / gsz;
  b = __builtin_amdgcn_readfirstlane(b);
  tm = __builtin_amdgcn_readfirstlane(tm);
  tn = __builtin_amdgcn_readfirstlane(tn);
}

// Workgroup id -> tile for kernels with several workgroups per CU: the
// hardware hands consecutive workgroup ids to the 8 XCDs round robin, so
// renumber to give each XCD one contiguous range of tiles (its own L2 sees
// neighbouring tiles).
__device__ __forceinline__ void tile_of(int id, const GemmArgs &a, int &b, int &tm, int &tn) {
  const int total = a.batch * a.tiles_m * a.tiles_n;
  if ((total & 7) == 0) {
    const int per_xcd = total >> 3;
    id = (id & 7) * per_xcd + (id >> 3);
  }
  band_tile(id, a, b, tm, tn);
}

// Workgroup id -> tile for kernels with one workgroup per CU, which run in
// rounds of a.round workgroups (a.round = CU count, a multiple of 8).  In
// each full round, XCD x (ids q = x mod 8 of the round) takes the round's
// tiles [x*round/8, (x+1)*round/8): all eight XCDs work on neighbouring
// tiles of the same band sweep, so an operand panel one XCD fetches from HBM
// is found in the MALL by the XCDs that share it, and each XCD's 32 tiles
// form a 4 x 8 block whose panels its L2 shares.  A last, partial round of
// rem tiles gets the same treatment when rem is a multiple of 8 (XCD x takes
// [x*rem/8, (x+1)*rem/8) of it); otherwise it keeps the identity order.
__device__ __forceinline__ void round_tile_of(int id, const GemmArgs &a, int &b, int &tm, int &tn) {
  const int total = a.batch * a.tiles_m * a.tiles_n;
  const int round = a.round;
  if (round > 0) {
    const int full = total / round * round;
    if (id < full) {
      const int r = id / round, q = id - r * round;
      id = r * round + (q & 7) * (round >> 3) + (q >> 3);
    } else if (((total - full) & 7) == 0) {
      const int q = id - full;
      id = full + (q & 7) * ((total - full) >> 3) + (q >> 3);
    }
  }
  band_tile(id, a, b, tm, tn);
}

// Epilogue for a wave's TM x TN grid of 32x32 accumulator tiles whose
// top-left output is (mw, nw) in batch bidx.  Accumulator element v of lane
// l sits at row 8*(v/4) + 4*(l/32) + v%4, column l%32 of its tile; a store
// instruction writes 32 consecutive columns of two rows.  Bounds-checked
// (edge tiles), specialised on output dtype and epilogue.  NT: f32 stores
// with the nontemporal hint, for callers whose store instructions write
// whole 128-byte lines (with partial lines the hint costs time).  It is a
// template parameter: behind a runtime branch the compiler merges the two
// stores into one and drops the hint.
template <int TM, int TN, int ODT, int EPI, bool NT = false>
__device__ __forceinline__ void store_outputs_t(const f32x16 (&acc)[TM][TN], const GemmArgs &a,
                                                int bidx, int mw, int nw, int lane) {
  constexpr bool kBias = (EPI == NOVA_HIP_EPI_BIAS || EPI == NOVA_HIP_EPI_BIAS_GELU);
  constexpr bool kGelu = (EPI == NOVA_HIP_EPI_BIAS_GELU || EPI == NOVA_HIP_EPI_GELU);
  const int lrow = lane & 31, lhalf = lane >> 5;
  typedef typename std::conditional<ODT == NOVA_HIP_DT_F32, float, uint16_t>::type T;
  T *Cb = static_cast<T *>(a.C) + (int64_t)bidx * a.scb;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = nw + j * 32 + lrow;
    const bool n_ok = n < a.N;
    const float bv = (kBias && n_ok) ? bias_at(a.bias, a.bias_dt, n) : 0.0f;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = mw + i * 32 + 8 * (v >> 2) + 4 * lhalf + (v & 3);
        float x = acc[i][j][v];
        if constexpr (kBias) x = x + bv;
        if constexpr (kGelu) x = gelu_tanh(x);
        if (n_ok && m < a.M) {
          T *dst = Cb + (int64_t)m * a.scm + n;
          if constexpr (ODT == NOVA_HIP_DT_F32) {
            if constexpr (NT) __builtin_nontemporal_store(x, dst);
            else *dst = x;
          }
          else if constexpr (ODT == NOVA_HIP_DT_BF16) *dst = to_bf16(x);
          else *dst = to_f16(x);
        }
      }
    }
  }
}

// The same with the output dtype and epilogue decided per element: smaller
// code, used for large per-wave grids (4 x 4 tiles), where the specialised
// form runs out of registers.
template <int TM, int TN>
__device__ __forceinline__ void store_outputs_any(const f32x16 (&acc)[TM][TN], const GemmArgs &a,
                                                  int bidx, int mw, int nw, int lane) {
  const int lrow = lane & 31, lhalf = lane >> 5;
  char *Cb = static_cast<char *>(a.C) +
             (int64_t)bidx * a.scb * (a.out_dt == NOVA_HIP_DT_F32 ? 4 : 2);
  const bool has_bias = (a.epi == NOVA_HIP_EPI_BIAS || a.epi == NOVA_HIP_EPI_BIAS_GELU);
  const bool has_gelu = (a.epi == NOVA_HIP_EPI_BIAS_GELU || a.epi == NOVA_HIP_EPI_GELU);
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = nw + j * 32 + lrow;
    if (n >= a.N) continue;
    const float bv = has_bias ? bias_at(a.bias, a.bias_dt, n) : 0.0f;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = mw + i * 32 + 8 * (v >> 2) + 4 * lhalf + (v & 3);
        if (m >= a.M) continue;
        float x = acc[i][j][v];
        if (has_bias) x = x + bv;
        if (has_gelu) x = gelu_tanh(x);
        const int64_t off = (int64_t)m * a.scm + n;
        if (a.out_dt == NOVA_HIP_DT_F32)
          reinterpret_cast<float *>(Cb)[off] = x;
        else if (a.out_dt == NOVA_HIP_DT_BF16)
          reinterpret_cast<uint16_t *>(Cb)[off] = to_bf16(x);
        else
          reinterpret_cast<uint16_t *>(Cb)[off] = to_f16(x);
      }
    }
  }
}

// Runtime (output dtype, epilogue) -> one specialisation of store_outputs_t
// (grids of up to 4 tiles per wave).
template <int TM, int TN, bool NT = false>
__device__ __forceinline__ void store_outputs(const f32x16 (&acc)[TM][TN], const GemmArgs &a,
                                              int bidx, int mw, int nw, int lane) {
  if constexpr (TM * TN > 4) {
    store_outputs_any<TM, TN>(acc, a, bidx, mw, nw, lane);
    return;
  }
  switch (a.out_dt * 4 + a.epi) {
#define NOVA_EPI_CASE(O, E) \
  case O * 4 + E:           \
    store_outputs_t<TM, TN, O, E, NT>(acc, a, bidx, mw, nw, lane); \
    break;
    NOVA_EPI_CASE(0, 0) NOVA_EPI_CASE(0, 1) NOVA_EPI_CASE(0, 2) NOVA_EPI_CASE(0, 3)
    NOVA_EPI_CASE(1, 0) NOVA_EPI_CASE(1, 1) NOVA_EPI_CASE(1, 2) NOVA_EPI_CASE(1, 3)
    NOVA_EPI_CASE(2, 0) NOVA_EPI_CASE(2, 1) NOVA_EPI_CASE(2, 2) NOVA_EPI_CASE(2, 3)
#undef NOVA_EPI_CASE
    default:
      break;
  }
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

}  // namespace gemm

// Launchers (host).  launch_gemm_dma returns NOVA_HIP_EDTYPE when the
// problem is not one the DMA kernel addresses (the caller then uses the
// register-staged kernel).
bool gemm_dma_applicable(const gemm::GemmArgs &a, bool akc, bool bkc, bool vec);
int32_t launch_gemm_dma(const gemm::GemmArgs &a, int in_dt, bool akc, bool bkc, hipStream_t s);
// Per output dtype (gemm_dma_out_{f32,bf16,f16}.hip, compiled separately).
int32_t launch_gemm_dma_f32out(const gemm::GemmArgs &a, int in_dt, bool akc, bool bkc,
                               hipStream_t s);
int32_t launch_gemm_dma_bf16out(const gemm::GemmArgs &a, int in_dt, bool akc, bool bkc,
                                hipStream_t s);
int32_t launch_gemm_dma_f16out(const gemm::GemmArgs &a, int in_dt, bool akc, bool bkc,
                               hipStream_t s);
// Small-K kernel (gemm_small.hip): whole K staged in LDS per output tile.
bool gemm_small_applicable(const gemm::GemmArgs &a, bool akc, bool bkc);
int32_t launch_gemm_small(const gemm::GemmArgs &a, int in_dt, bool akc, bool bkc, hipStream_t s);

}  // namespace nova_hip
