// MFMA GEMM / batch GEMM for gfx950: bf16 or f16 inputs, f32 accumulate,
// f32 / bf16 / f16 output, optional bias and GELU(tanh) epilogue.
//
// Replaces the NVPTX code generation of nova-gpu-optimized-pipeline for
// linalg.matmul / linalg.batch_matmul (lib/Transforms/LLVMGPU/Passes.cpp:
// 115-372: tile+distribute, pad, promote to shared memory, mma.sync,
// 3-stage cp.async).  Designed for CDNA4 instead:
//   * macro-tile BM x BN x 64, four wave64s in a 2x2 grid, each wave owning
//     (BM/2) x (BN/2) of the output as 32x32 v_mfma_f32_32x32x16_{bf16,f16}
//     tiles held in accumulation registers;
//   * operands staged through LDS, two stages (double buffer): global loads
//     of stage k+1 are in flight while stage k feeds the MFMAs;
//   * LDS holds both operands K-contiguous ([rows][64] per stage) with the
//     16-byte chunk index XOR-swizzled by (row & 7), so the ds_read_b128 of
//     eight consecutive rows and the ds_write_b128 of one row's eight chunks
//     hit distinct banks;
//   * an operand whose unit stride is on M or N (B of a row-major [K,N]
//     matrix, A of a transposed view) is fetched as 8x8 blocks and
//     transposed in registers before the LDS write;
//   * edge tiles (M, N, K not multiples of the tile) are zero-padded at
//     load time and masked at store time -- the role of NovaGPUPadOperands;
//   * workgroups are renumbered so the 1/8 of the grid that the hardware
//     dispatches to one XCD is one contiguous, tile-row-grouped range (its
//     own L2 then serves the operand re-reads).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "nova_hip_internal.h"

namespace nova_hip {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kBK = 64;        // K per LDS stage
constexpr int kThreads = 256;  // four wave64s

struct GemmArgs {
  const uint16_t *A;
  const uint16_t *B;
  void *C;
  const void *bias;
  int64_t sab, sa_outer;
  int64_t sbb, sb_outer;
  int64_t scb, scm;
  int M, N, K;
  int tiles_m, tiles_n, batch;
  int out_dt, bias_dt, epi;
};

template <int DT>
__device__ __forceinline__ f32x16 mfma_32x32x16(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (DT == NOVA_HIP_DT_BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
        0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(
        __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
        0);
  }
}

// LDS chunk slot of (row, 16-byte chunk c) inside one operand stage.
__device__ __forceinline__ int lds_slot(int row, int c) {
  return row * 8 + (c ^ (row & 7));
}

// ---------------------------------------------------------------------------
// Tile loaders.  An operand tile is R rows (M for A, N for B) x 64 k.
//   KC  : the operand's unit stride is on K.
//   VEC : 16-byte global loads are legal (aligned base, outer stride % 8 == 0,
//         K % 8 == 0 for KC; rows % 8 == 0 for !KC).  Otherwise elements are
//         fetched one by one.
// Registers: NREG chunks per thread.
// ---------------------------------------------------------------------------
template <int R, bool KC>
struct TileShape {
  // KC: R*8 chunks over 256 threads.  !KC: R/8*8 blocks of 8x8, one block
  // (8 chunks) per participating thread.
  static constexpr int kBlocks = KC ? 0 : (R / 8) * 8;
  static constexpr int kBlockIters = KC ? 0 : (kBlocks + kThreads - 1) / kThreads;
  static constexpr int NREG = KC ? (R * 8) / kThreads : 8 * kBlockIters;
};

template <int R, bool KC, bool VEC>
__device__ __forceinline__ void load_tile(u32x4 *reg, const uint16_t *base,
                                          int64_t s_outer, int row0, int rows,
                                          int k0, int K, int tid) {
  if constexpr (KC) {
#pragma unroll
    for (int i = 0; i < TileShape<R, KC>::NREG; ++i) {
      const int q = tid + i * kThreads;
      const int r = q >> 3, c = q & 7;
      const int gr = row0 + r, gk = k0 + c * 8;
      if constexpr (VEC) {
        u32x4 v = {0u, 0u, 0u, 0u};
        if (gr < rows && gk < K)
          v = *reinterpret_cast<const u32x4 *>(base + (int64_t)gr * s_outer + gk);
        reg[i] = v;
      } else {
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          uint32_t lo = 0, hi = 0;
          if (gr < rows) {
            const uint16_t *p = base + (int64_t)gr * s_outer;
            if (gk + 2 * e < K) lo = p[gk + 2 * e];
            if (gk + 2 * e + 1 < K) hi = p[gk + 2 * e + 1];
          }
          w[e] = lo | (hi << 16);
        }
        reg[i] = u32x4{w[0], w[1], w[2], w[3]};
      }
    }
  } else {
    // 8x8 blocks: block q -> (rb = q / 8 row-block, kb = q % 8 k-block);
    // chunk j of the block holds k-row (kb*8 + j), rows rb*8 .. rb*8+7.
#pragma unroll
    for (int it = 0; it < TileShape<R, KC>::kBlockIters; ++it) {
      const int q = tid + it * kThreads;
      const int kb = q & 7, rb = q >> 3;
      const int gr = row0 + rb * 8;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int gk = k0 + kb * 8 + j;
        if constexpr (VEC) {
          u32x4 v = {0u, 0u, 0u, 0u};
          if (q < TileShape<R, KC>::kBlocks && gk < K && gr < rows)
            v = *reinterpret_cast<const u32x4 *>(base + (int64_t)gk * s_outer + gr);
          reg[it * 8 + j] = v;
        } else {
          uint32_t w[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            uint32_t lo = 0, hi = 0;
            if (q < TileShape<R, KC>::kBlocks && gk < K) {
              const uint16_t *p = base + (int64_t)gk * s_outer;
              if (gr + 2 * e < rows) lo = p[gr + 2 * e];
              if (gr + 2 * e + 1 < rows) hi = p[gr + 2 * e + 1];
            }
            w[e] = lo | (hi << 16);
          }
          reg[it * 8 + j] = u32x4{w[0], w[1], w[2], w[3]};
        }
      }
    }
  }
}

template <int R, bool KC>
__device__ __forceinline__ void store_tile(u32x4 *lds, const u32x4 *reg,
                                           int tid) {
  if constexpr (KC) {
#pragma unroll
    for (int i = 0; i < TileShape<R, KC>::NREG; ++i) {
      const int q = tid + i * kThreads;
      lds[lds_slot(q >> 3, q & 7)] = reg[i];
    }
  } else {
#pragma unroll
    for (int it = 0; it < TileShape<R, KC>::kBlockIters; ++it) {
      const int q = tid + it * kThreads;
      if (q >= TileShape<R, KC>::kBlocks) break;
      const int kb = q & 7, rb = q >> 3;
      const u32x4 *in = reg + it * 8;  // in[j]: k-row j, 8 values along rows
      // Transpose: output row r (0..7) gathers element r of each k-row.
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int d = r >> 1;
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t x = in[2 * e][d], y = in[2 * e + 1][d];
          w[e] = (r & 1) ? ((x >> 16) | (y & 0xffff0000u))
                         : ((x & 0xffffu) | (y << 16));
        }
        lds[lds_slot(rb * 8 + r, kb)] = u32x4{w[0], w[1], w[2], w[3]};
      }
    }
  }
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

__device__ __forceinline__ uint16_t to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ uint16_t to_f16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Map the linear workgroup id to (batch, tile_m, tile_n).
__device__ __forceinline__ void tile_of(int id, const GemmArgs &a, int &b,
                                        int &tm, int &tn) {
  const int total = a.batch * a.tiles_m * a.tiles_n;
  // Hardware hands consecutive workgroup ids to the 8 XCDs round robin;
  // renumber so each XCD sees one contiguous range of tiles.
  if ((total & 7) == 0) {
    const int per_xcd = total >> 3;
    id = (id & 7) * per_xcd + (id >> 3);
  }
  const int per_batch = a.tiles_m * a.tiles_n;
  b = id / per_batch;
  int t = id - b * per_batch;
  // Group 4 tile-rows: consecutive ids sweep a 4-row band column by column.
  constexpr int G = 4;
  const int band = t / (G * a.tiles_n);
  const int first = band * G;
  const int gsz = min(a.tiles_m - first, G);
  const int in_band = t - band * G * a.tiles_n;
  tm = first + in_band % gsz;
  tn = in_band / gsz;
}

template <int DT, int BM, int BN, bool AKC, bool BKC, bool VEC>
__global__ __launch_bounds__(kThreads) void gemm_mfma_kernel(GemmArgs a) {
  constexpr int WTM = BM / 2, WTN = BN / 2;  // wave tile
  constexpr int TM = WTM / 32, TN = WTN / 32;
  using SA = TileShape<BM, AKC>;
  using SB = TileShape<BN, BKC>;

  __shared__ u32x4 lds_a[2][BM * 8];
  __shared__ u32x4 lds_b[2][BN * 8];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  int bidx, tm, tn;
  tile_of(blockIdx.x, a, bidx, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;

  const uint16_t *Ab = a.A + (int64_t)bidx * a.sab;
  const uint16_t *Bb = a.B + (int64_t)bidx * a.sbb;

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  u32x4 ra[SA::NREG];
  u32x4 rb[SB::NREG];

  const int nk = (a.K + kBK - 1) / kBK;
  load_tile<BM, AKC, VEC>(ra, Ab, a.sa_outer, m0, a.M, 0, a.K, tid);
  load_tile<BN, BKC, VEC>(rb, Bb, a.sb_outer, n0, a.N, 0, a.K, tid);
  store_tile<BM, AKC>(lds_a[0], ra, tid);
  store_tile<BN, BKC>(lds_b[0], rb, tid);
  __syncthreads();

  const int lrow = lane & 31;   // row (A) / column (B) inside a 32-tile
  const int lhalf = lane >> 5;  // which 8-wide k half of a 16-k step

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) {
      load_tile<BM, AKC, VEC>(ra, Ab, a.sa_outer, m0, a.M, (kt + 1) * kBK, a.K, tid);
      load_tile<BN, BKC, VEC>(rb, Bb, a.sb_outer, n0, a.N, (kt + 1) * kBK, a.K, tid);
    }
    const u32x4 *sa = lds_a[cur];
    const u32x4 *sb = lds_b[cur];
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      const int chunk = kk * 2 + lhalf;
      u32x4 fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[i] = sa[lds_slot(wm * WTM + i * 32 + lrow, chunk)];
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[j] = sb[lds_slot(wn * WTN + j * 32 + lrow, chunk)];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma_32x32x16<DT>(fa[i], fb[j], acc[i][j]);
    }
    if (kt + 1 < nk) {
      store_tile<BM, AKC>(lds_a[cur ^ 1], ra, tid);
      store_tile<BN, BKC>(lds_b[cur ^ 1], rb, tid);
    }
    __syncthreads();
  }

  // Epilogue.  Accumulator element v of lane l in a 32x32 tile sits at
  // row 8*(v/4) + 4*(l/32) + v%4, column l%32.
  char *Cb = static_cast<char *>(a.C) +
             (int64_t)bidx * a.scb * (a.out_dt == NOVA_HIP_DT_F32 ? 4 : 2);
  const bool has_bias = (a.epi == NOVA_HIP_EPI_BIAS || a.epi == NOVA_HIP_EPI_BIAS_GELU);
  const bool has_gelu = (a.epi == NOVA_HIP_EPI_BIAS_GELU || a.epi == NOVA_HIP_EPI_GELU);
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = n0 + wn * WTN + j * 32 + lrow;
    if (n >= a.N) continue;
    const float bv = has_bias ? bias_at(a.bias, a.bias_dt, n) : 0.0f;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + wm * WTM + i * 32 + 8 * (v >> 2) + 4 * lhalf + (v & 3);
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

template <int DT, int BM, int BN, bool AKC, bool BKC, bool VEC>
int32_t launch_cfg(const GemmArgs &a, hipStream_t s) {
  const int64_t total = (int64_t)a.batch * a.tiles_m * a.tiles_n;
  if (total > 0x7fffffff) return fail(NOVA_HIP_ERANGE, "gemm: grid too large");
  hipLaunchKernelGGL((gemm_mfma_kernel<DT, BM, BN, AKC, BKC, VEC>),
                     dim3((unsigned)total), dim3(kThreads), 0, s, a);
  return check_hip(hipGetLastError(), "gemm_mfma launch");
}

template <int DT, int BM, int BN, bool VEC>
int32_t dispatch_layout(const GemmArgs &a, bool akc, bool bkc, hipStream_t s) {
  if (akc && bkc) return launch_cfg<DT, BM, BN, true, true, VEC>(a, s);
  if (akc && !bkc) return launch_cfg<DT, BM, BN, true, false, VEC>(a, s);
  if (!akc && bkc) return launch_cfg<DT, BM, BN, false, true, VEC>(a, s);
  return launch_cfg<DT, BM, BN, false, false, VEC>(a, s);
}

template <int DT>
int32_t dispatch_dtype(const GemmArgs &a, bool akc, bool bkc, bool big, bool vec,
                       hipStream_t s) {
  if (big) return dispatch_layout<DT, 256, 256, true>(a, akc, bkc, s);
  if (vec) return dispatch_layout<DT, 64, 64, true>(a, akc, bkc, s);
  return dispatch_layout<DT, 64, 64, false>(a, akc, bkc, s);
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

int32_t launch_gemm_mfma(const GemmProblem &p, hipStream_t s) {
  if (p.batch == 0 || p.M == 0 || p.N == 0) return NOVA_HIP_SUCCESS;
  if (p.M > 0x7fffffff || p.N > 0x7fffffff || p.K > 0x7fffffff)
    return fail(NOVA_HIP_ERANGE, "gemm: dimension exceeds 2^31-1");

  GemmArgs a;
  a.A = static_cast<const uint16_t *>(p.A);
  a.B = static_cast<const uint16_t *>(p.B);
  a.C = p.C;
  a.bias = p.bias;
  a.sab = p.sab;
  a.sa_outer = p.sa_outer;
  a.sbb = p.sbb;
  a.sb_outer = p.sb_outer;
  a.scb = p.scb;
  a.scm = p.scm;
  a.M = (int)p.M;
  a.N = (int)p.N;
  a.K = (int)p.K;
  a.batch = (int)p.batch;
  a.out_dt = p.out_dt;
  a.bias_dt = p.bias_dt;
  a.epi = p.epi;

  // 16-byte global loads need aligned bases, outer strides that keep every
  // row aligned, and whole 8-element chunks along the contiguous dim.
  bool vec = aligned16(p.A) && aligned16(p.B) && (p.sa_outer % 8 == 0) &&
             (p.sb_outer % 8 == 0) && (p.sab % 8 == 0) && (p.sbb % 8 == 0);
  vec = vec && (p.a_kcontig ? (p.K % 8 == 0) : (p.M % 8 == 0));
  vec = vec && (p.b_kcontig ? (p.K % 8 == 0) : (p.N % 8 == 0));

  // Tile choice: 256x256 when the grid still fills the chip, else 64x64.
  const int64_t big_tiles = p.batch * ((p.M + 255) / 256) * ((p.N + 255) / 256);
  const bool big = vec && big_tiles >= 256;
  const int BMs = big ? 256 : 64;
  a.tiles_m = (int)((p.M + BMs - 1) / BMs);
  a.tiles_n = (int)((p.N + BMs - 1) / BMs);

  if (p.in_dt == NOVA_HIP_DT_BF16)
    return dispatch_dtype<NOVA_HIP_DT_BF16>(a, p.a_kcontig, p.b_kcontig, big, vec, s);
  return dispatch_dtype<NOVA_HIP_DT_F16>(a, p.a_kcontig, p.b_kcontig, big, vec, s);
}

}  // namespace nova_hip
