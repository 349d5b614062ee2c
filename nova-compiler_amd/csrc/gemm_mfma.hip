// MFMA GEMM / batch GEMM for gfx950: bf16 or f16 inputs, f32 accumulate,
// f32 / bf16 / f16 output, optional bias and GELU(tanh) epilogue.
//
// Replaces the NVPTX code generation of nova-gpu-optimized-pipeline for
// linalg.matmul / linalg.batch_matmul (lib/Transforms/LLVMGPU/Passes.cpp:
// 115-372: tile+distribute, pad, promote to shared memory, mma.sync,
// 3-stage cp.async).  Two kernels, chosen per problem by launch_gemm_mfma:
//
//  * gemm_dma.hip -- aligned problems made of whole 256x256x32 tiles (the
//    large configs): operands go global -> LDS by DMA, four stages deep.
//  * this file -- every other shape: register-staged loads, two LDS stages.
//    Macro-tile BM x BN x 64, four wave64s in a 2x2 grid, each owning
//    (BM/2) x (BN/2) of the output as 32x32 v_mfma_f32_32x32x16 tiles.
//    LDS holds both operands K-contiguous ([rows][64] per stage) with the
//    16-byte chunk index XOR-swizzled by row, so the ds_read_b128 of
//    consecutive rows and the ds_write_b128 of one row's eight chunks hit
//    distinct banks.  An operand whose unit stride is on M or N is
//    fetched as 8x8 blocks and transposed in registers before the LDS
//    write.  Edge tiles are zero-padded at load time (buffer loads outside
//    the operand's range return zero) and masked at store time -- the role
//    of NovaGPUPadOperands.
#include "gemm_common.h"

namespace nova_hip {
namespace {

using namespace gemm;

constexpr int kBK = 64;  // K per LDS stage

// LDS chunk slot of (row, 16-byte chunk c) inside one operand stage.  The
// XOR by (row ^ row/8) keeps both 8 and 16 consecutive rows of a
// ds_read_b128 on distinct banks (LDS serving 8 or 16 lanes per cycle).
__device__ __forceinline__ int lds_slot(int row, int c) {
  return row * 8 + (c ^ ((row ^ (row >> 3)) & 7));
}

// ---------------------------------------------------------------------------
// Tile loaders.  An operand tile is R rows (M for A, N for B) x 64 k, read
// through a buffer resource whose range covers the operand's batch slice:
// any load outside it (edge rows, k past K, whole tiles past the end of the
// K loop) returns zeros without touching memory, so edges need no branches.
//   KC  : the operand's unit stride is on K.
//   VEC : 16-byte loads are legal (16-byte aligned rows and chunks).
//         Otherwise elements are fetched one by one (2-byte buffer loads).
// ---------------------------------------------------------------------------
template <int R, bool KC>
struct TileShape {
  // KC: R*8 chunks over 256 threads.  !KC: R blocks of 8x8, one block
  // (8 chunks) per participating thread.
  static constexpr int kBlocks = KC ? 0 : R;
  static constexpr int kBlockIters = KC ? 0 : (kBlocks + kThreads - 1) / kThreads;
  static constexpr int NREG = KC ? (R * 8) / kThreads : 8 * kBlockIters;
};

struct Operand {
  __amdgpu_buffer_rsrc_t rsrc;
  int64_t s_outer;  // elements
  int row0, rows, K;
};

__device__ __forceinline__ u32x4 load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

__device__ __forceinline__ uint32_t load2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

template <int R, bool KC, bool VEC>
__device__ __forceinline__ void load_tile(u32x4 *reg, const Operand &o, int k0, int tid) {
  if constexpr (KC) {
#pragma unroll
    for (int i = 0; i < TileShape<R, KC>::NREG; ++i) {
      const int q = tid + i * kThreads;
      const int r = q >> 3, c = q & 7;
      const int gr = o.row0 + r, gk = k0 + c * 8;
      const uint32_t base = (uint32_t)(((int64_t)gr * o.s_outer + gk) * 2);
      if constexpr (VEC) {
        reg[i] = load16(o.rsrc, (gr < o.rows && gk < o.K) ? base : kOOB);
      } else {
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool rok = gr < o.rows;
          const uint32_t lo = load2(o.rsrc, (rok && gk + 2 * e < o.K) ? base + 4 * e : kOOB);
          const uint32_t hi = load2(o.rsrc, (rok && gk + 2 * e + 1 < o.K) ? base + 4 * e + 2 : kOOB);
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
      const int gr = o.row0 + rb * 8;
      const bool qok = q < TileShape<R, KC>::kBlocks;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int gk = k0 + kb * 8 + j;
        const uint32_t base = (uint32_t)(((int64_t)gk * o.s_outer + gr) * 2);
        if constexpr (VEC) {
          reg[it * 8 + j] = load16(o.rsrc, (qok && gk < o.K && gr < o.rows) ? base : kOOB);
        } else {
          uint32_t w[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const bool kok = qok && gk < o.K;
            const uint32_t lo = load2(o.rsrc, (kok && gr + 2 * e < o.rows) ? base + 4 * e : kOOB);
            const uint32_t hi = load2(o.rsrc, (kok && gr + 2 * e + 1 < o.rows) ? base + 4 * e + 2 : kOOB);
            w[e] = lo | (hi << 16);
          }
          reg[it * 8 + j] = u32x4{w[0], w[1], w[2], w[3]};
        }
      }
    }
  }
}

template <int R, bool KC>
__device__ __forceinline__ void store_tile(u32x4 *lds, const u32x4 *reg, int tid) {
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
          w[e] = (r & 1) ? ((x >> 16) | (y & 0xffff0000u)) : ((x & 0xffffu) | (y << 16));
        }
        lds[lds_slot(rb * 8 + r, kb)] = u32x4{w[0], w[1], w[2], w[3]};
      }
    }
  }
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

  Operand oa, ob;
  oa.rsrc = make_rsrc(a.A + (int64_t)bidx * a.sab, a.a_bytes);
  oa.s_outer = a.sa_outer;
  oa.row0 = m0;
  oa.rows = a.M;
  oa.K = a.K;
  ob.rsrc = make_rsrc(a.B + (int64_t)bidx * a.sbb, a.b_bytes);
  ob.s_outer = a.sb_outer;
  ob.row0 = n0;
  ob.rows = a.N;
  ob.K = a.K;

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  const int lrow = lane & 31;   // row (A) / column (B) inside a 32-tile
  const int lhalf = lane >> 5;  // which 8-wide k half of a 16-k step

  // One LDS stage through the MFMAs; fragments of step kk+1 are read while
  // the MFMAs of step kk run.  The scheduling barriers keep that order: left
  // alone, the scheduler sinks reads next to their first use to save
  // registers and exposes the LDS latency at every step.
  auto compute = [&](const u32x4 *sa, const u32x4 *sb) __attribute__((always_inline)) {
    u32x4 fa[2][TM], fb[2][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) fa[0][i] = sa[lds_slot(wm * WTM + i * 32 + lrow, lhalf)];
#pragma unroll
    for (int j = 0; j < TN; ++j) fb[0][j] = sb[lds_slot(wn * WTN + j * 32 + lrow, lhalf)];
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      const int cb = kk & 1, nb = cb ^ 1;
      if (kk + 1 < kBK / 16) {
        const int chunk = (kk + 1) * 2 + lhalf;
#pragma unroll
        for (int i = 0; i < TM; ++i) fa[nb][i] = sa[lds_slot(wm * WTM + i * 32 + lrow, chunk)];
#pragma unroll
        for (int j = 0; j < TN; ++j) fb[nb][j] = sb[lds_slot(wn * WTN + j * 32 + lrow, chunk)];
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma_32x32x16<DT>(fa[cb][i], fb[cb][j], acc[i][j]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // The global loads of tile t+1 are issued before the MFMAs of tile t and
  // written to the other LDS stage after them.  Loads past the last tile
  // fall outside the buffer range and return zeros, so the loop body is
  // unconditional.
  u32x4 ra[SA::NREG], rb[SB::NREG];
  const int nk = (a.K + kBK - 1) / kBK;
  load_tile<BM, AKC, VEC>(ra, oa, 0, tid);
  load_tile<BN, BKC, VEC>(rb, ob, 0, tid);
  store_tile<BM, AKC>(lds_a[0], ra, tid);
  store_tile<BN, BKC>(lds_b[0], rb, tid);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    load_tile<BM, AKC, VEC>(ra, oa, (kt + 1) * kBK, tid);
    load_tile<BN, BKC, VEC>(rb, ob, (kt + 1) * kBK, tid);
    __builtin_amdgcn_sched_barrier(0);
    compute(lds_a[cur], lds_b[cur]);
    store_tile<BM, AKC>(lds_a[cur ^ 1], ra, tid);
    store_tile<BN, BKC>(lds_b[cur ^ 1], rb, tid);
    __syncthreads();
  }

  store_outputs<TM, TN>(acc, a, bidx, m0 + wm * WTM, n0 + wn * WTN, lane);
}

template <int DT, int BM, int BN, bool AKC, bool BKC, bool VEC>
int32_t launch_cfg(const GemmArgs &a, hipStream_t s) {
  const int64_t total = (int64_t)a.batch * a.tiles_m * a.tiles_n;
  if (total > 0x7fffffff) return fail(NOVA_HIP_ERANGE, "gemm: grid too large");
  hipLaunchKernelGGL((gemm_mfma_kernel<DT, BM, BN, AKC, BKC, VEC>), dim3((unsigned)total),
                     dim3(kThreads), 0, s, a);
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
int32_t dispatch_dtype(const GemmArgs &a, bool akc, bool bkc, bool big, bool vec, hipStream_t s) {
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
  a.round = 0;

  // Byte extent of one batch slice of each operand: the buffer range the
  // kernel's loads are checked against.  Buffer offsets are 32-bit.
  const int64_t a_ext = p.a_kcontig ? (p.M - 1) * p.sa_outer + p.K : (p.K - 1) * p.sa_outer + p.M;
  const int64_t b_ext = p.b_kcontig ? (p.N - 1) * p.sb_outer + p.K : (p.K - 1) * p.sb_outer + p.N;
  if (a_ext * 2 > 0x7fffffff || b_ext * 2 > 0x7fffffff)
    return fail(NOVA_HIP_ERANGE, "gemm: an operand's batch slice exceeds 2 GiB");
  a.a_bytes = p.K > 0 ? (uint32_t)(a_ext * 2) : 0u;
  a.b_bytes = p.K > 0 ? (uint32_t)(b_ext * 2) : 0u;

  // 16-byte global loads need aligned bases, outer strides that keep every
  // row aligned, and whole 8-element chunks along the contiguous dim.
  bool vec = aligned16(p.A) && aligned16(p.B) && (p.sa_outer % 8 == 0) &&
             (p.sb_outer % 8 == 0) && (p.sab % 8 == 0) && (p.sbb % 8 == 0);
  vec = vec && (p.a_kcontig ? (p.K % 8 == 0) : (p.M % 8 == 0));
  vec = vec && (p.b_kcontig ? (p.K % 8 == 0) : (p.N % 8 == 0));

  if (gemm_dma_applicable(a, p.a_kcontig, p.b_kcontig, vec))
    return launch_gemm_dma(a, p.in_dt, p.a_kcontig, p.b_kcontig, s);
  // Rows without 16-byte alignment would cost the tiled kernel 2-byte loads;
  // with a small K the staged kernel copies them whole instead.
  if (!vec && gemm_small_applicable(a, p.a_kcontig, p.b_kcontig))
    return launch_gemm_small(a, p.in_dt, p.a_kcontig, p.b_kcontig, s);

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
