// MFMA GEMM for aligned problems made of whole 256x256x32 tiles (the large
// configs: batch GEMM 8x4096^3, linear 4096x4096x11008).
//
// Operands travel global -> LDS with buffer_load ... lds (LDS DMA): no
// staging registers, so the K loop can keep three tiles in flight in a
// four-stage LDS ring (4 x 32 KB).  Each stage holds
//   * a K-contiguous operand as [256 rows][4 chunks of 8 k], 16-byte chunk
//     index XOR-swizzled by row so the ds_read_b128 of 16 consecutive rows
//     covers all banks;
//   * an M/N-contiguous operand (row-major [K,N] B, or a transposed A) as
//     [32 k][32 chunks of 8 rows], chunk index XOR ((k & 3) << 1), read
//     with ds_read_b64_tr_b16, which transposes 16-bit data across each
//     16-lane group (lane i gets element i of four rows); an XOR by k keeps
//     the rows read together on distinct banks.
// A DMA instruction writes 64 lanes x 16 bytes contiguously, so the
// swizzle is applied by choosing, per lane, which global chunk to fetch.
//
// Four wave64s in a 2x2 grid each own 128x128 of the output as 4x4 tiles of
// v_mfma_f32_32x32x16 (256 accumulation registers), issued with B as the
// first operand so each lane accumulates four consecutive output columns
// and the epilogue writes them with one vector store.  Per K step (tile t):
//   read fragments of k16-step 1 | MFMAs of step 0 | wait for this wave's
//   DMA of tile t+1, barrier | DMA of tile t+4 into the freed stage |
//   read tile t+1's first fragments | MFMAs of step 1.
// so LDS latency is never exposed at a stage boundary and global latency
// has three tiles (~3000 MFMA cycles) to land.
#include "gemm_common.h"

namespace nova_hip {
namespace {

using namespace gemm;

constexpr int BM = 256, BN = 256, BK = 32;
constexpr int kSlots = 1024;  // 16-byte slots per operand per stage (16 KB)
constexpr int TM = 4, TN = 4;  // 32x32 tiles per wave (128 x 128)

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// Swizzles, conflict-free whether the LDS serves 8 (32 banks) or 16 (64
// banks) lanes of a ds_read_b128 per cycle, and 16 or 32 lanes of a
// ds_read_b64_tr_b16:
//   K-contiguous: chunk c of row r at c ^ ((r/2 ^ r/4) & 3)
//   M/N-contiguous: 16-byte chunk c of k-row k at c ^ (2(k&3) ^ 4(k&3))
__device__ __forceinline__ int kc_slot(int row, int c) {
  return row * 4 + (c ^ (((row >> 1) ^ (row >> 2)) & 3));
}
__device__ __forceinline__ int mn_slot(int k, int c16) {
  return k * 32 + (c16 ^ (((k & 3) << 1) ^ ((k & 3) << 2)));
}

// sched_group_barrier instruction classes.
constexpr int kSchedMfma = 0x008, kSchedVmemRead = 0x020, kSchedDsRead = 0x100;

// vmcnt(n) with expcnt and lgkmcnt left free (gfx9 encoding).
#define NOVA_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt((((n) & 15) | (((n) >> 4) << 14)) | 0x0F70)

// Scheduling pattern: spread NMEM memory instructions (the first NREADS are
// LDS reads, the rest DMA loads) evenly over the first NSLOT of NMFMA MFMAs,
// one scheduling group each, then leave the remaining MFMAs in one group.
template <int M, int HI, int NREADS, int SYNC>
__device__ __forceinline__ void sched_mem() {
  if constexpr (M < HI) {
    __builtin_amdgcn_sched_group_barrier(M < NREADS ? kSchedDsRead : kSchedVmemRead, 1, SYNC);
    sched_mem<M + 1, HI, NREADS, SYNC>();
  }
}
template <int I, int NSLOT, int NMFMA, int NMEM, int NREADS, int SYNC>
__device__ __forceinline__ void sched_interleave() {
  if constexpr (I < NSLOT) {
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, SYNC);
    sched_mem<I * NMEM / NSLOT, (I + 1) * NMEM / NSLOT, NREADS, SYNC>();
    sched_interleave<I + 1, NSLOT, NMFMA, NMEM, NREADS, SYNC>();
  } else if constexpr (NMFMA > NSLOT) {
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, NMFMA - NSLOT, SYNC);
  }
}

struct DmaOperand {
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t off[4];   // this lane's byte offset for each of its 4 DMA loads, k0 = 0
  uint32_t k_step;   // bytes to advance one K tile
};

// Per-lane source offsets: wave w's load i fills slots [(i*4 + w) * 64, +64).
template <bool KC>
__device__ __forceinline__ void dma_setup(DmaOperand &o, int64_t s_outer, int row0, int wave,
                                          int lane) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int s = (i * 4 + wave) * 64 + lane;
    int64_t e;
    // Slot s holds the chunk that kc_slot / mn_slot place there (the XOR
    // swizzle is its own inverse).
    if constexpr (KC) {
      const int row = s >> 2, c = (s & 3) ^ (((row >> 1) ^ (row >> 2)) & 3);
      e = (int64_t)(row0 + row) * s_outer + c * 8;
    } else {
      const int k = s >> 5, c16 = (s & 31) ^ (((k & 3) << 1) ^ ((k & 3) << 2));
      e = (int64_t)k * s_outer + row0 + c16 * 8;
    }
    o.off[i] = (uint32_t)(e * 2);
  }
  o.k_step = KC ? (uint32_t)(BK * 2) : (uint32_t)(BK * s_outer * 2);
}

// Issue the 4 DMA loads of K tile kt into `stage` (kt past the end: the
// offsets fall outside the buffer range and nothing is read).
__device__ __forceinline__ void dma_issue(const DmaOperand &o, u32x4 *stage, int kt, int nk,
                                          int wave) {
  const bool live = kt < nk;
  const uint32_t add = (uint32_t)kt * o.k_step;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        o.rsrc, (lds_void *)(stage + (i * 4 + wave) * 64), 16, live ? o.off[i] + add : kOOB, 0, 0,
        0);
  }
}

// Fragment of a 32-row block for k16-step kk.
template <bool KC>
__device__ __forceinline__ u32x4 read_frag(const u32x4 *stage, int row_base, int kk, int lane) {
  if constexpr (KC) {
    const int row = row_base + (lane & 31);
    return stage[kc_slot(row, kk * 2 + (lane >> 5))];
  } else {
    const int g = lane >> 4, p = lane & 15;
    const int n = row_base + 16 * (g & 1) + 4 * (p & 3);
    const int kb = kk * 16 + 8 * (g >> 1) + (p >> 2);
    const uint16_t *base = reinterpret_cast<const uint16_t *>(stage);
    const int e0 = mn_slot(kb, n >> 3) * 8 + (n & 7);
    const int e1 = mn_slot(kb + 4, n >> 3) * 8 + (n & 7);
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(base + e0));
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(base + e1));
    const uint32_t w0 = (uint16_t)lo[0] | ((uint32_t)(uint16_t)lo[1] << 16);
    const uint32_t w1 = (uint16_t)lo[2] | ((uint32_t)(uint16_t)lo[3] << 16);
    const uint32_t w2 = (uint16_t)hi[0] | ((uint32_t)(uint16_t)hi[1] << 16);
    const uint32_t w3 = (uint16_t)hi[2] | ((uint32_t)(uint16_t)hi[3] << 16);
    return u32x4{w0, w1, w2, w3};
  }
}

template <int DT, bool AKC, bool BKC>
__global__ __launch_bounds__(kThreads) void gemm_dma_kernel(GemmArgs a) {
  __shared__ u32x4 sa0[kSlots], sa1[kSlots], sa2[kSlots], sa3[kSlots];
  __shared__ u32x4 sb0[kSlots], sb1[kSlots], sb2[kSlots], sb3[kSlots];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  int bidx, tm, tn;
  tile_of(blockIdx.x, a, bidx, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;

  DmaOperand oa, ob;
  oa.rsrc = make_rsrc(a.A + (int64_t)bidx * a.sab, a.a_bytes);
  ob.rsrc = make_rsrc(a.B + (int64_t)bidx * a.sbb, a.b_bytes);
  dma_setup<AKC>(oa, a.sa_outer, m0, wave, lane);
  dma_setup<BKC>(ob, a.sb_outer, n0, wave, lane);

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  const int nk = a.K / BK;
  const int am = wm * 128, bn = wn * 128;
  // LDS read instructions per read_all: one per K-contiguous fragment, two
  // (transposing reads) per M/N-contiguous one.
  constexpr int kReads = (AKC ? TM : 2 * TM) + (BKC ? TN : 2 * TN);

  u32x4 fa0[TM], fb0[TN], fa1[TM], fb1[TN];

  auto read_all = [&](u32x4 (&fa)[TM], u32x4 (&fb)[TN], const u32x4 *A, const u32x4 *B,
                      int kk) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < TM; ++i) fa[i] = read_frag<AKC>(A, am + i * 32, kk, lane);
#pragma unroll
    for (int j = 0; j < TN; ++j) fb[j] = read_frag<BKC>(B, bn + j * 32, kk, lane);
  };
  auto mfma_all = [&](const u32x4 (&fa)[TM], const u32x4 (&fb)[TN]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = mfma_32x32x16<DT>(fb[j], fa[i], acc[i][j]);
  };

  // Prologue: tiles 0..3 in flight, tile 0 landed, its first fragments read.
  dma_issue(oa, sa0, 0, nk, wave);
  dma_issue(ob, sb0, 0, nk, wave);
  dma_issue(oa, sa1, 1, nk, wave);
  dma_issue(ob, sb1, 1, nk, wave);
  dma_issue(oa, sa2, 2, nk, wave);
  dma_issue(ob, sb2, 2, nk, wave);
  dma_issue(oa, sa3, 3, nk, wave);
  dma_issue(ob, sb3, 3, nk, wave);
  NOVA_WAIT_VMCNT(24);
  __syncthreads();
  read_all(fa0, fb0, sa0, sb0, 0);

  // One K step on stage (A, B); (NA, NB) is the next stage.
  // (Every lambda here must inline: a call would force acc into memory.)
  auto step = [&](const u32x4 *A, const u32x4 *B, u32x4 *FA, u32x4 *FB, const u32x4 *NA,
                  const u32x4 *NB, int t) __attribute__((always_inline)) {
    // Fragment reads of k16-step 1 slotted between the first MFMAs of step 0
    // (early, so they have landed by the barrier).
    read_all(fa1, fb1, A, B, 1);
    mfma_all(fa0, fb0);
    sched_interleave<0, 8, TM * TN, kReads, kReads, 0>();
    __builtin_amdgcn_sched_barrier(0);
    NOVA_WAIT_VMCNT(16);  // this wave's DMA of tile t+1 has landed
    __syncthreads();      // ... everyone's has, and nobody reads tile t any more
    // Next stage's first fragments, then the DMA of tile t+4, each slotted
    // between MFMAs of step 1 so the matrix pipe never waits on issue.
    read_all(fa0, fb0, NA, NB, 0);
    dma_issue(oa, FA, t + 4, nk, wave);
    dma_issue(ob, FB, t + 4, nk, wave);
    mfma_all(fa1, fb1);
    sched_interleave<0, 12, TM * TN, kReads + 8, kReads, 1>();
    __builtin_amdgcn_sched_barrier(0);
  };

  // nk is a multiple of 4 (K % 128 == 0): one exit, so the accumulators
  // keep a single register assignment through the loop.
  for (int t = 0; t < nk; t += 4) {
    step(sa0, sb0, sa0, sb0, sa1, sb1, t);
    step(sa1, sb1, sa1, sb1, sa2, sb2, t + 1);
    step(sa2, sb2, sa2, sb2, sa3, sb3, t + 2);
    step(sa3, sb3, sa3, sb3, sa0, sb0, t + 3);
  }
  // No DMA may still target this workgroup's LDS when it retires.
  NOVA_WAIT_VMCNT(0);

  store_full<TM, TN>(acc, a, bidx, m0 + am, n0 + bn, lane);
}

template <int DT, bool AKC, bool BKC>
int32_t launch(const GemmArgs &a, hipStream_t s) {
  hipLaunchKernelGGL((gemm_dma_kernel<DT, AKC, BKC>),
                     dim3((unsigned)(a.batch * a.tiles_m * a.tiles_n)), dim3(kThreads), 0, s, a);
  return check_hip(hipGetLastError(), "gemm_dma launch");
}

template <int DT>
int32_t launch_layout(const GemmArgs &a, bool akc, bool bkc, hipStream_t s) {
  if (akc && bkc) return launch<DT, true, true>(a, s);
  if (akc && !bkc) return launch<DT, true, false>(a, s);
  if (!akc && bkc) return launch<DT, false, true>(a, s);
  return launch<DT, false, false>(a, s);
}

}  // namespace

bool gemm_dma_applicable(const gemm::GemmArgs &a, bool akc, bool bkc, bool vec) {
  (void)akc;
  (void)bkc;
  const int64_t tiles = (int64_t)a.batch * (a.M / BM) * (a.N / BN);
  // Full tiles only, and vector stores need 16-byte aligned output rows.
  const bool c_ok = (reinterpret_cast<uintptr_t>(a.C) & 15u) == 0 && a.scm % 8 == 0 &&
                    a.scb % 8 == 0;
  return vec && c_ok && a.M % BM == 0 && a.N % BN == 0 && a.K % (4 * BK) == 0 && a.K > 0 &&
         tiles >= 128 && tiles <= 0x7fffffff;
}

int32_t launch_gemm_dma(const gemm::GemmArgs &a_in, int in_dt, bool akc, bool bkc, hipStream_t s) {
  gemm::GemmArgs a = a_in;
  a.tiles_m = a.M / BM;
  a.tiles_n = a.N / BN;
  if (in_dt == NOVA_HIP_DT_BF16) return launch_layout<NOVA_HIP_DT_BF16>(a, akc, bkc, s);
  return launch_layout<NOVA_HIP_DT_F16>(a, akc, bkc, s);
}

}  // namespace nova_hip
