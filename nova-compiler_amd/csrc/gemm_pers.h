// Persistent form of the LDS-DMA GEMM (gemm_dma.h), with or without a bias /
// GELU epilogue: one workgroup per CU computes its output tiles one after
// another, so the DMA of the next tile's first two K steps is in
// flight while the current tile's epilogue runs, and no workgroup is
// dispatched, set up or retired between rounds.
//
// Workgroup g of G takes tiles g, g + G, g + 2G, ... in round_tile_of
// order (G = a.round, one per CU), i.e. the same tile -> CU assignment as
// the one-tile-per-workgroup kernel.  The K loop, LDS ring and swizzles are
// those of gemm_dma_kernel.  Differences:
//   * each DMA offset is a lane part (fixed) plus a wave-uniform tile and
//     K part, so the loads can target the next tile;
//   * the last K step of a tile issues all of the next tile's second K step
//     (both halves) before the epilogue, so the first K step after the
//     epilogue waits for the DMA with vmcnt(#stores) while the epilogue
//     stores (the youngest memory operations) may still be in flight;
//   * the epilogue stages through its own 16 KB of LDS (4 KB per wave), not
//     the ring, which holds the next tile's data; the tile's bias goes to
//     LDS as f32, double-buffered by tile parity.  146 KB of LDS in all.
#pragma once
#include <type_traits>

#include "gemm_dma.h"

namespace nova_hip {
namespace pers {

using namespace gemm;
using namespace dma;

// Tile-independent part of each DMA byte offset of this lane: load i of
// wave w fills slots [(i*4 + w) * 64, +64) of a stage, as in dma_setup.
template <bool KC>
__device__ __forceinline__ void lane_offsets(uint32_t (&off)[kLoads], int64_t s_outer, int wave,
                                             int lane) {
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    const int s = (i * 4 + wave) * 64 + lane;
    int64_t e;
    if constexpr (KC) {
      const int row = s / kChunks, c = (s % kChunks) ^ kc_swz(s / kChunks);
      e = (int64_t)row * s_outer + c * 8;
    } else {
      const int k = s >> 5, c16 = (s & 31) ^ mn_swz(s >> 5);
      e = (int64_t)k * s_outer + c16 * 8;
    }
    off[i] = (uint32_t)(e * 2);
  }
}

// An output tile: batch and first row / column (wave-uniform).
struct Tile {
  int bidx, m0, n0;
};

__device__ __forceinline__ Tile tile_at(const GemmArgs &a, int ti) {
  int b, tm, tn;
  round_tile_of(blockIdx.x + ti * gridDim.x, a, b, tm, tn);
  return Tile{b, tm * BM, tn * BN};
}

// DMA load q (q < kLoads: A, else B) of K tile kt of tile t; nothing is read
// (the offset is out of range) when !live.
template <bool AKC, bool BKC>
__device__ __forceinline__ void dma_issue(const GemmArgs &a, const uint32_t (&la)[kLoads],
                                          const uint32_t (&lb)[kLoads], u32x4 *sa, u32x4 *sb,
                                          int q, const Tile &t, int kt, bool live, int wave) {
  if (q < kLoads) {
    const uint32_t base =
        AKC ? (uint32_t)((int64_t)t.m0 * a.sa_outer * 2) + (uint32_t)(kt * BK * 2)
            : (uint32_t)(t.m0 * 2) + (uint32_t)((int64_t)kt * BK * a.sa_outer * 2);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        make_rsrc(a.A + (int64_t)t.bidx * a.sab, a.a_bytes),
        (lds_void *)(sa + (q * 4 + wave) * 64), 16, live ? la[q] + base : kOOB, 0, 0, 0);
  } else {
    const int r = q - kLoads;
    const uint32_t base =
        BKC ? (uint32_t)((int64_t)t.n0 * a.sb_outer * 2) + (uint32_t)(kt * BK * 2)
            : (uint32_t)(t.n0 * 2) + (uint32_t)((int64_t)kt * BK * a.sb_outer * 2);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        make_rsrc(a.B + (int64_t)t.bidx * a.sbb, a.b_bytes),
        (lds_void *)(sb + (r * 4 + wave) * 64), 16, live ? lb[r] + base : kOOB, 0, 0, 0);
  }
}

// Global store instructions of one wave's epilogue (the wait after it).
template <int ODT>
constexpr int kEpiStores = ODT == NOVA_HIP_DT_F32 ? 64 : 32;

// Epilogue of a wave's 128x128 output tile through its own 4 KB of LDS, in
// rounds of 32 rows x 128 bytes (f32: one 32-column block, 16-bit: two), so
// that every global store instruction writes eight rows x 128 B, i.e. whole
// 128-byte lines.  16-byte chunk c of staging row R sits at c ^ (R & 7),
// conflict-free for the column-wise writes and the row-wise reads.  Bias
// (f32, staged in LDS for the tile's 256 columns) and GELU are applied on
// the way.  The staging accesses are plain C++ on arrays of their own: the
// compiler then stores the accumulation registers to LDS directly where no
// arithmetic intervenes, and as they are not the DMA ring it places no DMA
// wait before them.
template <int ODT>
__device__ __forceinline__ void store_tile(const f32x16 (&acc)[TM][TN], const GemmArgs &a,
                                           int bidx, int mw, int nw, int lane, char *stg,
                                           const float *bias_w) {
  const bool has_bias = (a.epi == NOVA_HIP_EPI_BIAS || a.epi == NOVA_HIP_EPI_BIAS_GELU);
  const bool has_gelu = (a.epi == NOVA_HIP_EPI_BIAS_GELU || a.epi == NOVA_HIP_EPI_GELU);
  // Lane-derived addresses are recomputed per tile: an opaque copy of the
  // lane id keeps the compiler from hoisting them out of the tile loop,
  // where they would stay live across the K loop.
  int ln = lane;
  asm volatile("" : "+v"(ln));
  const int lr = ln & 31, lh = ln >> 5;
  constexpr bool kF32 = ODT == NOVA_HIP_DT_F32;
  constexpr int kEsz = kF32 ? 4 : 2;
  constexpr int kJ = kF32 ? 1 : 2;   // 32-column blocks per round
  constexpr int kJR = TN / kJ;       // rounds per 32-row block
  char *Cb = static_cast<char *>(a.C) + (int64_t)bidx * a.scb * kEsz;
#pragma unroll
  for (int jr = 0; jr < kJR; ++jr) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int jj = 0; jj < kJ; ++jj)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int j = jr * kJ + jj;
          f32x4 x = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                     acc[i][j][4 * g + 3]};
          if (has_bias) x = x + *reinterpret_cast<const f32x4 *>(bias_w + 32 * j + 8 * g + 4 * lh);
          if (has_gelu) {
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = gelu_tanh_fast(x[e]);
          }
          const int R = lr;
          if constexpr (kF32) {
            const int c = 2 * g + lh;
            *reinterpret_cast<f32x4 *>(stg + R * 128 + ((c ^ (R & 7)) << 4)) = x;
          } else {
            const int c = 4 * jj + g;
            const u32x2 w = ODT == NOVA_HIP_DT_BF16
                                ? u32x2{pack_bf16(x[0], x[1]), pack_bf16(x[2], x[3])}
                                : u32x2{pack_f16(x[0], x[1]), pack_f16(x[2], x[3])};
            *reinterpret_cast<u32x2 *>(stg + R * 128 + ((c ^ (R & 7)) << 4) + 8 * lh) = w;
          }
        }
      u32x4 v[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int R = 8 * t + (ln >> 3), c = ln & 7;
        v[t] = *reinterpret_cast<const u32x4 *>(stg + R * 128 + ((c ^ (R & 7)) << 4));
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int R = 8 * t + (ln >> 3), c = ln & 7;
        char *dst = Cb + ((int64_t)(mw + 32 * i + R) * a.scm + nw + 32 * kJ * jr) * kEsz + 16 * c;
        *reinterpret_cast<u32x4 *>(dst) = v[t];
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// Launch: gridDim.x <= number of tiles, a.K / BK >= 2.
template <int DT, bool AKC, bool BKC, int ODT>
__global__ __launch_bounds__(kThreads) void gemm_pers_kernel(GemmArgs a) {
  __shared__ u32x4 ring_a[kStages][kSlots];
  __shared__ u32x4 ring_b[kStages][kSlots];
  __shared__ u32x4 stage_out[4][256];  // 4 KB per wave
  // The bias of the tile's 256 columns as f32, double-buffered by tile
  // parity: a tile's bias is written at its start while the previous tile's
  // epilogue may still read the other buffer.
  __shared__ __attribute__((aligned(16))) float bias_s[2][BN];
  static_assert(sizeof(ring_a) + sizeof(ring_b) + sizeof(stage_out) + sizeof(bias_s) <=
                    160 * 1024,
                "LDS");
  const bool has_bias = (a.epi == NOVA_HIP_EPI_BIAS || a.epi == NOVA_HIP_EPI_BIAS_GELU);
  static_assert(kThreads == BN, "one bias column per thread");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int am = wm * 128, bn = wn * 128;

  const int total = a.batch * a.tiles_m * a.tiles_n;
  const int ntiles = (total - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
  const int nk = a.K / BK;

  uint32_t la[kLoads], lb[kLoads];
  lane_offsets<AKC>(la, a.sa_outer, wave, lane);
  lane_offsets<BKC>(lb, a.sb_outer, wave, lane);

  f32x16 acc[TM][TN];
  constexpr int kSteps = BK / 16;
  constexpr int kFrags = TM + TN;
  static_assert(kSpread == 2 && kPerStep == kLoads && kPerStep * 2 == TM * TN,
                "one DMA load per MFMA: A's in the last k16 step, B's in the first two");
  u32x4 fa[2][TM], fb[2][TN];

  // Every fragment read's byte offset from its stage base, computed once:
  // only the stage changes between K steps, so each read costs one add
  // (computed per read, the swizzled addresses took ~100 VALU instructions
  // per K step beside the 64 MFMAs, now 64; config 2 0.898 -> 0.885 ms and
  // config 3 ~1% faster in A/B runs in both orders, the same bits).
  uint32_t fofs[kSteps][kFrags];
#pragma unroll
  for (int kk = 0; kk < kSteps; ++kk)
#pragma unroll
    for (int f = 0; f < kFrags; ++f)
      fofs[kk][f] = f < TM ? frag_ofs<AKC>(am + f * 32, kk, lane)
                           : frag_ofs<BKC>(bn + (f - TM) * 32, kk, lane);
  // (Every lambda here must inline: a call would force acc into memory.)
  auto read_one = [&](int f, int buf, const u32x4 *A, const u32x4 *B, int kk)
                      __attribute__((always_inline)) {
    if (f < TM) fa[buf][f] = read_frag_at<AKC>(lds_addr(A) + fofs[kk][f]);
    else fb[buf][f - TM] = read_frag_at<BKC>(lds_addr(B) + fofs[kk][f]);
  };
  auto mfma_one = [&](int m, int buf) __attribute__((always_inline)) {
    const int i = m / TN, j = m % TN;
    acc[i][j] = mfma_32x32x16<DT>(fb[buf][j], fa[buf][i], acc[i][j]);
  };
  auto dma = [&](int q, u32x4 *sa, u32x4 *sb, const Tile &t, int kt, bool live)
                 __attribute__((always_inline)) {
    dma_issue<AKC, BKC>(a, la, lb, sa, sb, q, t, kt, live, wave);
  };

  Tile tc = tile_at(a, 0);  // the tile being computed
  Tile tn = tc;             // the next one
  bool tn_live = ntiles > 1;
  if (tn_live) tn = tile_at(a, 1);

  // Prologue: K steps 0 and 1 of the first tile in flight, step 0 landed,
  // its first fragments read.
#pragma unroll
  for (int q = 0; q < 2 * kLoads; ++q) dma(q, ring_a[0], ring_b[0], tc, 0, true);
#pragma unroll
  for (int q = 0; q < 2 * kLoads; ++q) dma(q, ring_a[1], ring_b[1], tc, 1, true);
  NOVA_WAIT_VMCNT(2 * kLoads);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int f = 0; f < kFrags; ++f) read_one(f, 0, ring_a[0], ring_b[0], 0);
  __builtin_amdgcn_sched_barrier(0);

  int cur = 0;
  // K step kt of the current tile, as in gemm_dma_kernel.  KIND 0: the
  // tile's first, whose successor was issued whole before (after an
  // epilogue, ahead of its stores); 1: a middle one; 2: the last, which
  // issues all of the next tile's second K step (the next tile's first
  // fragments are read after the epilogue).
  auto kstep = [&](auto kind, int kt, int ti) __attribute__((always_inline)) {
    constexpr int KIND = decltype(kind)::value;
    u32x4 *A = ring_a[cur], *B = ring_b[cur];
    const int nxt = cur ^ 1;
    NOVA_WAIT_LGKMCNT0();
    __builtin_amdgcn_sched_barrier(0);
    // The next K step's B loads go out half in k16 step 0 and half in k16
    // step 1, beside that step's fragment reads: all eight in step 0 made
    // a burst that ran 0.6-3.4% slower depending on the box (C2, in-process
    // A/B, same bits); in step 2 they no longer land in time (3% slower).
    constexpr int kHalf = kPerStep / 2;
#pragma unroll
    for (int m = 0; m < TM * TN; ++m) {
      mfma_one(m, 0);
      if (m < kFrags) read_one(m, 1, A, B, 1);
      if (KIND == 1 && m < kHalf)
        dma(kPerStep + m, ring_a[nxt], ring_b[nxt], tc, kt + 1, true);
      if (KIND == 2 && m < kHalf) dma(kPerStep + m, ring_a[nxt], ring_b[nxt], tn, 0, tn_live);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int s = 1; s < kSteps - 1; ++s) {
      NOVA_WAIT_LGKMCNT0();
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int m = 0; m < TM * TN; ++m) {
        mfma_one(m, s & 1);
        if (m < kFrags) read_one(m, (s + 1) & 1, A, B, s + 1);
        if (s == 1 && KIND == 1 && m < kPerStep - kHalf)
          dma(kPerStep + kHalf + m, ring_a[nxt], ring_b[nxt], tc, kt + 1, true);
        if (s == 1 && KIND == 2 && m < kPerStep - kHalf)
          dma(kPerStep + kHalf + m, ring_a[nxt], ring_b[nxt], tn, 0, tn_live);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // The next K step has landed for this wave (after a tile's epilogue only
    // its stores, issued later, may still be in flight: memory operations
    // retire in issue order for vmcnt); after the barrier, for every wave,
    // and this K step's stage is free.
    NOVA_WAIT_LGKMCNT0();
    if (KIND == 0 && ti > 0) {
      NOVA_WAIT_VMCNT(kEpiStores<ODT> < 63 ? kEpiStores<ODT> : 63);
    } else {
      NOVA_WAIT_VMCNT(0);
    }
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (KIND != 2) {
      // Portion 0 of the K step after next: this tile's, or the next tile's
      // first when this is the second to last.
      const bool in_tile = kt + 2 < nk;
      const Tile t2 = in_tile ? tc : tn;
      const int kt2 = in_tile ? kt + 2 : kt + 2 - nk;
      const bool live2 = in_tile || tn_live;
#pragma unroll
      for (int m = 0; m < TM * TN; ++m) {
        mfma_one(m, (kSteps - 1) & 1);
        if (m < kFrags) read_one(m, 0, ring_a[nxt], ring_b[nxt], 0);
        if (m < kPerStep) dma(m, A, B, t2, kt2, live2);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int m = 0; m < TM * TN; ++m) {
        mfma_one(m, (kSteps - 1) & 1);
        dma(m, A, B, tn, 1, tn_live);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    cur = nxt;
  };

  char *stg = reinterpret_cast<char *>(stage_out[wave]);
  for (int ti = 0; ti < ntiles; ++ti) {
    // This tile's bias, read by its epilogue (after the K loop's barriers).
    if (has_bias) bias_s[ti & 1][tid] = bias_at(a.bias, a.bias_dt, tc.n0 + tid);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
    kstep(std::integral_constant<int, 0>{}, 0, ti);
    for (int kt = 1; kt < nk - 1; ++kt) kstep(std::integral_constant<int, 1>{}, kt, ti);
    kstep(std::integral_constant<int, 2>{}, nk - 1, ti);
    store_tile<ODT>(acc, a, tc.bidx, tc.m0 + am, tc.n0 + bn, lane, stg, bias_s[ti & 1] + bn);
    tc = tn;
    tn_live = ti + 2 < ntiles;
    if (tn_live) tn = tile_at(a, ti + 2);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < kFrags; ++q) read_one(q, 0, ring_a[cur], ring_b[cur], 0);
    __builtin_amdgcn_sched_barrier(0);
  }
  // No DMA may still target this workgroup's LDS when it retires.
  NOVA_WAIT_VMCNT(0);
  NOVA_WAIT_LGKMCNT0();
}

template <int DT, bool AKC, bool BKC, int ODT>
int32_t launch(const GemmArgs &a, hipStream_t s) {
  const int total = a.batch * a.tiles_m * a.tiles_n;
  const int grid = total < a.round ? total : a.round;
  hipLaunchKernelGGL((gemm_pers_kernel<DT, AKC, BKC, ODT>), dim3((unsigned)grid), dim3(kThreads),
                     0, s, a);
  return check_hip(hipGetLastError(), "gemm_pers launch");
}

// The persistent kernel's problems: two K steps or more, a round size (one
// workgroup per CU) and at least one full round of tiles.
inline bool applicable(const GemmArgs &a) {
  return a.K / BK >= 2 && a.round > 0 &&
         (int64_t)a.batch * a.tiles_m * a.tiles_n >= a.round;
}

template <int ODT>
int32_t launch_out(const GemmArgs &a, int in_dt, bool akc, bool bkc, hipStream_t s) {
  if (in_dt == NOVA_HIP_DT_BF16) {
    if (akc && bkc) return launch<NOVA_HIP_DT_BF16, true, true, ODT>(a, s);
    if (akc) return launch<NOVA_HIP_DT_BF16, true, false, ODT>(a, s);
    if (bkc) return launch<NOVA_HIP_DT_BF16, false, true, ODT>(a, s);
    return launch<NOVA_HIP_DT_BF16, false, false, ODT>(a, s);
  }
  if (akc && bkc) return launch<NOVA_HIP_DT_F16, true, true, ODT>(a, s);
  if (akc) return launch<NOVA_HIP_DT_F16, true, false, ODT>(a, s);
  if (bkc) return launch<NOVA_HIP_DT_F16, false, true, ODT>(a, s);
  return launch<NOVA_HIP_DT_F16, false, false, ODT>(a, s);
}

}  // namespace pers
}  // namespace nova_hip
