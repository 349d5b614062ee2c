// MFMA GEMM for aligned problems made of whole 256x256 tiles (the large
// configs: batch GEMM 8x4096^3, linear 4096x4096x11008).
//
// Operands travel global -> LDS with buffer_load ... lds (LDS DMA): no
// staging registers.  K is consumed in steps of BK = 64 so that every
// K-contiguous row segment a DMA instruction fetches is one whole 128-byte
// line (with BK = 32 the L2 served twice the requests for the same bytes
// and ran 93% busy at half the needed rate).  Two LDS stages of 64 KB: the
// DMA of tile t+1 runs under the MFMAs of tile t.  Each stage holds
//   * a K-contiguous operand as [256 rows][8 chunks of 8 k], 16-byte chunk
//     index XOR-swizzled by row so the ds_read_b128 of 16 consecutive rows
//     covers all banks;
//   * an M/N-contiguous operand (row-major [K,N] B, or a transposed A) as
//     [64 k][32 chunks of 8 rows], read with ds_read_b64_tr_b16, which
//     transposes 16-bit data across each 16-lane group (lane i gets element
//     i of four rows); an XOR by k keeps the rows read together on distinct
//     banks.
// A DMA instruction writes 64 lanes x 16 bytes contiguously, so the
// swizzle is applied by choosing, per lane, which global chunk to fetch.
//
// Four wave64s in a 2x2 grid each own 128x128 of the output as 4x4 tiles of
// v_mfma_f32_32x32x16 (256 accumulation registers), issued with B as the
// first operand so each lane accumulates four consecutive output columns
// and the epilogue writes them with one vector store.  Per K step (tile t,
// four k16 steps): the fragments of k16-step s+1 are read while the MFMAs
// of step s run; after step 2 the wave waits for its DMA of tile t+1, one
// barrier, then the DMA of tile t+2 goes into the freed stage while tile
// t+1's first fragments are read under the MFMAs of step 3.
#pragma once

#include "gemm_common.h"

namespace nova_hip {
namespace dma {

using namespace gemm;

constexpr int BM = 256, BN = 256;
#ifndef NOVA_DMA_BK
#define NOVA_DMA_BK 64
#endif
constexpr int BK = NOVA_DMA_BK;
constexpr int kChunks = BK / 8;              // 16-byte chunks per K-contiguous row
constexpr int kSlots = BM * BK / 8;          // 16-byte slots per operand per stage
constexpr int kLoads = kSlots / kThreads;    // DMA instructions per thread per operand
constexpr int kStages = 2;
// The DMA of a tile is spread over this many k16 steps (see the main loop).
#ifndef NOVA_DMA_SPREAD
#define NOVA_DMA_SPREAD 2
#endif
constexpr int kSpread = NOVA_DMA_SPREAD;
constexpr int kPerStep = (2 * kLoads + kSpread - 1) / kSpread;  // DMA loads per k16 step
constexpr int TM = 4, TN = 4;  // 32x32 tiles per wave (128 x 128)
static_assert(kStages * 2 * kSlots * 16 <= 160 * 1024, "LDS budget");
static_assert(kPerStep <= TM * TN && TM + TN <= TM * TN &&
                  kSpread <= BK / 16,
              "one DMA load and one fragment read per MFMA at most");

typedef __attribute__((address_space(3))) void lds_void;

// vmcnt(n) with expcnt and lgkmcnt left free; lgkmcnt(0) with the others
// free (gfx9 encodings).
#define NOVA_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt((((n) & 15) | (((n) >> 4) << 14)) | 0x0F70)
#define NOVA_WAIT_LGKMCNT0() __builtin_amdgcn_s_waitcnt(0xC07F)

// Swizzles, conflict-free whether the LDS serves 8 or 16 lanes of a
// ds_read_b128 per cycle (16 or 32 lanes of a ds_read_b64_tr_b16):
//   K-contiguous: chunk c of row r at c ^ f(r)
//   M/N-contiguous: 16-byte chunk c of k-row k at c ^ (2(k&3) ^ 4(k&3))
__device__ __forceinline__ int kc_swz(int row) {
  if constexpr (kChunks == 8) return (row ^ (row >> 3)) & 7;
  else return ((row >> 1) ^ (row >> 2)) & 3;
}
__device__ __forceinline__ int kc_slot(int row, int c) { return row * kChunks + (c ^ kc_swz(row)); }
__device__ __forceinline__ int mn_swz(int k) { return ((k & 3) << 1) ^ ((k & 3) << 2); }
__device__ __forceinline__ int mn_slot(int k, int c16) { return k * 32 + (c16 ^ mn_swz(k)); }

struct DmaOperand {
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t off[kLoads];  // this lane's byte offset for each of its DMA loads, k0 = 0
  uint32_t k_step;       // bytes to advance one K tile
};

// Per-lane source offsets: wave w's load i fills slots [(i*4 + w) * 64, +64).
// Slot s holds the chunk kc_slot / mn_slot place there (the XOR swizzle is
// its own inverse).
template <bool KC>
__device__ __forceinline__ void dma_setup(DmaOperand &o, int64_t s_outer, int row0, int wave,
                                          int lane) {
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    const int s = (i * 4 + wave) * 64 + lane;
    int64_t e;
    if constexpr (KC) {
      const int row = s / kChunks, c = (s % kChunks) ^ kc_swz(s / kChunks);
      e = (int64_t)(row0 + row) * s_outer + c * 8;
    } else {
      const int k = s >> 5, c16 = (s & 31) ^ mn_swz(s >> 5);
      e = (int64_t)k * s_outer + row0 + c16 * 8;
    }
    o.off[i] = (uint32_t)(e * 2);
  }
  o.k_step = KC ? (uint32_t)(BK * 2) : (uint32_t)(BK * s_outer * 2);
}

// DMA load q of K tile kt: q < kLoads are A's loads into sa, the rest B's
// into sb (kt past the end: the offset falls outside the buffer range and
// nothing is read).
__device__ __forceinline__ void dma_load(const DmaOperand &oa, const DmaOperand &ob, u32x4 *sa,
                                         u32x4 *sb, int q, int kt, int nk, int wave) {
  const bool live = kt < nk;
  if (q < kLoads)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(oa.rsrc, (lds_void *)(sa + (q * 4 + wave) * 64), 16,
                                             live ? oa.off[q] + (uint32_t)kt * oa.k_step : kOOB, 0,
                                             0, 0);
  else
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        ob.rsrc, (lds_void *)(sb + ((q - kLoads) * 4 + wave) * 64), 16,
        live ? ob.off[q - kLoads] + (uint32_t)kt * ob.k_step : kOOB, 0, 0, 0);
}

// LDS reads as inline assembly.  Written as intrinsics or plain loads, the
// compiler assumes they may read what any in-flight LDS DMA writes and
// drains the DMA queue (vmcnt) before them; it cannot tell the two ring
// stages apart.  As assembly they are invisible to that analysis, and the
// kernel places the lgkmcnt waits for them itself.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const lds_void *)p;
}
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u32x4 lds_read_b128(uint32_t addr) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}
__device__ __forceinline__ u32x2v lds_read_tr(uint32_t addr) {
  u32x2v v;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}

__device__ __forceinline__ u32x2v lds_read_tr_hi(uint32_t addr) {
  u32x2v v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:2048" : "=v"(v) : "v"(addr));
  return v;
}
// Byte offset, from the stage base, of this lane's read of fragment
// row_base for k16-step kk (the second transposing read is 2048 bytes on).
template <bool KC>
__device__ __forceinline__ uint32_t frag_ofs(int row_base, int kk, int lane) {
  if constexpr (KC) {
    const int row = row_base + (lane & 31);
    return (uint32_t)kc_slot(row, kk * 2 + (lane >> 5)) * 16u;
  } else {
    const int g = lane >> 4, p = lane & 15;
    const int n = row_base + 16 * (g & 1) + 4 * (p & 3);
    const int kb = kk * 16 + 8 * (g >> 1) + (p >> 2);
    return (uint32_t)(mn_slot(kb, n >> 3) * 8 + (n & 7)) * 2u;
  }
}
template <bool KC>
__device__ __forceinline__ u32x4 read_frag_at(uint32_t addr) {
  if constexpr (KC) {
    return lds_read_b128(addr);
  } else {
    const u32x2v lo = lds_read_tr(addr);
    const u32x2v hi = lds_read_tr_hi(addr);
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  }
}

// Fragment of a 32-row block for k16-step kk (issued, not yet landed).
template <bool KC>
__device__ __forceinline__ u32x4 read_frag(const u32x4 *stage, int row_base, int kk, int lane) {
  if constexpr (KC) {
    const int row = row_base + (lane & 31);
    return lds_read_b128(lds_addr(stage + kc_slot(row, kk * 2 + (lane >> 5))));
  } else {
    const int g = lane >> 4, p = lane & 15;
    const int n = row_base + 16 * (g & 1) + 4 * (p & 3);
    const int kb = kk * 16 + 8 * (g >> 1) + (p >> 2);
    const uint16_t *base = reinterpret_cast<const uint16_t *>(stage);
    const int e0 = mn_slot(kb, n >> 3) * 8 + (n & 7);
    const int e1 = mn_slot(kb + 4, n >> 3) * 8 + (n & 7);
    const u32x2v lo = lds_read_tr(lds_addr(base + e0));
    const u32x2v hi = lds_read_tr(lds_addr(base + e1));
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  }
}

// Epilogue of a wave's 128x128 output tile, staged through kStageBytes of
// LDS so that every global store instruction writes whole 128-byte lines.
// Stored straight from the accumulators (lane l holding 16 or 8 bytes of
// one row, 32 rows per instruction) the lines were written in 32-byte
// slices, and while the DMA stream cycled the L2 some partly written lines
// were evicted and written back more than once (20-35% more HBM writes than
// the output).  Here the accumulators go to LDS in output layout (bias and
// GELU applied on the way), and are read back as whole row segments: f32 in
// two rounds of 64 rows x 512 B, bf16/f16 in one round of 128 rows x 256 B.
// 16-byte chunk c of LDS row R sits at chunk c ^ (R mod #chunks per row),
// which keeps both the column-wise writes and the row-wise reads free of
// bank conflicts.
constexpr int kStageBytes = 32768;
static_assert(4 * kStageBytes <= kStages * 2 * kSlots * 16, "staging fits the ring");

// The bias of the workgroup's 256 columns is staged to LDS as f32 at kernel
// start (bias_s, nw0 = its first column) and read here with 16-byte LDS
// loads, and the 16-bit conversions are the branch-free hardware ones: with
// a per-element global bias load (behind a switch over the bias dtype) and a
// NaN branch per converted value the compiler split the epilogue into ~1600
// basic blocks whose loads each waited out a memory latency (config 3 spent
// ~90 us of ~400 there).
template <int ODT>
__device__ __forceinline__ void store_staged(const f32x16 (&acc)[TM][TN], const GemmArgs &a,
                                             int bidx, int mw, int nw, int lane, char *stg,
                                             const float *bias_s, int nw0) {
  static_assert(TM == 4 && TN == 4, "staging assumes a 128x128 wave tile");
  const bool has_bias = (a.epi == NOVA_HIP_EPI_BIAS || a.epi == NOVA_HIP_EPI_BIAS_GELU);
  const bool has_gelu = (a.epi == NOVA_HIP_EPI_BIAS_GELU || a.epi == NOVA_HIP_EPI_GELU);
  const int lr = lane & 31, lh = lane >> 5;
  constexpr bool kF32 = ODT == NOVA_HIP_DT_F32;
  constexpr int kRounds = kF32 ? 2 : 1;      // 64 or 128 rows per round
  constexpr int kRowBytes = kF32 ? 512 : 256;
  constexpr int kChunks = kRowBytes / 16;    // 16-byte chunks per LDS row
  constexpr int kEsz = kF32 ? 4 : 2;
  char *Cb = static_cast<char *>(a.C) + (int64_t)bidx * a.scb * kEsz;
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f32x4 bv = {0.f, 0.f, 0.f, 0.f};
        if (has_bias)
          bv = *reinterpret_cast<const f32x4 *>(bias_s + (nw - nw0) + 32 * j + 8 * g + 4 * lh);
#pragma unroll
        for (int ii = 0; ii < TM / kRounds; ++ii) {
          const int i = r * (TM / kRounds) + ii;
          f32x4 x = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                     acc[i][j][4 * g + 3]};
          if (has_bias) x = x + bv;
          if (has_gelu) {
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = gelu_tanh_fast(x[e]);
          }
          const int R = 32 * ii + lr;  // row within the round
          if constexpr (kF32) {
            const int c = 8 * j + 2 * g + lh;
            *reinterpret_cast<f32x4 *>(stg + R * kRowBytes + ((c ^ (R & (kChunks - 1))) << 4)) = x;
          } else {
            const int c = 4 * j + g;
            const u32x2 w = ODT == NOVA_HIP_DT_BF16
                                ? u32x2{pack_bf16(x[0], x[1]), pack_bf16(x[2], x[3])}
                                : u32x2{pack_f16(x[0], x[1]), pack_f16(x[2], x[3])};
            *reinterpret_cast<u32x2 *>(stg + R * kRowBytes + ((c ^ (R & (kChunks - 1))) << 4) +
                                       8 * lh) = w;
          }
        }
      }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes done
    constexpr int kRowsPerInst = 1024 / kRowBytes;  // 64 lanes x 16 bytes
    constexpr int kRoundRows = 128 / kRounds;
#pragma unroll
    for (int t = 0; t < kRoundRows / kRowsPerInst; ++t) {
      const int R = kRowsPerInst * t + lane / kChunks, c = lane % kChunks;
      const u32x4 v = *reinterpret_cast<const u32x4 *>(stg + R * kRowBytes +
                                                       ((c ^ (R & (kChunks - 1))) << 4));
      char *dst = Cb + ((int64_t)(mw + kRoundRows * r + R) * a.scm + nw) * kEsz + 16 * c;
      *reinterpret_cast<u32x4 *>(dst) = v;
    }
    if (r + 1 < kRounds) __builtin_amdgcn_s_waitcnt(0xC07F);  // reads done before the next round
  }
}

template <int DT, bool AKC, bool BKC, int ODT>
__global__ __launch_bounds__(kThreads) void gemm_dma_kernel(GemmArgs a) {
  __shared__ u32x4 ring_a[kStages][kSlots];
  __shared__ u32x4 ring_b[kStages][kSlots];
  __shared__ __attribute__((aligned(16))) float bias_s[BN];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  int bidx, tm, tn;
  round_tile_of(blockIdx.x, a, bidx, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  // The tile's bias as f32 (read by the epilogue after its barrier).
  if ((a.epi == NOVA_HIP_EPI_BIAS || a.epi == NOVA_HIP_EPI_BIAS_GELU) && tid < BN)
    bias_s[tid] = bias_at(a.bias, a.bias_dt, n0 + tid);

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
  constexpr int kSteps = BK / 16;
  constexpr int kFrags = TM + TN;

  u32x4 fa[2][TM], fb[2][TN];

  // (Every lambda here must inline: a call would force acc into memory.)
  auto read_one = [&](int f, int buf, const u32x4 *A, const u32x4 *B, int kk)
                      __attribute__((always_inline)) {
    if (f < TM) fa[buf][f] = read_frag<AKC>(A, am + f * 32, kk, lane);
    else fb[buf][f - TM] = read_frag<BKC>(B, bn + (f - TM) * 32, kk, lane);
  };
  auto mfma_one = [&](int m, int buf) __attribute__((always_inline)) {
    const int i = m / TN, j = m % TN;
    acc[i][j] = mfma_32x32x16<DT>(fb[buf][j], fa[buf][i], acc[i][j]);
  };

  // The DMA of tile t+2 goes into tile t's stage, which is free from tile
  // t's barrier on.  Its 2*kLoads loads are spread over kSpread k16 steps:
  // portion 0 in the last step of tile t (after the barrier), portion p in
  // step p-1 of tile t+1.  All must land before tile t+1's barrier, which
  // waits for them (vmcnt(0)) ahead of the first read of tile t+2.
  auto dma_portion = [&](int p, u32x4 *sa, u32x4 *sb, int kt, int m)
                         __attribute__((always_inline)) {
    if (m < kPerStep && p * kPerStep + m < 2 * kLoads)
      dma_load(oa, ob, sa, sb, p * kPerStep + m, kt, nk, wave);
  };

  // Prologue: tile 0 and portion 0 of tile 1 in flight, tile 0 landed, its
  // first fragments read.
#pragma unroll
  for (int q = 0; q < 2 * kLoads; ++q) dma_load(oa, ob, ring_a[0], ring_b[0], q, 0, nk, wave);
#pragma unroll
  for (int m = 0; m < kPerStep; ++m) dma_portion(0, ring_a[1], ring_b[1], 1, m);
  NOVA_WAIT_VMCNT(kPerStep);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int f = 0; f < kFrags; ++f) read_one(f, 0, ring_a[0], ring_b[0], 0);
  __builtin_amdgcn_sched_barrier(0);

  // Every instruction group below is fenced with sched_barrier(0), so the
  // order written is the order issued: MFMA m of a k16 step, then the
  // fragment read m of the next step, then DMA load m of the step's portion.
  int cur = 0;
  for (int t = 0; t < nk; ++t) {
    u32x4 *A = ring_a[cur], *B = ring_b[cur];
    const int nxt = cur ^ 1;
#pragma unroll
    for (int s = 0; s < kSteps - 1; ++s) {
      NOVA_WAIT_LGKMCNT0();  // fragments of step s
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int m = 0; m < TM * TN; ++m) {
        mfma_one(m, s & 1);
        if (m < kFrags) read_one(m, (s + 1) & 1, A, B, s + 1);
        if (s + 1 < kSpread) dma_portion(s + 1, ring_a[nxt], ring_b[nxt], t + 1, m);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // This wave's fragments of the last step and its DMA of tile t+1 have
    // landed; after the barrier everyone's have, and tile t's stage is free.
    NOVA_WAIT_LGKMCNT0();
    NOVA_WAIT_VMCNT(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    // Last step: tile t+1's first fragments and portion 0 of tile t+2's DMA.
#pragma unroll
    for (int m = 0; m < TM * TN; ++m) {
      mfma_one(m, (kSteps - 1) & 1);
      if (m < kFrags) read_one(m, 0, ring_a[nxt], ring_b[nxt], 0);
      dma_portion(0, A, B, t + 2, m);
      __builtin_amdgcn_sched_barrier(0);
    }
    cur = nxt;
  }
  // No DMA may still target this workgroup's LDS when it retires, and the
  // (unused) fragment reads past the last tile must have landed.
  NOVA_WAIT_VMCNT(0);
  NOVA_WAIT_LGKMCNT0();
  __builtin_amdgcn_sched_barrier(0);

  // Epilogue through LDS (the ring is free once every wave is past its last
  // fragment read).
  __syncthreads();
  char *stg = (wave < 2 ? reinterpret_cast<char *>(ring_a) : reinterpret_cast<char *>(ring_b)) +
              (wave & 1) * kStageBytes;
  store_staged<ODT>(acc, a, bidx, m0 + am, n0 + bn, lane, stg, bias_s, n0);
}

template <int DT, bool AKC, bool BKC, int ODT>
int32_t launch(const GemmArgs &a, hipStream_t s) {
  hipLaunchKernelGGL((gemm_dma_kernel<DT, AKC, BKC, ODT>),
                     dim3((unsigned)(a.batch * a.tiles_m * a.tiles_n)), dim3(kThreads), 0, s, a);
  return check_hip(hipGetLastError(), "gemm_dma launch");
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

}  // namespace dma
}  // namespace nova_hip
