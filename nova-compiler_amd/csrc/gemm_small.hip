// MFMA GEMM for small K (config 4: fp16 96x197x197x64 and 96x197x64x197,
// attention-score shaped).  Such problems move far more output than they
// compute, and their rows are rarely 16-byte aligned (197 fp16 = 394 B), so
// the tiled kernels would fall back to 2-byte loads and several passes.
//
// One workgroup owns a 64 (or 128) x NT output tile of one batch (NT =
// 64..256) and the whole K range.  Both operands are staged into LDS once, normalised:
//   * an operand is a set of "lines", each contiguous in memory -- rows of
//     a K-contiguous operand (A rows / B columns), or k-lines of an M/N-
//     contiguous one;
//   * each thread writes one aligned 16-byte LDS chunk of a line: it loads
//     the two aligned global chunks covering it and funnel-shifts them by the
//     line's misalignment (v_alignbyte), zeroing elements past the line's
//     end; lines past the operand are written as zeros;
//   * the buffer resource starts at the slice base rounded down to 16 bytes
//     and ends at its end rounded up (the rounding never leaves the 16-byte
//     blocks, hence the pages, holding the slice's first and last bytes).
// The LDS layouts are then the ones the MFMA wants: [row][k] read with
// ds_read_b128, or [k][row] read with the transposing ds_read_b64_tr_b16.
// A K-contiguous A with 16-byte aligned rows and K a multiple of 16 (up to
// 64) is not staged: each computing wave loads its A fragments straight from
// memory before the B staging starts (config 4a: 10.4 -> 9.7 us, same bits).
// Eight waves stage (sixteen in a workgroup alone on its CU, so that the
// chunks go out in half the rounds: configs 4a / 4b 8.90 -> 8.62 /
// 7.75 -> 7.36 us, the same bits).  In a 64-row window four of them, in a 2x2 grid, then
// each own 32 rows x NT/2 columns as NT/64 tiles of v_mfma_f32_32x32x16; in
// a 128-row window all eight do, in a 4x2 grid.  The MFMA loops are
// specialised per operand layout and read the next fragments from LDS while
// the current ones multiply; with A read directly and an f32 output each
// 32-column block is stored before the next block multiplies (configs 4a /
// 4b: 9.66 -> 8.94 / 8.75 -> 8.19 us, the same bits).  The epilogue writes
// bounds-checked coalesced stores.
#include <algorithm>

#include "gemm_common.h"

namespace nova_hip {
namespace {

using namespace gemm;

constexpr int kBM = 64;
constexpr int kMaxNT = 256;
constexpr int kLdsBytes = 80 * 1024;    // staging budget per workgroup (two fit a CU)
constexpr int kCuLdsBytes = 160 * 1024;  // a CU's LDS, for a workgroup alone on its CU
// Staging runs on eight waves, the MFMAs and the epilogue on the first four
// (2x2 grid): staging is the long, latency-bound part.  A workgroup alone on
// its CU stages on sixteen (kWideThreads); waves 8-15 only stage.
constexpr int kStageThreads = 512;
constexpr int kWideThreads = 1024;
// Chunks staged per thread per round, for A and for B (two loads each).  A
// wide workgroup whose A is read directly stages B alone, whose at most
// ~2,100 chunks (K <= 64) two per thread cover: four would issue loads past
// the end (config 4a: 8.63 -> 8.38 us, the same bits).
constexpr int kBatchA = 4, kBatchB = 4, kBatchBWide = 2;

typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

struct SmallArgs {
  GemmArgs g;
  int bm;          // output rows per workgroup: 64 (2x2 computing waves) or 128 (4x2)
  int a_kc, b_kc;  // unit stride on K
  int pa, pb;      // LDS bytes per staged line of A / B (multiple of 16)
  int kp;          // K rounded up to 16
  int nt;          // output columns per workgroup
  int a_direct;    // A fragments loaded from memory, A not staged
  int nt_store;    // f32 output in whole 128-byte lines: nontemporal stores
  int threads;     // staging threads: kStageThreads, or kWideThreads when alone on a CU
  int buf_store;   // f32 output whose batch slice fits 31-bit byte offsets: buffer stores
};

// Staging geometry of one operand for one workgroup.
struct Lines {
  __amdgpu_buffer_rsrc_t rsrc;  // slice base rounded down to 16 B .. end rounded up
  uint32_t c0;                  // byte offset of line 0 from the resource base
  uint32_t step;                // bytes between consecutive lines
  int nvalid;                   // lines holding data
  int nalloc;                   // lines written to LDS (those past nvalid as zeros)
  int len;                      // valid elements per line
  int ncpl;                     // 16-byte LDS chunks written per line
  int pitch;                    // LDS bytes per line
  bool aligned;                 // every line starts 16-byte aligned: one load per chunk
};

__device__ __forceinline__ Lines make_lines(const uint16_t *slice, uint32_t slice_bytes,
                                            int64_t line0, int64_t stride, int nvalid,
                                            int nalloc, int len, int ncpl, int pitch) {
  Lines l;
  // Every input is wave-uniform; readfirstlane keeps the resource in scalar
  // registers (a resource in vector registers turns each load into a loop).
  const uint64_t addr = reinterpret_cast<uintptr_t>(slice);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)addr);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(addr >> 32));
  const uint32_t delta = lo & 15u;
  const char *base = reinterpret_cast<const char *>(((uint64_t)hi << 32) | (lo & ~15u));
  const int range = __builtin_amdgcn_readfirstlane((int)((slice_bytes + delta + 15u) & ~15u));
  l.rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(base), (short)0, range, 0x00020000);
  l.c0 = delta + (uint32_t)(line0 * 2);
  l.step = (uint32_t)(stride * 2);
  l.nvalid = nvalid;
  l.nalloc = nalloc;
  l.len = len;
  l.ncpl = ncpl;
  l.pitch = pitch;
  l.aligned = ((l.c0 | l.step) & 15u) == 0;
  return l;
}

// Normalised chunk q (line i = q / ncpl, chunk c = q % ncpl): the two aligned
// global chunks holding elements 8c .. 8c+7 of line i, or only the first
// when every line is 16-byte aligned (config 4b's B: 8.17 -> 7.92 us).
// Chunks with no valid element load from beyond the resource's range: zeros,
// no memory access, and no branch to split the batch of loads.  (Loading
// each aligned chunk once and taking its neighbour from the next lane with a
// shuffle measured slower: 9.60 / 8.86 against 8.94 / 8.11 us on 4a / 4b.)
struct Raw {
  u32x4 lo, hi;
};
__device__ __forceinline__ Raw chunk_load(const Lines &l, int q, int nq) {
  const int i = q / l.ncpl, c = q - i * l.ncpl;
  const bool live = q < nq && i < l.nvalid && 8 * c < l.len;
  const uint32_t off = ((l.c0 + (uint32_t)i * l.step) & ~15u) + 16u * c;
  Raw r;
  r.lo = __builtin_amdgcn_raw_buffer_load_b128(l.rsrc, live ? off : kOOB, 0, 0);
  if (l.aligned)
    r.hi = u32x4{0u, 0u, 0u, 0u};  // the shift is zero: unused
  else
    r.hi = __builtin_amdgcn_raw_buffer_load_b128(l.rsrc, live ? off + 16u : kOOB, 0, 0);
  return r;
}

// Bytes [s, s+16) of lo:hi (s even, 0..14), elements of the line at or past
// `len` zeroed, written to the chunk's LDS slot.
__device__ __forceinline__ void chunk_store(const Lines &l, char *lds, int q, int nq, Raw r) {
  if (q >= nq) return;
  const int i = q / l.ncpl, c = q - i * l.ncpl;
  const uint32_t sh = (l.c0 + (uint32_t)i * l.step) & 15u;
  const uint32_t w[8] = {r.lo[0], r.lo[1], r.lo[2], r.lo[3], r.hi[0], r.hi[1], r.hi[2], r.hi[3]};
  // Skip sh/4 whole dwords in two steps (by 1, then by 2), as bit masks:
  // written as conditional selects, the compiler turns them into an indexed
  // array and routes it through scratch memory.
  const uint32_t m1 = 0u - ((sh >> 2) & 1u), m2 = 0u - ((sh >> 3) & 1u);
  uint32_t t[7], sel[5];
#pragma unroll
  for (int e = 0; e < 7; ++e) t[e] = w[e] ^ ((w[e] ^ w[e + 1]) & m1);
#pragma unroll
  for (int e = 0; e < 5; ++e) sel[e] = t[e] ^ ((t[e] ^ t[e + 2]) & m2);
  u32x4 out;
  const int e0 = 8 * c;
  const bool line_ok = i < l.nvalid;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    uint32_t v = __builtin_amdgcn_alignbyte(sel[d + 1], sel[d], sh & 3u);
    const int e = e0 + 2 * d;
    if (!line_ok || e >= l.len) v = 0u;
    else if (e + 1 >= l.len) v &= 0xffffu;
    out[d] = v;
  }
  *reinterpret_cast<u32x4 *>(lds + i * l.pitch + 16 * c) = out;
}

// Stage both operands.  Each round issues up to kBatchA chunks of A and
// kBatchB of B per thread (two loads each) before their LDS writes, so the
// latencies overlap.  (A and B get loops of their own: a resource chosen per
// lane would leave the wave-uniform registers.)
// SA: A is staged (otherwise B alone is).
template <int T, bool SA>
__device__ __forceinline__ void stage(const Lines &la, const Lines &lb, char *lds_a, char *lds_b,
                                      int tid) {
  constexpr int BA = SA ? kBatchA : 0;
  constexpr int BB = !SA && T == kWideThreads ? kBatchBWide : kBatchB;
  const int na = SA ? la.nalloc * la.ncpl : 0, nb = lb.nalloc * lb.ncpl;
  for (int r = 0; r * T * BA < na || r * T * BB < nb; ++r) {
    Raw va[SA ? BA : 1], vb[BB];
    const int qa = tid + r * T * BA, qb = tid + r * T * BB;
#pragma unroll
    for (int u = 0; u < BA; ++u) va[u] = chunk_load(la, qa + u * T, na);
#pragma unroll
    for (int u = 0; u < BB; ++u) vb[u] = chunk_load(lb, qb + u * T, nb);
#pragma unroll
    for (int u = 0; u < BA; ++u) chunk_store(la, lds_a, qa + u * T, na, va[u]);
#pragma unroll
    for (int u = 0; u < BB; ++u) chunk_store(lb, lds_b, qb + u * T, nb, vb[u]);
  }
}

// MFMA fragment of 32 rows (M rows of A or N columns of B) starting at
// `row0` of the workgroup's window, k16 step kk: lane l gets row row0 + l%32,
// k = 16 kk + 8 (l/32) + 0..7.  kc: LDS holds [row][k] (one 16-byte read);
// otherwise [k][row], read with ds_read_b64_tr_b16 (within each 16-lane group
// lane i receives element i of the four k-lines its group addresses).
__device__ __forceinline__ u32x4 read_frag(const char *lds, int pitch, bool kc, int row0, int kk,
                                           int lane) {
  if (kc) {
    const int row = row0 + (lane & 31), k0 = kk * 16 + 8 * (lane >> 5);
    return *reinterpret_cast<const u32x4 *>(lds + row * pitch + 2 * k0);
  }
  const int g = lane >> 4, p = lane & 15;
  const int n = row0 + 16 * (g & 1) + 4 * (p & 3);
  const int kb = kk * 16 + 8 * (g >> 1) + (p >> 2);
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4 *)(lds + kb * pitch + 2 * n));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4 *)(lds + (kb + 4) * pitch + 2 * n));
  const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
  return u32x4{l2[0], l2[1], h2[0], h2[1]};
}

// f32 epilogue through buffer stores, one 32-column block (columns n0j ..
// n0j + 31 of rows mw ..): one resource per batch slice whose range ends at
// its last element, a per-lane 32-bit offset (a column past N gets one past
// every range) plus the row's uniform offset, so rows past M and columns
// past N are dropped by the range check, with one add per store instead of
// 64-bit address arithmetic (config 4b: 9.10 -> 8.74 us).
template <bool NT>
__device__ __forceinline__ void store_f32_blk(const f32x16 &acc, const GemmArgs &a, int bidx,
                                              int mw, int n0j, int lane) {
  const bool has_bias = (a.epi == NOVA_HIP_EPI_BIAS || a.epi == NOVA_HIP_EPI_BIAS_GELU);
  const bool has_gelu = (a.epi == NOVA_HIP_EPI_BIAS_GELU || a.epi == NOVA_HIP_EPI_GELU);
  float *Cb = static_cast<float *>(a.C) + (int64_t)bidx * a.scb;
  const int range = (int)(((int64_t)(a.M - 1) * a.scm + a.N) * 4);
  const __amdgpu_buffer_rsrc_t rc =
      __builtin_amdgcn_make_buffer_rsrc(Cb, (short)0, range, 0x00020000);
  const int lrow = lane & 31, lh = lane >> 5;
  const uint32_t rstep = (uint32_t)a.scm * 4u;
  const int n = n0j + lrow;
  const uint32_t base = n < a.N ? (uint32_t)((mw + 4 * lh) * a.scm + n) * 4u : kOOB;
  const float bv = (has_bias && n < a.N) ? bias_at(a.bias, a.bias_dt, n) : 0.0f;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    float x = acc[v];
    if (has_bias) x = x + bv;
    if (has_gelu) x = gelu_tanh(x);
    const uint32_t off = base + (uint32_t)(8 * (v >> 2) + (v & 3)) * rstep;
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, x), rc, off, 0,
                                          NT ? 2 : 0);  // 2: nontemporal
  }
}

template <int TNW, bool NT>
__device__ __forceinline__ void store_f32_buf(const f32x16 (&acc)[1][TNW], const GemmArgs &a,
                                              int bidx, int mw, int nw, int lane) {
#pragma unroll
  for (int j = 0; j < TNW; ++j) store_f32_blk<NT>(acc[0][j], a, bidx, mw, nw + 32 * j, lane);
}

// MFMA phase of a window whose A is staged: the fragments of the next k16
// steps are read from LDS while step kk multiplies, D - 1 steps ahead in a
// ring of D fragment sets (the loop unrolled by D keeps the ring's indices
// constant).  D = 3 for up to two 32-column blocks per wave (config 4b:
// 7.37 -> 7.28 us, the same bits; four sets ran 7.88), 2 for more, whose
// third set would not fit the 128 VGPRs of a sixteen-wave workgroup.  The
// layouts are template parameters, so the loop has no branches around its
// LDS reads (with the layouts as runtime values every step waited for its
// own reads).
template <int DT, int TNW, bool AKC, bool BKC>
__device__ __forceinline__ void mfma_staged(f32x16 (&acc)[1][TNW], const char *lds_a, int pa,
                                            const char *lds_b, int pb, int row0, int nw,
                                            int ksteps, int lane) {
  constexpr int D = TNW <= 2 ? 3 : 2;
  u32x4 fa[D], fb[D][TNW];
#pragma unroll
  for (int d = 0; d < D - 1; ++d) {
    const int ks = d < ksteps ? d : ksteps - 1;
    fa[d] = read_frag(lds_a, pa, AKC, row0, ks, lane);
#pragma unroll
    for (int j = 0; j < TNW; ++j) fb[d][j] = read_frag(lds_b, pb, BKC, nw + 32 * j, ks, lane);
  }
  for (int k0 = 0; k0 < ksteps; k0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int kk = k0 + d;
      if (kk < ksteps) {
        // D - 1 steps ahead; past the end the last step is read again (in
        // bounds, unused).
        const int kr = kk + D - 1 < ksteps ? kk + D - 1 : ksteps - 1;
        const int w = (d + D - 1) % D;
        fa[w] = read_frag(lds_a, pa, AKC, row0, kr, lane);
#pragma unroll
        for (int j = 0; j < TNW; ++j) fb[w][j] = read_frag(lds_b, pb, BKC, nw + 32 * j, kr, lane);
#pragma unroll
        for (int j = 0; j < TNW; ++j) acc[0][j] = mfma_32x32x16<DT>(fa[d], fb[d][j], acc[0][j]);
      }
    }
  }
}

// MFMA phase of a window whose A fragments were loaded from memory (at most
// four k16 steps): every B fragment of the step read before its MFMAs.
template <int DT, int TNW, bool BKC>
__device__ __forceinline__ void mfma_direct(f32x16 (&acc)[1][TNW], const u32x4 (&fad)[4],
                                            const char *lds_b, int pb, int nw, int ksteps,
                                            int lane) {
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    if (kk >= ksteps) break;
    u32x4 fb[TNW];
#pragma unroll
    for (int j = 0; j < TNW; ++j) fb[j] = read_frag(lds_b, pb, BKC, nw + 32 * j, kk, lane);
#pragma unroll
    for (int j = 0; j < TNW; ++j) acc[0][j] = mfma_32x32x16<DT>(fad[kk], fb[j], acc[0][j]);
  }
}

// The same with the f32 buffer-store epilogue folded in, one 32-column block
// at a time: the next block's B fragments are read while this block
// multiplies, and this block's stores go out before the next block's MFMAs.
template <int DT, int TNW, bool BKC, bool NT>
__device__ __forceinline__ void mfma_direct_store(f32x16 (&acc)[1][TNW], const u32x4 (&fad)[4],
                                                  const char *lds_b, int pb, int nw, int ksteps,
                                                  const GemmArgs &a, int bidx, int mw, int n0,
                                                  int lane) {
  u32x4 fb[2][4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk)
    if (kk < ksteps) fb[0][kk] = read_frag(lds_b, pb, BKC, nw, kk, lane);
#pragma unroll
  for (int j = 0; j < TNW; ++j) {
    if (j + 1 < TNW) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        if (kk < ksteps)
          fb[(j + 1) & 1][kk] = read_frag(lds_b, pb, BKC, nw + 32 * (j + 1), kk, lane);
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      if (kk < ksteps) acc[0][j] = mfma_32x32x16<DT>(fad[kk], fb[j & 1][kk], acc[0][j]);
    store_f32_blk<NT>(acc[0][j], a, bidx, mw, n0 + nw + 32 * j, lane);
  }
}

template <int DT, int TNW, bool AD, bool NT, int ST>
__global__ __launch_bounds__(ST) void gemm_small_kernel(SmallArgs s) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const GemmArgs &a = s.g;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  // Tile indices come out of VALU divisions; readfirstlane tells the compiler
  // they are wave-uniform, so the buffer resources stay in scalar registers
  // (otherwise every load becomes a waterfall loop).
  const int per_batch = a.tiles_m * a.tiles_n;
  const int bidx = __builtin_amdgcn_readfirstlane(blockIdx.x / per_batch);
  const int t = blockIdx.x - bidx * per_batch;
  const int tm = __builtin_amdgcn_readfirstlane(t / a.tiles_n);
  const int tn = __builtin_amdgcn_readfirstlane(t - tm * a.tiles_n);
  const int m0 = tm * s.bm, n0 = tn * s.nt;
  const int m_valid = min(s.bm, a.M - m0), n_valid = min(s.nt, a.N - n0);
  // The epilogue writes rows [m0, m0 + m_valid) only: its own copy of the
  // arguments ends the output at the window's last row, so every store of a
  // row past it is dropped by the range check (or the row test).
  GemmArgs ge = a;
  ge.M = m0 + m_valid;

  const uint16_t *A = a.A + (int64_t)bidx * a.sab;
  const uint16_t *B = a.B + (int64_t)bidx * a.sbb;
  // A K-contiguous: lines are the valid rows m0.. (sa_outer apart), kp
  // elements each (k >= K zeroed); otherwise lines are k = 0..kp-1 (sa_outer
  // apart, k >= K zeroed) over the valid part of the row window m0...
  // Likewise B with N and NT.  LDS rows or columns past the valid ones are
  // left unwritten: they only feed outputs the epilogue discards.
  const int ka = (m_valid + 7) / 8, kb = (n_valid + 7) / 8;
  // A read directly (AD) has no lines to stage.
  const Lines la = AD       ? make_lines(A, a.a_bytes, 0, a.sa_outer, 0, 0, a.K, s.kp / 8, s.pa)
                   : s.a_kc ? make_lines(A, a.a_bytes, (int64_t)m0 * a.sa_outer, a.sa_outer,
                                         m_valid, m_valid, a.K, s.kp / 8, s.pa)
                            : make_lines(A, a.a_bytes, m0, a.sa_outer, a.K, s.kp, m_valid, ka,
                                         s.pa);
  const Lines lb = s.b_kc ? make_lines(B, a.b_bytes, (int64_t)n0 * a.sb_outer, a.sb_outer,
                                       n_valid, n_valid, a.K, s.kp / 8, s.pb)
                          : make_lines(B, a.b_bytes, n0, a.sb_outer, a.K, s.kp, n_valid, kb,
                                       s.pb);
  char *lds_a = smem;
  char *lds_b = AD ? smem : smem + (s.a_kc ? s.bm : s.kp) * s.pa;
  // Direct A fragments (K-contiguous A, 16-byte aligned rows, K % 16 == 0,
  // K <= 64): lane l of a computing wave loads row m0 + 32 wm + l % 32,
  // k = 16 kk + 8 (l / 32) .. + 7 for every k16 step, issued before the B
  // staging so that the latencies overlap.  Rows past the slice read zero;
  // rows past M inside it feed discarded outputs.
  u32x4 fad[4];
  if constexpr (AD) {
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t *>(A), (short)0, (int)a.a_bytes, 0x00020000);
    const bool computes = !(s.bm == 64 && wave >= 4) && wm * 32 < m_valid;
    const uint32_t rowoff = (uint32_t)((m0 + wm * 32 + (lane & 31)) * a.sa_outer * 2) +
                            16u * (lane >> 5);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      if (computes && kk * 16 < s.kp)
        fad[kk] = __builtin_amdgcn_raw_buffer_load_b128(ra, rowoff + 32u * kk, 0, 0);
  }
  stage<ST, !AD>(la, lb, lds_a, lds_b, tid);
  __syncthreads();
  // 64-row windows: waves 0-3 compute (2x2); 128-row windows: waves 0-7
  // (4x2), a wave past the window's valid rows stops here (waves 8-15 of a
  // wide workgroup, whose wm >= 4, always do).
  if (s.bm == 64 && wave >= 4) return;
  if (wm * 32 >= m_valid) return;

  f32x16 acc[1][TNW];
#pragma unroll
  for (int j = 0; j < TNW; ++j)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[0][j][v] = 0.0f;

  const int ksteps = s.kp / 16;
  const int nw = wn * (TNW * 32);
  if constexpr (AD) {
    if (s.buf_store) {
      if (s.b_kc)
        mfma_direct_store<DT, TNW, true, NT>(acc, fad, lds_b, s.pb, nw, ksteps, ge, bidx,
                                             m0 + wm * 32, n0, lane);
      else
        mfma_direct_store<DT, TNW, false, NT>(acc, fad, lds_b, s.pb, nw, ksteps, ge, bidx,
                                              m0 + wm * 32, n0, lane);
      return;
    }
    if (s.b_kc)
      mfma_direct<DT, TNW, true>(acc, fad, lds_b, s.pb, nw, ksteps, lane);
    else
      mfma_direct<DT, TNW, false>(acc, fad, lds_b, s.pb, nw, ksteps, lane);
  } else if (s.a_kc) {
    if (s.b_kc)
      mfma_staged<DT, TNW, true, true>(acc, lds_a, s.pa, lds_b, s.pb, wm * 32, nw, ksteps, lane);
    else
      mfma_staged<DT, TNW, true, false>(acc, lds_a, s.pa, lds_b, s.pb, wm * 32, nw, ksteps, lane);
  } else {
    if (s.b_kc)
      mfma_staged<DT, TNW, false, true>(acc, lds_a, s.pa, lds_b, s.pb, wm * 32, nw, ksteps, lane);
    else
      mfma_staged<DT, TNW, false, false>(acc, lds_a, s.pa, lds_b, s.pb, wm * 32, nw, ksteps,
                                         lane);
  }
  if (s.buf_store)
    store_f32_buf<TNW, NT>(acc, ge, bidx, m0 + wm * 32, n0 + nw, lane);
  else
    store_outputs<1, TNW, NT>(acc, ge, bidx, m0 + wm * 32, n0 + nw, lane);
}

template <int DT, int ST>
int32_t launch_st(const SmallArgs &s, size_t lds, hipStream_t st) {
  const dim3 grid((unsigned)(s.g.batch * s.g.tiles_m * s.g.tiles_n)), block(ST);
  switch ((s.a_direct ? 8 : 0) + (s.nt_store ? 4 : 0) + s.nt / 64 - 1) {
#define NOVA_SMALL(AD, NT, T)                                                            \
  case (AD ? 8 : 0) + (NT ? 4 : 0) + T - 1:                                             \
    hipLaunchKernelGGL((gemm_small_kernel<DT, T, AD, NT, ST>), grid, block, lds, st, s); \
    break;
    NOVA_SMALL(false, false, 1) NOVA_SMALL(false, false, 2)
    NOVA_SMALL(false, false, 3) NOVA_SMALL(false, false, 4)
    NOVA_SMALL(false, true, 1) NOVA_SMALL(false, true, 2)
    NOVA_SMALL(false, true, 3) NOVA_SMALL(false, true, 4)
    NOVA_SMALL(true, false, 1) NOVA_SMALL(true, false, 2)
    NOVA_SMALL(true, false, 3) NOVA_SMALL(true, false, 4)
    NOVA_SMALL(true, true, 1) NOVA_SMALL(true, true, 2)
    NOVA_SMALL(true, true, 3) NOVA_SMALL(true, true, 4)
#undef NOVA_SMALL
    default: break;
  }
  return check_hip(hipGetLastError(), "gemm_small launch");
}

template <int DT>
int32_t launch_dt(const SmallArgs &s, size_t lds, hipStream_t st) {
  return s.threads == kWideThreads ? launch_st<DT, kWideThreads>(s, lds, st)
                                   : launch_st<DT, kStageThreads>(s, lds, st);
}

// Staging geometry chosen on the host: output columns per workgroup, K
// rounded up to whole k16 steps, and each operand's LDS line pitch: a [row][k]
// line's padded width plus 16 bytes, which spreads the rows of a 16-byte
// fragment read over the banks; a [k][row] line's plus 64 bytes, so that the
// four k-lines a 16-lane group of ds_read_b64_tr_b16 reads (64 bytes each
// per half wave) fall on disjoint banks (config 4a: 9.69 -> 9.53 us).
struct SmallPlan {
  int nt, kp, pa, pb, a_lines, b_lines;
  size_t lds;
};

SmallPlan plan_small(int64_t N, int64_t K, bool akc, bool bkc, int bm = kBM) {
  SmallPlan p;
  p.nt = N >= kMaxNT ? kMaxNT : (int)(((N + 63) / 64) * 64);
  p.kp = (int)(((K + 15) / 16) * 16);
  p.pa = akc ? p.kp * 2 + 16 : bm * 2 + 64;
  p.a_lines = akc ? bm : p.kp;
  p.pb = bkc ? p.kp * 2 + 16 : p.nt * 2 + 64;
  p.b_lines = bkc ? p.nt : p.kp;
  p.lds = (size_t)p.a_lines * p.pa + (size_t)p.b_lines * p.pb;
  return p;
}

}  // namespace

bool gemm_small_applicable(const gemm::GemmArgs &a, bool akc, bool bkc) {
  if (a.K <= 0 || a.K > 512) return false;
  // Resources reach up to 30 bytes past a slice (both ends rounded to 16).
  if (a.a_bytes > 0x7fffff00u || a.b_bytes > 0x7fffff00u) return false;
  // The whole K range of a 64-row A window and an NT-column B window must
  // fit the staging budget (80 KB: two workgroups per CU).
  const SmallPlan p = plan_small(a.N, a.K, akc, bkc);
  return p.lds <= (size_t)kLdsBytes;
}

int32_t launch_gemm_small(const gemm::GemmArgs &a_in, int in_dt, bool akc, bool bkc,
                          hipStream_t st) {
  SmallArgs s;
  s.g = a_in;
  SmallPlan p = plan_small(a_in.N, a_in.K, akc, bkc);
  s.bm = kBM;
  s.threads = kStageThreads;
  // 128-row windows (eight computing waves) when they still fit the staging
  // budget and cut the workgroups a CU must run: each wave's share of the
  // work is the same, so the time follows the most loaded CU.  Config 4a:
  // 192 workgroups instead of 384 on 256 CUs, 11.40 -> 10.35 us, the same
  // bits (in-process A/B).  When there are no more such workgroups than CUs,
  // each has a CU to itself and may use its whole LDS: config 4b's 128-row
  // A window (95 KB) then runs 7.73 against 7.91 us in 64-row windows.
  {
    const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
    const int64_t tn = (a_in.N + p.nt - 1) / p.nt;
    const int64_t t64 = (int64_t)a_in.batch * ((a_in.M + kBM - 1) / kBM) * tn;
    const int64_t t128 = (int64_t)a_in.batch * ((a_in.M + 2 * kBM - 1) / (2 * kBM)) * tn;
    const SmallPlan p2 = plan_small(a_in.N, a_in.K, akc, bkc, 2 * kBM);
    const size_t cu_lds = (size_t)std::min(kCuLdsBytes, device_lds_per_block());
    const size_t budget = t128 <= cus ? std::max(cu_lds, (size_t)kLdsBytes) : (size_t)kLdsBytes;
    if (p2.lds <= budget && (t128 + cus - 1) / cus < (t64 + cus - 1) / cus) {
      p = p2;
      s.bm = 2 * kBM;
      // No more workgroups than CUs: each runs alone and stages on sixteen
      // waves (the CU's 64 wave slots hold them at up to 128 VGPRs).
      if (t128 <= cus) s.threads = kWideThreads;
    }
  }
  // A read straight into MFMA fragments: K-contiguous, every row 16-byte
  // aligned, whole k16 steps (no k past K to zero), at most four of them.
  s.a_direct = akc && (reinterpret_cast<uintptr_t>(a_in.A) & 15u) == 0 &&
               a_in.sa_outer % 8 == 0 && a_in.sab % 8 == 0 && a_in.K % 16 == 0 && a_in.K <= 64;
  if (s.a_direct) p.lds -= (size_t)p.a_lines * p.pa;
  // Each store instruction writes 32 consecutive f32 of two rows: whole
  // 128-byte lines when the rows and the slices are line-aligned and N is a
  // multiple of 32.  Those go out with the nontemporal hint (config 4b's
  // [96, 197, 64] output: 9.54 -> 9.08 us); partial lines (config 4a's
  // 788-byte rows) would take longer with it (9.7 -> 12.8 us).
  s.nt_store = a_in.out_dt == NOVA_HIP_DT_F32 && (reinterpret_cast<uintptr_t>(a_in.C) & 127u) == 0 &&
               a_in.scm % 32 == 0 && a_in.scb % 32 == 0 && a_in.N % 32 == 0;
  // Buffer stores: 32-bit byte offsets.  A store instruction addresses rows
  // up to 31 past the last valid one (dropped by the range), so the offsets
  // of rows up to M + 31 must not wrap around 2^32 into the range either.
  s.buf_store = a_in.out_dt == NOVA_HIP_DT_F32 &&
                ((int64_t)(a_in.M - 1) * a_in.scm + a_in.N) * 4 <= 0x7fffffff &&
                ((int64_t)(a_in.M + 31) * a_in.scm + a_in.N) * 4 < ((int64_t)1 << 32);
  s.a_kc = akc;
  s.b_kc = bkc;
  s.pa = p.pa;
  s.pb = p.pb;
  s.nt = p.nt;
  s.kp = p.kp;
  s.g.tiles_m = (a_in.M + s.bm - 1) / s.bm;
  s.g.tiles_n = (a_in.N + p.nt - 1) / p.nt;
  if ((int64_t)s.g.batch * s.g.tiles_m * s.g.tiles_n > 0x7fffffff)
    return fail(NOVA_HIP_ERANGE, "gemm: too many output tiles");
  if (in_dt == NOVA_HIP_DT_BF16) return launch_dt<NOVA_HIP_DT_BF16>(s, p.lds, st);
  return launch_dt<NOVA_HIP_DT_F16>(s, p.lds, st);
}

}  // namespace nova_hip
