// f32 GEMM on the f32 matrix cores (v_mfma_f32_32x32x2_f32): the products
// are exact f32 multiplies and the sums f32, but the accumulation order is
// the MFMA's and the tile loop's, not the reference's sequential k.  The
// result is therefore not bit-identical to Nova's CPU pipeline (the exact
// kernel in gemm_f32.hip is), but it is within the f32 parity bar (1e-4
// relative): the error is the ordinary rounding of an f32 dot product.  It
// is what a GPU lowering of an f32 linalg.matmul would run (the reference's
// NVPTX path uses tf32 mma.sync, which is not within 1e-4); a caller opts
// in with NOVA_HIP_GEMM_F32_MFMA.
//
// 128x128 output tile per 256-thread workgroup (2x2 waves of 64x64, each
// 2x2 tiles of 32x32), K staged through LDS 32 at a time, register-staged
// global loads two stages ahead of the stage being multiplied.  Each MFMA takes
// k = 2 values per lane half: lane half h of MFMA j (j = 0..3) of an
// 8-deep k group holds k = 8g + 4h + j, so a K-contiguous operand's four
// values for the four MFMAs are one 16-byte LDS read.  An operand whose
// unit stride is on M / N keeps that layout in LDS and is read with four
// 4-byte reads.  Long-K problems with few tiles split K over several
// workgroups; the partial sums go to the workspace and a second kernel adds
// them in split order, so the result is the same on every run.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "nova_hip_internal.h"

namespace nova_hip {
namespace {

constexpr int kBM = 128, kBN = 128, kBK = 32;
constexpr int kThreads = 256;
constexpr int kStrK = kBK + 4;     // K-contiguous stage: [128 rows][36]
constexpr int kStrMN = kBM + 8;    // M/N-contiguous stage: [32 k][136]
constexpr int kStage = kBM * kStrK > kBK * kStrMN ? kBM * kStrK : kBK * kStrMN;
constexpr uint32_t kOOB = 0x80000000u;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct F32MArgs {
  const float *A;
  const float *B;
  float *C;
  const void *bias;
  float *part;  // split-K partials [splits][batch][M][N], or null
  int64_t sab, sa_outer, sbb, sb_outer, scb, scm;
  uint32_t a_bytes, b_bytes;
  int M, N, K;
  int tiles_m, tiles_n, batch;
  int splits, k_split;  // K range of split s: [s * k_split, min(K, (s + 1) * k_split))
  int bias_dt, epi;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_of(const float *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(p), (short)0, (int)bytes,
                                           0x00020000);
}

__device__ __forceinline__ float bias_f32(const void *bias, int dt, int n) {
  if (dt == NOVA_HIP_DT_F32) return static_cast<const float *>(bias)[n];
  const uint16_t h = static_cast<const uint16_t *>(bias)[n];
  if (dt == NOVA_HIP_DT_BF16) return __uint_as_float(static_cast<uint32_t>(h) << 16);
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// GELU in the op order of NovaGeluForwardPattern (NovaToLinalgGeneric.cpp:
// 1310-1331).
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

// One operand's global -> register -> LDS staging for a 128 x 32 (rows x k)
// stage.  KC: unit stride on K.  VEC: 16-byte loads (aligned rows, whole
// 4-element chunks along the unit-stride dim).  Loads outside the operand
// (rows >= R, k >= K) read zero.
template <bool KC, bool VEC>
struct Stager {
  __amdgpu_buffer_rsrc_t rsrc;
  int64_t s_outer;
  int row0, R, K;
  f32x4 v[4];

  // Chunk q (0..3) of this thread: 4 consecutive elements along the unit-
  // stride dim.  KC: row = c / 8, k = 4 (c % 8); MN: k = c / 32, row = 4 (c % 32).
  __device__ __forceinline__ void chunk(int q, int &row, int &k) const {
    const int c = threadIdx.x + q * kThreads;
    if (KC) { row = c >> 3; k = (c & 7) * 4; }
    else { k = c >> 5; row = (c & 31) * 4; }
  }
  __device__ __forceinline__ void load(int k0, int kend) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      int r, k;
      chunk(q, r, k);
      const int gr = row0 + r, gk = k0 + k;
      if constexpr (VEC) {
        const bool ok = gr < R && gk < kend;
        const int64_t e = KC ? (int64_t)gr * s_outer + gk : (int64_t)gk * s_outer + gr;
        const uint32_t off = ok ? (uint32_t)(e * 4) : kOOB;
        v[q] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0));
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int rr = KC ? gr : gr + u, kk = KC ? gk + u : gk;
          const bool ok = rr < R && kk < kend;
          const int64_t e = KC ? (int64_t)rr * s_outer + kk : (int64_t)kk * s_outer + rr;
          const uint32_t off = ok ? (uint32_t)(e * 4) : kOOB;
          v[q][u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc, off, 0, 0));
        }
      }
    }
  }
  __device__ __forceinline__ void store(float *lds) const {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      int r, k;
      chunk(q, r, k);
      float *dst = KC ? lds + r * kStrK + k : lds + k * kStrMN + r;
      *reinterpret_cast<f32x4 *>(dst) = v[q];
    }
  }
};

// The four values (k = 8g + 4h + j, j = 0..3) of row `row` for lane half h.
template <bool KC>
__device__ __forceinline__ f32x4 frag(const float *lds, int row, int g, int h) {
  if constexpr (KC) {
    return *reinterpret_cast<const f32x4 *>(lds + row * kStrK + 8 * g + 4 * h);
  } else {
    const float *p = lds + (8 * g + 4 * h) * kStrMN + row;
    return f32x4{p[0], p[kStrMN], p[2 * kStrMN], p[3 * kStrMN]};
  }
}

template <bool AKC, bool BKC, bool VEC>
__global__ __launch_bounds__(kThreads, 2) void gemm_f32_mfma_kernel(F32MArgs a) {
  __shared__ __attribute__((aligned(16))) float sa[2][kStage];
  __shared__ __attribute__((aligned(16))) float sb[2][kStage];

  const int tiles = a.tiles_m * a.tiles_n;
  int id = blockIdx.x;
  const int split = id / (tiles * a.batch);
  id -= split * tiles * a.batch;
  const int b = id / tiles;
  int t = id - b * tiles;
  // Bands of four tile rows swept column by column: neighbouring workgroups
  // share operand panels in L2.
  const int band = t / (4 * a.tiles_n);
  const int first = band * 4;
  const int gsz = min(a.tiles_m - first, 4);
  const int in_band = t - band * 4 * a.tiles_n;
  const int tm = first + in_band % gsz, tn = in_band / gsz;
  const int m0 = tm * kBM, n0 = tn * kBN;

  const int kbeg = split * a.k_split;
  const int kend = min(a.K, kbeg + a.k_split);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, h = lane >> 5;

  Stager<AKC, VEC> ga;
  ga.rsrc = rsrc_of(a.A + (int64_t)b * a.sab, a.a_bytes);
  ga.s_outer = a.sa_outer;
  ga.row0 = m0;
  ga.R = a.M;
  ga.K = a.K;
  Stager<BKC, VEC> gb;
  gb.rsrc = rsrc_of(a.B + (int64_t)b * a.sbb, a.b_bytes);
  gb.s_outer = a.sb_outer;
  gb.row0 = n0;
  gb.R = a.N;
  gb.K = a.K;

  const bool has_bias = (a.epi == NOVA_HIP_EPI_BIAS || a.epi == NOVA_HIP_EPI_BIAS_GELU) && split == 0;
  f32x16 acc[2][2];
#pragma unroll
  for (int jb = 0; jb < 2; ++jb) {
    const int n = n0 + wn * 64 + jb * 32 + l32;
    const float init = (has_bias && n < a.N) ? bias_f32(a.bias, a.bias_dt, n) : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][jb][v] = init;
  }

  // Global loads run two stages ahead: register set P holds the stage that
  // goes into LDS buffer P.  Stage s + 2 is loaded into set P (whose stage s
  // is already in LDS) while stage s is multiplied, and stage s + 1 (set
  // P ^ 1, loaded a stage earlier) is written to LDS after it, so each load
  // has two stages' MFMA time to arrive.
  Stager<AKC, VEC> ga1 = ga;
  Stager<BKC, VEC> gb1 = gb;
  ga.load(kbeg, kend);
  gb.load(kbeg, kend);
  ga.store(sa[0]);
  gb.store(sb[0]);
  if (kbeg + kBK < kend) {
    ga1.load(kbeg + kBK, kend);
    gb1.load(kbeg + kBK, kend);
  }
  __syncthreads();
  auto multiply = [&](const float *A, const float *B) __attribute__((always_inline)) {
#pragma unroll
    for (int g = 0; g < kBK / 8; ++g) {
      f32x4 fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) fa[i] = frag<AKC>(A, wm * 64 + i * 32 + l32, g, h);
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) fb[jb] = frag<BKC>(B, wn * 64 + jb * 32 + l32, g, h);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int jb = 0; jb < 2; ++jb)
            acc[i][jb] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][j], fb[jb][j], acc[i][jb],
                                                              0, 0, 0);
    }
  };
  for (int k0 = kbeg; k0 < kend; k0 += 2 * kBK) {
    // stage k0: LDS buffer 0, register set 0 / 1 for stages k0 + 2 / k0 + 1
    if (k0 + 2 * kBK < kend) {
      ga.load(k0 + 2 * kBK, kend);
      gb.load(k0 + 2 * kBK, kend);
    }
    multiply(sa[0], sb[0]);
    if (k0 + kBK < kend) {
      ga1.store(sa[1]);
      gb1.store(sb[1]);
    }
    __syncthreads();
    if (k0 + kBK >= kend) break;
    // stage k0 + 1: LDS buffer 1, register sets swapped
    if (k0 + 3 * kBK < kend) {
      ga1.load(k0 + 3 * kBK, kend);
      gb1.load(k0 + 3 * kBK, kend);
    }
    multiply(sa[1], sb[1]);
    if (k0 + 2 * kBK < kend) {
      ga.store(sa[0]);
      gb.store(sb[0]);
    }
    __syncthreads();
  }

  // Accumulator element v of lane l: row 8 (v / 4) + 4 h + v % 4, column l % 32
  // of its 32 x 32 tile.
  const bool has_gelu = a.epi == NOVA_HIP_EPI_BIAS_GELU || a.epi == NOVA_HIP_EPI_GELU;
#pragma unroll
  for (int jb = 0; jb < 2; ++jb) {
    const int n = n0 + wn * 64 + jb * 32 + l32;
    if (n >= a.N) continue;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + wm * 64 + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
        if (m >= a.M) continue;
        float x = acc[i][jb][v];
        if (a.part) {
          a.part[(((int64_t)split * a.batch + b) * a.M + m) * a.N + n] = x;
        } else {
          if (has_gelu) x = gelu_ref(x);
          a.C[(int64_t)b * a.scb + (int64_t)m * a.scm + n] = x;
        }
      }
  }
}

// C = epilogue(sum of the split partials, in split order).
__global__ __launch_bounds__(256) void split_reduce_kernel(const float *part, int splits,
                                                           int64_t per_split, int M, int N,
                                                           float *C, int64_t scb, int64_t scm,
                                                           int gelu) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= per_split) return;
  float s = part[i];
  for (int k = 1; k < splits; ++k) s = s + part[(int64_t)k * per_split + i];
  if (gelu) s = gelu_ref(s);
  const int64_t mn = (int64_t)M * N;
  const int64_t b = i / mn;
  const int64_t r = i - b * mn;
  const int64_t m = r / N, n = r - m * N;
  C[b * scb + m * scm + n] = s;
}

template <bool AKC, bool BKC>
void launch_layouts(const F32MArgs &a, bool vec, dim3 grid, hipStream_t s) {
  if (vec)
    hipLaunchKernelGGL((gemm_f32_mfma_kernel<AKC, BKC, true>), grid, dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL((gemm_f32_mfma_kernel<AKC, BKC, false>), grid, dim3(kThreads), 0, s, a);
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

int32_t launch_gemm_f32_mfma(const GemmProblem &p, hipStream_t s) {
  if (p.batch == 0 || p.M == 0 || p.N == 0) return NOVA_HIP_SUCCESS;
  if (p.M > 0x7fffffff || p.N > 0x7fffffff || p.K > 0x7fffffff)
    return fail(NOVA_HIP_ERANGE, "gemm_f32_mfma: dimension exceeds 2^31-1");
  if (p.out_dt != NOVA_HIP_DT_F32 || p.in_dt != NOVA_HIP_DT_F32)
    return fail(NOVA_HIP_EDTYPE, "gemm_f32_mfma: f32 inputs and output only");
  F32MArgs a;
  a.A = static_cast<const float *>(p.A);
  a.B = static_cast<const float *>(p.B);
  a.C = static_cast<float *>(p.C);
  a.bias = p.bias;
  a.part = nullptr;
  a.sab = p.sab;
  a.sa_outer = p.sa_outer;
  a.sbb = p.sbb;
  a.sb_outer = p.sb_outer;
  a.scb = p.scb;
  a.scm = p.scm;
  // Byte extent of one batch slice of each operand (the buffer range).
  const int64_t a_ext = p.K == 0 ? 0 : p.a_kcontig ? (p.M - 1) * p.sa_outer + p.K
                                                   : (p.K - 1) * p.sa_outer + p.M;
  const int64_t b_ext = p.K == 0 ? 0 : p.b_kcontig ? (p.N - 1) * p.sb_outer + p.K
                                                   : (p.K - 1) * p.sb_outer + p.N;
  if (a_ext * 4 > 0x7fffffff || b_ext * 4 > 0x7fffffff)
    return fail(NOVA_HIP_ERANGE, "gemm_f32_mfma: an operand's batch slice exceeds 2 GiB");
  a.a_bytes = (uint32_t)(a_ext * 4);
  a.b_bytes = (uint32_t)(b_ext * 4);
  a.M = (int)p.M;
  a.N = (int)p.N;
  a.K = (int)p.K;
  a.tiles_m = (int)((p.M + kBM - 1) / kBM);
  a.tiles_n = (int)((p.N + kBN - 1) / kBN);
  a.batch = (int)p.batch;
  a.bias_dt = p.bias_dt;
  a.epi = p.epi;
  const int64_t tiles = p.batch * a.tiles_m * a.tiles_n;
  // Split K when K is long enough to share: up to 8 splits of at least
  // 1024, the count that minimises the estimated time, i.e. the rounds of
  // resident workgroups (two per CU) times the K stages each runs (~3 us
  // per 32-deep stage of a 128x128 tile with two workgroups per CU,
  // measured on the GPT step's grad_input GEMM) plus the split reduction's
  // HBM traffic (splits + 1 passes over the output at ~5 TB/s).  Rounds
  // count whole: 576 workgroups on 512 slots take two rounds, so 192 tiles
  // run fastest with 8 splits (3 rounds of 197 stages), not 3 (2 rounds of
  // 524); and 1179 tiles of K = 8192 (2.3 rounds) with 3 (7 rounds of 86
  // stages instead of 3 of 256).
  const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
  int splits = 1;
  if (p.K >= 2048) {
    const int64_t slots = 2 * (int64_t)cus;
    const int64_t stages = (p.K + kBK - 1) / kBK;
    const double out_bytes = (double)p.batch * p.M * p.N * 4.0;
    double best = 0.0;
    // The partials take splits x the output of workspace: at most 1 GiB.
    for (int sp = 1; sp <= 8 && (sp == 1 || (p.K / sp >= 1024 && sp * out_bytes <= 1073741824.0));
         ++sp) {
      const int64_t rounds = (tiles * sp + slots - 1) / slots;
      const double us = (double)(rounds * ((stages + sp - 1) / sp)) * 3.0 +
                        (sp > 1 ? (sp + 1) * out_bytes / 5e12 * 1e6 : 0.0);
      if (sp == 1 || us < best) {
        best = us;
        splits = sp;
      }
    }
  }
  const int64_t k_split = ((p.K + splits - 1) / splits + kBK - 1) / kBK * kBK;
  a.k_split = (int)(k_split > 0 ? k_split : kBK);
  splits = (int)((p.K + a.k_split - 1) / a.k_split);
  if (splits < 1) splits = 1;
  a.splits = splits;
  const int64_t per_split = p.batch * p.M * p.N;
  WorkspaceLease lease;  // the partials, held until their reduction is enqueued
  if (splits > 1) {
    a.part = static_cast<float *>(lease.acquire(s, (size_t)(splits * per_split) * 4));
    if (!a.part) return NOVA_HIP_ENOMEM;
  }
  const int64_t grid = tiles * splits;
  if (grid > 0x7fffffff) return fail(NOVA_HIP_ERANGE, "gemm_f32_mfma: grid too large");
  // 16-byte loads: aligned bases, rows that stay aligned, whole 4-element
  // chunks along each operand's unit-stride dim.
  bool vec = aligned16(p.A) && aligned16(p.B) && p.sa_outer % 4 == 0 && p.sb_outer % 4 == 0 &&
             p.sab % 4 == 0 && p.sbb % 4 == 0;
  vec = vec && (p.a_kcontig ? p.K % 4 == 0 : p.M % 4 == 0);
  vec = vec && (p.b_kcontig ? p.K % 4 == 0 : p.N % 4 == 0);
  const dim3 g((unsigned)grid);
  if (p.a_kcontig && p.b_kcontig) launch_layouts<true, true>(a, vec, g, s);
  else if (p.a_kcontig) launch_layouts<true, false>(a, vec, g, s);
  else if (p.b_kcontig) launch_layouts<false, true>(a, vec, g, s);
  else launch_layouts<false, false>(a, vec, g, s);
  int32_t rc = check_hip(hipGetLastError(), "gemm_f32_mfma launch");
  if (rc || splits == 1) return rc;
  const int gelu = (p.epi == NOVA_HIP_EPI_BIAS_GELU || p.epi == NOVA_HIP_EPI_GELU) ? 1 : 0;
  hipLaunchKernelGGL(split_reduce_kernel, dim3((unsigned)((per_split + 255) / 256)), dim3(256), 0,
                     s, a.part, splits, per_split, a.M, a.N, a.C, p.scb, p.scm, gelu);
  return check_hip(hipGetLastError(), "gemm_f32_mfma split reduce launch");
}

}  // namespace nova_hip
