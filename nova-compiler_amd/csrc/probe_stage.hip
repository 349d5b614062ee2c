// Measurement probe for bench.py --telemetry (not part of the op path): the
// energy of the two ways a GEMM brings its operands into LDS.  One
// workgroup per CU runs the persistent GEMM's per-K-step work without its
// tile addressing and without HBM traffic: 64 KB per step from a 2 MB
// L2-resident buffer into the free stage of a two-stage LDS ring, while
// each of the four waves reads eight 16-byte fragments and issues sixteen
// v_mfma_f32_32x32x16_bf16 per k16 step (64 per K step) from the other
// stage.  The operands reach LDS either by LDS-DMA (buffer_load ... lds,
// as gemm_pers_kernel does) or by 16-byte loads into registers followed by
// ds_write (the register-staged path); a third mode stages by LDS-DMA and
// reads the B fragments as gemm_pers_kernel reads an N-contiguous B: two
// transposing ds_read_b64_tr_b16 per fragment from [k][n] lines with the
// GEMM's chunk swizzle.  Under the board's power limit the MFMA rate each
// sustains, with its power and clock, tells which path costs more energy.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kStageBytes = 64 * 1024;                // a 256x64 A and B panel of bf16
constexpr int kSlots = kStageBytes / 16;              // 16-byte slots per stage
constexpr int kLoads = kSlots / kThreads;             // 16 per thread per step
constexpr int kSrcBytes = 2 * 1024 * 1024;            // source, resident in each XCD's L2
constexpr int kSrcSteps = kSrcBytes / kStageBytes;    // 32 distinct steps of source

// 16-byte slot of fragment f (0-3: A rows, 4-7: B rows, 32 rows each) for
// k16 step kk, lane l: row 32 f + l % 32, chunk 2 kk + l / 32, chunks XOR-
// swizzled by row (conflict-free 16-byte reads, as in the GEMM).
__device__ __forceinline__ int frag_slot(int f, int kk, int lane, int wave) {
  const int row = ((wave & 1) * 4 + f) * 32 + (lane & 31);  // 0..255 within the operand
  const int c = (2 * kk + (lane >> 5)) ^ (row & 7);
  return (f >= 4 ? kSlots / 2 : 0) + (row & 255) * 8 + c;
}

// B fragment f (0-3) of k16 step kk from the stage's [k][n] B half (64
// k-lines of 256 bf16, 16-byte chunk c of line k at chunk c ^ swz(k)): lane
// group g = l / 16 reads four k-lines at n = base + 16 (g & 1) + 4 (l % 4)
// with ds_read_b64_tr_b16, twice (k and k + 4), as gemm_pers_kernel does.
__device__ __forceinline__ u32x4 frag_tr(const u32x4 *stage, int f, int kk, int lane, int wave) {
  const int g = lane >> 4, p = lane & 15;
  const int n = (wave & 1) * 128 + f * 32 + 16 * (g & 1) + 4 * (p & 3);
  const int kb = kk * 16 + 8 * (g >> 1) + (p >> 2);
  auto slot = [](int k, int c16) { return k * 32 + (c16 ^ (((k & 3) << 1) ^ ((k & 3) << 2))); };
  const char *b = reinterpret_cast<const char *>(stage + kSlots / 2);
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4 *)(b + 16 * slot(kb, n >> 3) + 2 * (n & 7)));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4 *)(b + 16 * slot(kb + 4, n >> 3) + 2 * (n & 7)));
  const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
  return u32x4{l2[0], l2[1], h2[0], h2[1]};
}

// MODE 0: LDS-DMA, 16-byte fragment reads; 1: registers + ds_write, 16-byte
// reads; 2: LDS-DMA, B fragments by transposing reads.
template <int MODE>
__global__ __launch_bounds__(kThreads) void stage_loop(const u32x4 *src, float *out, int iters) {
  constexpr bool DMA = MODE != 1;
  __shared__ u32x4 ring[2][kSlots];  // 128 KB: one workgroup per CU
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<u32x4 *>(src), (short)0, kSrcBytes, 0x00020000);
  f32x16 acc[16];
#pragma unroll
  for (int m = 0; m < 16; ++m)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[m][v] = 0.0f;
  u32x4 r[kLoads];
  // Step it's 64 KB: slot q * kThreads + tid of the stage (each wave's
  // instruction q fills 64 consecutive slots, as the GEMM's DMA does).
  auto issue = [&](int it, int buf) __attribute__((always_inline)) {
    const uint32_t base = (uint32_t)(((int)blockIdx.x + it) % kSrcSteps) * kStageBytes;
#pragma unroll
    for (int q = 0; q < kLoads; ++q) {
      const uint32_t off = base + (uint32_t)(q * kThreads + tid) * 16u;
      if constexpr (DMA)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rs, (lds_void *)(&ring[buf][(q * 4 + wave) * 64]), 16, off, 0, 0, 0);
      else
        r[q] = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
    }
  };
  issue(0, 0);
  if constexpr (!DMA) {
#pragma unroll
    for (int q = 0; q < kLoads; ++q) ring[0][q * kThreads + tid] = r[q];
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  int cur = 0;
  for (int it = 0; it < iters; ++it) {
    const int nxt = cur ^ 1;
    issue(it + 1, nxt);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      u32x4 fr[8];
#pragma unroll
      for (int f = 0; f < 8; ++f)
        fr[f] = (MODE == 2 && f >= 4) ? frag_tr(ring[cur], f - 4, kk, lane, wave)
                                      : ring[cur][frag_slot(f, kk, lane, wave)];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i * 4 + j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(bf16x8, fr[4 + j]), __builtin_bit_cast(bf16x8, fr[i]),
              acc[i * 4 + j], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (!DMA) {
#pragma unroll
      for (int q = 0; q < kLoads; ++q) ring[nxt][q * kThreads + tid] = r[q];
    }
    __builtin_amdgcn_s_waitcnt(0);  // the step's loads (and LDS writes) done
    __syncthreads();
    cur = nxt;
  }
  float s = 0.0f;
#pragma unroll
  for (int m = 0; m < 16; ++m)
#pragma unroll
    for (int v = 0; v < 16; ++v) s += acc[m][v];
  out[blockIdx.x * kThreads + tid] = s;
}
}  // namespace

// src: kSrcBytes (2 MiB) of bf16 operands, 16-byte aligned; out: grid * 256
// floats; dma: 1 the LDS-DMA path, 0 the register-staged one, 2 LDS-DMA with
// transposing B fragment reads.
// FLOP per launch: grid * 4 waves * iters * 64 * 32768 (through *flop).
// Returns a hipError_t.
extern "C" int nova_probe_stage(const void *src, float *out, int grid, int iters, int dma,
                                void *stream, double *flop) {
  if (!src || !out || grid <= 0 || iters <= 0 || (reinterpret_cast<uintptr_t>(src) & 15u))
    return (int)hipErrorInvalidValue;
  const u32x4 *s = static_cast<const u32x4 *>(src);
  if (dma == 2)
    hipLaunchKernelGGL(stage_loop<2>, dim3(grid), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), s, out, iters);
  else if (dma)
    hipLaunchKernelGGL(stage_loop<0>, dim3(grid), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), s, out, iters);
  else
    hipLaunchKernelGGL(stage_loop<1>, dim3(grid), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), s, out, iters);
  if (flop) *flop = (double)grid * 4 * iters * 64 * 32768.0;
  return (int)hipGetLastError();
}

// Bytes of source nova_probe_stage reads (its `src` must hold this many).
extern "C" int64_t nova_probe_stage_src_bytes() { return kSrcBytes; }
