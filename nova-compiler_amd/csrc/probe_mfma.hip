// Measurement probe for bench.py --telemetry (not part of the op path): a
// loop of nothing but v_mfma_f32_32x32x16_bf16 on random non-zero register
// operands, eight independent accumulators per wave, no memory traffic.
// Under the board's power limit it gives the MFMA ceiling that the GEMM
// kernels' data movement is measured against.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kAcc = 8;

__global__ __launch_bounds__(256) void mfma_loop(float *out, int iters, uint32_t seed) {
  const int lane = threadIdx.x;
  uint32_t x = seed ^ (lane * 2654435761u) ^ (blockIdx.x * 40503u);
  u32x4 a, b;
  // bf16 values in [0.5, 1) with random mantissas and signs
  for (int i = 0; i < 4; ++i) {
    x = x * 1664525u + 1013904223u;
    const uint32_t lo = (x >> 9) | 0x3f000000u;
    x = x * 1664525u + 1013904223u;
    const uint32_t hi = (x >> 9) | 0x3f000000u;
    x = x * 1664525u + 1013904223u;
    a[i] = (lo >> 16) | (hi & 0xffff0000u) | ((x & 1u) << 15);
    b[i] = (hi >> 16) | (lo & 0xffff0000u) | ((x & 2u) << 30);
  }
  f32x16 acc[kAcc];
  for (int j = 0; j < kAcc; ++j)
    for (int v = 0; v < 16; ++v) acc[j][v] = 0.f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < kAcc; ++j)
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), acc[j], 0,
                                                       0, 0);
  }
  float s = 0.f;
  for (int j = 0; j < kAcc; ++j)
    for (int v = 0; v < 16; ++v) s += acc[j][v];
  out[blockIdx.x * 256 + lane] = s;
}

// The same loop on v_mfma_f32_16x16x32_bf16 (half the accumulator bytes per
// FLOP, twice the operand bytes): sixteen independent 16x16 accumulators.
constexpr int kAcc16 = 16;
typedef float f32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void mfma_loop16(float *out, int iters, uint32_t seed) {
  const int lane = threadIdx.x;
  uint32_t x = seed ^ (lane * 2654435761u) ^ (blockIdx.x * 40503u);
  u32x4 a, b;
  for (int i = 0; i < 4; ++i) {
    x = x * 1664525u + 1013904223u;
    const uint32_t lo = (x >> 9) | 0x3f000000u;
    x = x * 1664525u + 1013904223u;
    const uint32_t hi = (x >> 9) | 0x3f000000u;
    x = x * 1664525u + 1013904223u;
    a[i] = (lo >> 16) | (hi & 0xffff0000u) | ((x & 1u) << 15);
    b[i] = (hi >> 16) | (lo & 0xffff0000u) | ((x & 2u) << 30);
  }
  f32x4 acc[kAcc16];
  for (int j = 0; j < kAcc16; ++j)
    for (int v = 0; v < 4; ++v) acc[j][v] = 0.f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < kAcc16; ++j)
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), acc[j], 0,
                                                       0, 0);
  }
  float s = 0.f;
  for (int j = 0; j < kAcc16; ++j)
    for (int v = 0; v < 4; ++v) s += acc[j][v];
  out[blockIdx.x * 256 + lane] = s;
}
}  // namespace

// 16x16x32 form of nova_probe_mfma_loop: FLOP per launch grid * 4 waves *
// iters * 16 * 16384.
extern "C" int nova_probe_mfma_loop16(float *out, int grid, int iters, void *stream, double *flop) {
  if (grid <= 0 || iters <= 0 || !out) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(mfma_loop16, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream), out,
                     iters, 12345u);
  if (flop) *flop = (double)grid * 4 * iters * kAcc16 * 16384.0;
  return (int)hipGetLastError();
}

// out: grid * 256 floats.  FLOP per launch: grid * 4 waves * iters * kAcc *
// 32768 (returned through *flop).  Returns a hipError_t.
extern "C" int nova_probe_mfma_loop(float *out, int grid, int iters, void *stream, double *flop) {
  if (grid <= 0 || iters <= 0 || !out) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(mfma_loop, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream), out,
                     iters, 12345u);
  if (flop) *flop = (double)grid * 4 * iters * kAcc * 32768.0;
  return (int)hipGetLastError();
}
