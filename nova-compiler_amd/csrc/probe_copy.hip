// Measurement probe for bench.py (not part of the op path): the practical
// HBM read+write ceiling the reductions are compared with.  A plain copy,
// one 16-byte element per thread, nontemporal loads and stores, one
// workgroup per 4 KB: of the copy forms timed on MI355X (grid-stride loops
// with 1-8 elements in flight per thread, a contiguous block per workgroup,
// plain or nontemporal accesses, torch's copy) this one moved the most
// bytes per second (6.64 TB/s over 2 x 256 MiB, against 5.4 for torch's).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {
typedef float f32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void copy16(const f32x4 *x, f32x4 *y, int64_t n16) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n16) __builtin_nontemporal_store(__builtin_nontemporal_load(x + i), y + i);
}
}  // namespace

// Copy `bytes` (a multiple of 16; x and y 16-byte aligned) from x to y on
// `stream`.  Returns a hipError_t.
extern "C" int nova_probe_copy(const void *x, void *y, int64_t bytes, void *stream) {
  if (!x || !y || bytes <= 0 || bytes % 16 || (reinterpret_cast<uintptr_t>(x) & 15u) ||
      (reinterpret_cast<uintptr_t>(y) & 15u))
    return (int)hipErrorInvalidValue;
  const int64_t n16 = bytes / 16, grid = (n16 + 255) / 256;
  if (grid > 0x7fffffff) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(copy16, dim3((unsigned)grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const f32x4 *>(x), static_cast<f32x4 *>(y), n16);
  return (int)hipGetLastError();
}
