// Program-glue ops for gfx950: the elementwise, index and reduction ops a
// whole Nova training step needs around the GEMMs and row reductions
// (nova.add / sub / mul / div with broadcasting, a splat nova.constant,
// nova.gelu and nova.gelu_backward, nova.gather, nova.scatter_add,
// nova.reduce<sum>, and the widening of narrow label / index types).  All
// are HBM-bound streams: 16-byte loads and stores where the operands are
// dense and aligned, a general strided form otherwise.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "nova_hip_internal.h"

namespace nova_hip {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;

unsigned blocks_for(int64_t n, int64_t per_block, int64_t cap = 65536) {
  const int64_t b = (n + per_block - 1) / per_block;
  return (unsigned)(b < 1 ? 1 : (b > cap ? cap : b));
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---------------------------------------------------------------------------
// Binary ops (Nova_BinaryOp, NovaOps.td:600-700): one IEEE operation per
// element, operands broadcast numpy-style (a stride of 0 on a broadcast
// dimension).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float apply(float x, float y, int op) {
  switch (op) {
    case NOVA_HIP_BIN_ADD: return x + y;
    case NOVA_HIP_BIN_SUB: return x - y;
    case NOVA_HIP_BIN_MUL: return x * y;
    default: return x / y;
  }
}

template <int OP>
__global__ __launch_bounds__(kThreads) void binary_dense_kernel(const f32x4 *a, const f32x4 *b,
                                                                f32x4 *c, int64_t n4) {
  for (int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x; i < n4;
       i += (int64_t)gridDim.x * kThreads) {
    const f32x4 x = __builtin_nontemporal_load(a + i), y = __builtin_nontemporal_load(b + i);
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = apply(x[e], y[e], OP);
    __builtin_nontemporal_store(o, c + i);
  }
}

// One operand a scalar (the nova.mul by a [1] constant of a loss scale).
template <int OP, bool SCALAR_B>
__global__ __launch_bounds__(kThreads) void binary_scalar_kernel(const f32x4 *v, const float *s,
                                                                 f32x4 *c, int64_t n4) {
  const float k = *s;
  for (int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x; i < n4;
       i += (int64_t)gridDim.x * kThreads) {
    const f32x4 x = __builtin_nontemporal_load(v + i);
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = SCALAR_B ? apply(x[e], k, OP) : apply(k, x[e], OP);
    __builtin_nontemporal_store(o, c + i);
  }
}

// One operand repeating over leading dims (the [B,T,D] + [1,T,D] add of a
// position embedding): the dense operand v with n4 float4s, the repeating
// one r with period p4 float4s, v-side op order kept by SWAP.
template <int OP, bool SWAP>
__global__ __launch_bounds__(kThreads) void binary_periodic_kernel(const f32x4 *v, const f32x4 *r,
                                                                   f32x4 *c, int64_t n4,
                                                                   int64_t p4) {
  for (int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x; i < n4;
       i += (int64_t)gridDim.x * kThreads) {
    const f32x4 x = __builtin_nontemporal_load(v + i), y = r[i % p4];
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = SWAP ? apply(y[e], x[e], OP) : apply(x[e], y[e], OP);
    __builtin_nontemporal_store(o, c + i);
  }
}

__global__ __launch_bounds__(kThreads) void binary_strided_kernel(BinaryProblem p) {
  const int64_t n = p.size[0] * p.size[1] * p.size[2] * p.size[3];
  for (int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads) {
    int64_t r = i;
    const int64_t i3 = r % p.size[3];
    r /= p.size[3];
    const int64_t i2 = r % p.size[2];
    r /= p.size[2];
    const int64_t i1 = r % p.size[1];
    const int64_t i0 = r / p.size[1];
    const float x = p.a[i0 * p.sa[0] + i1 * p.sa[1] + i2 * p.sa[2] + i3 * p.sa[3]];
    const float y = p.b[i0 * p.sb[0] + i1 * p.sb[1] + i2 * p.sb[2] + i3 * p.sb[3]];
    p.c[i0 * p.sc[0] + i1 * p.sc[1] + i2 * p.sc[2] + i3 * p.sc[3]] = apply(x, y, p.op);
  }
}

bool dense4(const int64_t *size, const int64_t *st) {
  int64_t want = 1;
  for (int d = 3; d >= 0; --d) {
    if (size[d] != 1 && st[d] != want) return false;
    want *= size[d];
  }
  return true;
}

// Operand strides that repeat a dense block over the leading dims: 0 on
// dims d < k, dense (c's own strides) on d >= k, for some k.  The period in
// elements, or 0 if the strides are not of that form.
int64_t period_of(const int64_t *size, const int64_t *st) {
  int64_t want = 1;
  int d = 3;
  for (; d >= 0; --d) {
    if (size[d] == 1) continue;
    if (st[d] != want) break;
    want *= size[d];
  }
  for (; d >= 0; --d)
    if (size[d] != 1 && st[d] != 0) return 0;
  return want;
}

bool all_zero(const int64_t *size, const int64_t *st) {
  for (int d = 0; d < 4; ++d)
    if (size[d] != 1 && st[d] != 0) return false;
  return true;
}

template <int OP>
void launch_binary_op(const BinaryProblem &p, int64_t n, hipStream_t s) {
  const bool dc = dense4(p.size, p.sc) && aligned16(p.c) && n % 4 == 0;
  const bool da = dense4(p.size, p.sa) && aligned16(p.a);
  const bool db = dense4(p.size, p.sb) && aligned16(p.b);
  const unsigned g = blocks_for(n / 4, kThreads * 4, 16384);
  if (dc && da && db) {
    hipLaunchKernelGGL(binary_dense_kernel<OP>, dim3(g), dim3(kThreads), 0, s,
                       reinterpret_cast<const f32x4 *>(p.a), reinterpret_cast<const f32x4 *>(p.b),
                       reinterpret_cast<f32x4 *>(p.c), n / 4);
  } else if (dc && da && all_zero(p.size, p.sb)) {
    hipLaunchKernelGGL((binary_scalar_kernel<OP, true>), dim3(g), dim3(kThreads), 0, s,
                       reinterpret_cast<const f32x4 *>(p.a), p.b, reinterpret_cast<f32x4 *>(p.c),
                       n / 4);
  } else if (dc && db && all_zero(p.size, p.sa)) {
    hipLaunchKernelGGL((binary_scalar_kernel<OP, false>), dim3(g), dim3(kThreads), 0, s,
                       reinterpret_cast<const f32x4 *>(p.b), p.a, reinterpret_cast<f32x4 *>(p.c),
                       n / 4);
  } else if (dc && da && aligned16(p.b) && period_of(p.size, p.sb) % 4 == 0 &&
             period_of(p.size, p.sb) > 0) {
    hipLaunchKernelGGL((binary_periodic_kernel<OP, false>), dim3(g), dim3(kThreads), 0, s,
                       reinterpret_cast<const f32x4 *>(p.a), reinterpret_cast<const f32x4 *>(p.b),
                       reinterpret_cast<f32x4 *>(p.c), n / 4, period_of(p.size, p.sb) / 4);
  } else if (dc && db && aligned16(p.a) && period_of(p.size, p.sa) % 4 == 0 &&
             period_of(p.size, p.sa) > 0) {
    hipLaunchKernelGGL((binary_periodic_kernel<OP, true>), dim3(g), dim3(kThreads), 0, s,
                       reinterpret_cast<const f32x4 *>(p.b), reinterpret_cast<const f32x4 *>(p.a),
                       reinterpret_cast<f32x4 *>(p.c), n / 4, period_of(p.size, p.sa) / 4);
  } else {
    hipLaunchKernelGGL(binary_strided_kernel, dim3(blocks_for(n, kThreads * 4, 16384)),
                       dim3(kThreads), 0, s, p);
  }
}

// ---------------------------------------------------------------------------
// Fill (a splat nova.constant, NovaOps.td:331).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void fill_kernel(float *out, int64_t n, int64_t stride,
                                                        float v) {
  for (int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads)
    out[i * stride] = v;
}

__global__ __launch_bounds__(kThreads) void fill4_kernel(f32x4 *out, int64_t n4, float v) {
  for (int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x; i < n4;
       i += (int64_t)gridDim.x * kThreads)
    __builtin_nontemporal_store(f32x4{v, v, v, v}, out + i);
}

// ---------------------------------------------------------------------------
// GELU (NovaGeluForwardPattern, NovaToLinalgGeneric.cpp:1277-1337) and its
// backward (NovaGeluBackwardPattern, :1339-1425), in the reference's
// operation order with no contraction; tanh is the device library's tanhf.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float gelu_ref(float x) {
#pragma clang fp contract(off)
  const float x2 = x * x;
  const float x3 = x2 * x;
  const float c = 0.044715f * x3;
  const float in = x + c;
  const float sc = 0.7978845608028654f * in;
  const float t = tanhf(sc);
  const float hx = 0.5f * x;
  return hx * (1.0f + t);
}

__device__ __forceinline__ float gelu_bwd_ref(float go, float x) {
#pragma clang fp contract(off)
  const float k = 0.797884583f;
  const float x2 = x * x;
  const float x3 = x2 * x;
  const float cubic = 4.471500e-02f * x3;
  const float inner = x + cubic;
  const float gx = k * inner;
  const float xsq_c = x2 * 0.134145f;
  const float poly = 1.0f + xsq_c;
  const float dgx = poly * k;
  const float th = tanhf(gx);
  const float th2 = th * th;
  const float term1 = 0.5f * (1.0f + th);
  const float om = 1.0f - th2;
  const float t2a = dgx * om;
  const float t2b = x * t2a;
  const float term2 = 0.5f * t2b;
  return go * (term1 + term2);
}

__global__ __launch_bounds__(kThreads) void gelu_kernel(const float *x, float *y, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads)
    y[i] = gelu_ref(x[i]);
}

__global__ __launch_bounds__(kThreads) void gelu_bwd_kernel(const float *go, const float *x,
                                                            float *out, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads)
    out[i] = gelu_bwd_ref(go[i], x[i]);
}

// ---------------------------------------------------------------------------
// Index loads: narrow integers zero-extended (NovaToLinalgGeneric.cpp:
// 2434-2449, NovaToLinalg.cpp:1240-1244), i64 taken as a signed index.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int64_t load_index(const void *idx, int64_t i, int dt) {
  if (dt == NOVA_HIP_DT_I16) return (int64_t)static_cast<const uint16_t *>(idx)[i];
  if (dt == NOVA_HIP_DT_I32) return (int64_t)static_cast<const int32_t *>(idx)[i];
  return static_cast<const int64_t *>(idx)[i];
}

// nova.gather along axis 0 (NovaGatherOpLowering, NovaToLinalgGeneric.cpp:
// 2372-2471): out[i, :] = table[idx[i], :].  An index outside the table
// (undefined in the reference's tensor.extract) gives a NaN row.
__global__ __launch_bounds__(kThreads) void gather_kernel(GatherProblem p) {
  const int64_t i = blockIdx.y;
  const int64_t r = load_index(p.idx, i * p.sidx, p.idx_dt);
  const bool ok = r >= 0 && r < p.rows;
  const float *src = p.table + (ok ? r : 0) * p.st;
  float *dst = p.out + i * p.so;
  for (int64_t c = blockIdx.x * (int64_t)kThreads + threadIdx.x; c < p.D;
       c += (int64_t)gridDim.x * kThreads)
    dst[c] = ok ? src[c] : __builtin_nanf("");
}

// nova.scatter_add along axis 0 (NovaScatterAddOpLowering, NovaToLinalg.cpp:
// 1086-1290): out[idx[i], :] += src[i, :] by f32 atomic adds, as the
// reference's memref.atomic_rmw addf; an index outside [0, rows) is
// skipped (its scf.if bounds check).  The order of the adds into one row is
// the hardware's, as in the reference's GPU lowering.
__global__ __launch_bounds__(kThreads) void scatter_add_kernel(ScatterAddProblem p) {
  const int64_t i = blockIdx.y;
  const int64_t r = load_index(p.idx, i * p.sidx, p.idx_dt);
  if (r < 0 || r >= p.rows) return;
  const float *src = p.src + i * p.ss;
  float *dst = p.out + r * p.so;
  for (int64_t c = blockIdx.x * (int64_t)kThreads + threadIdx.x; c < p.D;
       c += (int64_t)gridDim.x * kThreads)
    unsafeAtomicAdd(dst + c, src[c]);
}

// Labels / indices to i32 (NovaSceForwardLowering zero-extends non-i32
// labels, NovaToLinalgGeneric.cpp:801-1010; i64 is truncated).
__global__ __launch_bounds__(kThreads) void index_to_i32_kernel(const void *src, int64_t stride,
                                                                int dt, int32_t *dst, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads)
    dst[i] = (int32_t)load_index(src, i * stride, dt);
}

// ---------------------------------------------------------------------------
// nova.reduce<sum> over one dimension: x viewed as [outer, n, inner],
// out[o, i] = sum_j x[o, j, i], j ascending (the linalg.reduce order of the
// reference's lowering).  Thread per (o, i); a thread's loads go out 16 at a
// time before the in-order adds.
// ---------------------------------------------------------------------------
constexpr int kRedBatch = 16;

__global__ __launch_bounds__(kThreads) void reduce_sum_kernel(ReduceSumProblem p) {
  const int64_t total = p.outer * p.inner;
  for (int64_t t = blockIdx.x * (int64_t)kThreads + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * kThreads) {
    const int64_t o = t / p.inner, i = t - o * p.inner;
    const float *x = p.x + o * p.so + i * p.si;
    float acc = 0.0f;
    int64_t j = 0;
    for (; j + kRedBatch <= p.n; j += kRedBatch) {
      float v[kRedBatch];
#pragma unroll
      for (int u = 0; u < kRedBatch; ++u) v[u] = x[(j + u) * p.sn];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < kRedBatch; ++u) acc = acc + v[u];
    }
    for (; j < p.n; ++j) acc = acc + x[j * p.sn];
    p.out[o * p.soo + i * p.soi] = acc;
  }
}

}  // namespace

int32_t launch_binary(const BinaryProblem &p, hipStream_t s) {
  const int64_t n = p.size[0] * p.size[1] * p.size[2] * p.size[3];
  if (n == 0) return NOVA_HIP_SUCCESS;
  switch (p.op) {
    case NOVA_HIP_BIN_ADD: launch_binary_op<NOVA_HIP_BIN_ADD>(p, n, s); break;
    case NOVA_HIP_BIN_SUB: launch_binary_op<NOVA_HIP_BIN_SUB>(p, n, s); break;
    case NOVA_HIP_BIN_MUL: launch_binary_op<NOVA_HIP_BIN_MUL>(p, n, s); break;
    default: launch_binary_op<NOVA_HIP_BIN_DIV>(p, n, s); break;
  }
  return check_hip(hipGetLastError(), "binary launch");
}

int32_t launch_fill(float *out, int64_t n, int64_t stride, float v, hipStream_t s) {
  if (n == 0) return NOVA_HIP_SUCCESS;
  if (stride == 1 && aligned16(out) && n % 4 == 0)
    hipLaunchKernelGGL(fill4_kernel, dim3(blocks_for(n / 4, kThreads * 4, 16384)), dim3(kThreads),
                       0, s, reinterpret_cast<f32x4 *>(out), n / 4, v);
  else
    hipLaunchKernelGGL(fill_kernel, dim3(blocks_for(n, kThreads * 4, 16384)), dim3(kThreads), 0,
                       s, out, n, stride, v);
  return check_hip(hipGetLastError(), "fill launch");
}

int32_t launch_gelu(const float *x, float *y, int64_t n, hipStream_t s) {
  if (n == 0) return NOVA_HIP_SUCCESS;
  hipLaunchKernelGGL(gelu_kernel, dim3(blocks_for(n, kThreads * 4, 16384)), dim3(kThreads), 0, s,
                     x, y, n);
  return check_hip(hipGetLastError(), "gelu launch");
}

int32_t launch_gelu_backward(const float *go, const float *x, float *out, int64_t n,
                             hipStream_t s) {
  if (n == 0) return NOVA_HIP_SUCCESS;
  hipLaunchKernelGGL(gelu_bwd_kernel, dim3(blocks_for(n, kThreads * 4, 16384)), dim3(kThreads),
                     0, s, go, x, out, n);
  return check_hip(hipGetLastError(), "gelu_backward launch");
}

int32_t launch_gather(const GatherProblem &p, hipStream_t s) {
  if (p.n == 0 || p.D == 0) return NOVA_HIP_SUCCESS;
  if (p.n > 65535) {
    // One launch per 65535 indices (grid.y limit).
    for (int64_t i0 = 0; i0 < p.n; i0 += 65535) {
      GatherProblem q = p;
      q.n = p.n - i0 < 65535 ? p.n - i0 : 65535;
      q.idx = static_cast<const char *>(p.idx) +
              i0 * p.sidx * (p.idx_dt == NOVA_HIP_DT_I16 ? 2 : p.idx_dt == NOVA_HIP_DT_I32 ? 4 : 8);
      q.out = p.out + i0 * p.so;
      int32_t rc = launch_gather(q, s);
      if (rc) return rc;
    }
    return NOVA_HIP_SUCCESS;
  }
  hipLaunchKernelGGL(gather_kernel, dim3(blocks_for(p.D, kThreads, 64), (unsigned)p.n),
                     dim3(kThreads), 0, s, p);
  return check_hip(hipGetLastError(), "gather launch");
}

int32_t launch_scatter_add(const ScatterAddProblem &p, hipStream_t s) {
  if (p.n == 0 || p.D == 0) return NOVA_HIP_SUCCESS;
  if (p.n > 65535) {
    for (int64_t i0 = 0; i0 < p.n; i0 += 65535) {
      ScatterAddProblem q = p;
      q.n = p.n - i0 < 65535 ? p.n - i0 : 65535;
      q.idx = static_cast<const char *>(p.idx) +
              i0 * p.sidx * (p.idx_dt == NOVA_HIP_DT_I16 ? 2 : p.idx_dt == NOVA_HIP_DT_I32 ? 4 : 8);
      q.src = p.src + i0 * p.ss;
      int32_t rc = launch_scatter_add(q, s);
      if (rc) return rc;
    }
    return NOVA_HIP_SUCCESS;
  }
  hipLaunchKernelGGL(scatter_add_kernel, dim3(blocks_for(p.D, kThreads, 64), (unsigned)p.n),
                     dim3(kThreads), 0, s, p);
  return check_hip(hipGetLastError(), "scatter_add launch");
}

int32_t launch_index_to_i32(const void *src, int64_t stride, int dt, int32_t *dst, int64_t n,
                            hipStream_t s) {
  if (n == 0) return NOVA_HIP_SUCCESS;
  hipLaunchKernelGGL(index_to_i32_kernel, dim3(blocks_for(n, kThreads * 4, 16384)),
                     dim3(kThreads), 0, s, src, stride, dt, dst, n);
  return check_hip(hipGetLastError(), "index_to_i32 launch");
}

int32_t launch_reduce_sum(const ReduceSumProblem &p, hipStream_t s) {
  const int64_t total = p.outer * p.inner;
  if (total == 0) return NOVA_HIP_SUCCESS;
  hipLaunchKernelGGL(reduce_sum_kernel, dim3(blocks_for(total, kThreads, 16384)), dim3(kThreads),
                     0, s, p);
  return check_hip(hipGetLastError(), "reduce_sum launch");
}

}  // namespace nova_hip
