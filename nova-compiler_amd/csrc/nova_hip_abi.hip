// C ABI of libnova_hip: descriptor validation, flag decoding, per-thread
// stream and error text, and the per-stream workspace cache.  Every check
// here runs on the host before any HIP call, so malformed calls fail with a
// status code instead of reaching a kernel.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <memory>
#include <unordered_map>
#include <vector>

#include "nova_hip_internal.h"

namespace nova_hip {

namespace {
thread_local char t_err[512] = {0};
thread_local hipStream_t t_stream = nullptr;

struct Workspace {
  void *ptr = nullptr;
  size_t bytes = 0;
};
std::mutex g_ws_mu;
std::unordered_map<hipStream_t, Workspace> g_ws;

// One enqueue mutex per stream, never erased (a later stream with a
// recycled handle shares it, which only serialises more).  Lock order: a
// stream's mutex, then g_ws_mu.
std::mutex g_stream_mu_mu;
std::unordered_map<hipStream_t, std::unique_ptr<std::mutex>> g_stream_mu;

std::mutex &stream_mutex(hipStream_t s) {
  std::lock_guard<std::mutex> lock(g_stream_mu_mu);
  std::unique_ptr<std::mutex> &m = g_stream_mu[s];
  if (!m) m.reset(new std::mutex);
  return *m;
}
}  // namespace

int32_t fail(int32_t code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(t_err, sizeof(t_err), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { t_err[0] = 0; }

hipStream_t current_stream() { return t_stream; }

namespace {
// A device attribute of the current device, queried once per device.
int cached_attribute(std::atomic<int> *cache, int n, hipDeviceAttribute_t attr) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < n) {
    const int c = cache[dev].load(std::memory_order_relaxed);  // 0: not queried yet
    if (c) return c > 0 ? c : 0;
  }
  int v = 0;
  if (hipDeviceGetAttribute(&v, attr, dev) != hipSuccess) v = 0;
  if (dev < n) cache[dev].store(v > 0 ? v : -1, std::memory_order_relaxed);
  return v > 0 ? v : 0;
}
constexpr int kMaxDevices = 64;
}  // namespace

int device_cu_count() {
  static std::atomic<int> cache[kMaxDevices];
  return cached_attribute(cache, kMaxDevices, hipDeviceAttributeMultiprocessorCount);
}

int device_lds_per_block() {
  static std::atomic<int> cache[kMaxDevices];
  return cached_attribute(cache, kMaxDevices, hipDeviceAttributeMaxSharedMemoryPerBlock);
}

int32_t check_hip(hipError_t e, const char *what) {
  if (e == hipSuccess) return NOVA_HIP_SUCCESS;
  return fail(NOVA_HIP_EDEVICE, "%s: %s", what, hipGetErrorString(e));
}

namespace {
// The stream's buffer, grown to at least `bytes`; the caller holds the
// stream's mutex.
void *workspace_locked(hipStream_t s, size_t bytes) {
  std::lock_guard<std::mutex> lock(g_ws_mu);
  Workspace &w = g_ws[s];
  if (w.bytes >= bytes && w.ptr) return w.ptr;
  if (w.ptr) {
    // The old buffer may still be read by queued work on this stream.
    hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
      check_hip(e, "workspace: stream synchronize");
      return nullptr;
    }
    (void)hipFree(w.ptr);
    w.ptr = nullptr;
    w.bytes = 0;
  }
  size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, want);
  if (e != hipSuccess) {
    fail(NOVA_HIP_ENOMEM, "workspace: hipMalloc(%zu): %s", want, hipGetErrorString(e));
    return nullptr;
  }
  w.ptr = p;
  w.bytes = want;
  return p;
}
}  // namespace

void *WorkspaceLease::acquire(hipStream_t s, size_t bytes) {
  lock_ = std::unique_lock<std::mutex>(stream_mutex(s));
  ptr_ = workspace_locked(s, bytes);
  return ptr_;
}

namespace {

// ---- descriptor helpers ----------------------------------------------------
template <typename D>
const char *data_of(const D *d) {
  return static_cast<const char *>(d->aligned);
}

template <typename D>
bool nonneg_sizes(const D *d, int rank) {
  for (int i = 0; i < rank; ++i)
    if (d->sizes[i] < 0) return false;
  return true;
}

int decode_flags(int32_t flags, int &in_dt, int &out_dt, int &epi, int &bias_dt) {
  if (flags & ~(0xffff | NOVA_HIP_GEMM_ACC_OUT | NOVA_HIP_GEMM_F32_MFMA | NOVA_HIP_GEMM_ACC_C))
    return fail(NOVA_HIP_EINVAL, "gemm: unknown flag bits 0x%x", flags);
  in_dt = flags & 0xf;
  out_dt = (flags >> 4) & 0xf;
  epi = (flags >> 8) & 0xf;
  bias_dt = (flags >> 12) & 0xf;
  if (in_dt > NOVA_HIP_DT_F16 || out_dt > NOVA_HIP_DT_F16 || bias_dt > NOVA_HIP_DT_F16 ||
      epi > NOVA_HIP_EPI_GELU)
    return fail(NOVA_HIP_EDTYPE, "gemm: bad dtype/epilogue code in flags 0x%x", flags);
  if (in_dt == NOVA_HIP_DT_F32 && out_dt != NOVA_HIP_DT_F32)
    return fail(NOVA_HIP_EDTYPE, "gemm: f32 inputs produce f32 output only");
  if ((flags & NOVA_HIP_GEMM_F32_MFMA) && (in_dt != NOVA_HIP_DT_F32 || (flags & NOVA_HIP_GEMM_ACC_OUT)))
    return fail(NOVA_HIP_EDTYPE, "gemm: the f32 MFMA form takes f32 operands");
  if (flags & NOVA_HIP_GEMM_ACC_OUT) {
    if (in_dt == NOVA_HIP_DT_F32 || out_dt != in_dt)
      return fail(NOVA_HIP_EDTYPE,
                  "gemm: accumulating in the output dtype needs bf16 or f16 inputs of that dtype");
    if (epi == NOVA_HIP_EPI_GELU || epi == NOVA_HIP_EPI_BIAS_GELU ||
        (epi == NOVA_HIP_EPI_BIAS && bias_dt != out_dt))
      return fail(NOVA_HIP_EDTYPE,
                  "gemm: a bf16 / f16 accumulator takes no GELU, and a bias of its own dtype only");
  }
  if (flags & NOVA_HIP_GEMM_ACC_C) {
    // Accumulating into C's data runs on the exact kernel: f32, or a 16-bit
    // accumulator of the operands' own type.
    if (flags & NOVA_HIP_GEMM_F32_MFMA)
      return fail(NOVA_HIP_EINVAL, "gemm: accumulating into C is not an f32 MFMA form");
    if (in_dt != NOVA_HIP_DT_F32 && !(flags & NOVA_HIP_GEMM_ACC_OUT))
      return fail(NOVA_HIP_EDTYPE,
                  "gemm: accumulating into C needs f32 operands, or 16-bit ones with "
                  "NOVA_HIP_GEMM_ACC_OUT");
    if (epi != NOVA_HIP_EPI_NONE)
      return fail(NOVA_HIP_EINVAL, "gemm: accumulating into C takes no epilogue");
  }
  return NOVA_HIP_SUCCESS;
}

// Validate and normalise a batched GEMM given 3-D views, then launch it
// (with launch false: validate only, so that an entry point with several
// outputs can check them all before it writes any).
int32_t gemm_core(const NovaMemRef3D *A, const NovaMemRef3D *B, NovaMemRef3D *C,
                  const NovaMemRef1D *bias, int32_t flags, bool launch = true) {
  clear_error();
  if (!A || !B || !C) return fail(NOVA_HIP_EINVAL, "gemm: null descriptor");
  int in_dt, out_dt, epi, bias_dt;
  int32_t rc = decode_flags(flags, in_dt, out_dt, epi, bias_dt);
  if (rc) return rc;
  if (!nonneg_sizes(A, 3) || !nonneg_sizes(B, 3) || !nonneg_sizes(C, 3))
    return fail(NOVA_HIP_ESHAPE, "gemm: negative size");
  const int64_t batch = C->sizes[0], M = C->sizes[1], N = C->sizes[2];
  const int64_t K = A->sizes[2];
  if (A->sizes[1] != M || B->sizes[2] != N || B->sizes[1] != K)
    return fail(NOVA_HIP_ESHAPE,
                "gemm: shapes A[%lld,%lld,%lld] B[%lld,%lld,%lld] C[%lld,%lld,%lld] disagree",
                (long long)A->sizes[0], (long long)A->sizes[1], (long long)A->sizes[2],
                (long long)B->sizes[0], (long long)B->sizes[1], (long long)B->sizes[2],
                (long long)batch, (long long)M, (long long)N);
  // Batch: equal, or 1 with any stride (broadcast a rank-2 operand).
  if ((A->sizes[0] != batch && A->sizes[0] != 1) || (B->sizes[0] != batch && B->sizes[0] != 1))
    return fail(NOVA_HIP_ESHAPE, "gemm: batch sizes %lld/%lld do not broadcast to %lld",
                (long long)A->sizes[0], (long long)B->sizes[0], (long long)batch);
  const bool has_bias = (epi == NOVA_HIP_EPI_BIAS || epi == NOVA_HIP_EPI_BIAS_GELU);
  if (has_bias) {
    if (!bias || !bias->aligned) return fail(NOVA_HIP_EINVAL, "gemm: epilogue needs a bias");
    if (bias->sizes[0] != N) return fail(NOVA_HIP_ESHAPE, "gemm: bias size %lld != N %lld",
                                         (long long)bias->sizes[0], (long long)N);
    if (bias->strides[0] != 1 && N > 1) return fail(NOVA_HIP_ESTRIDE, "gemm: bias must be contiguous");
  }
  const bool empty = batch == 0 || M == 0 || N == 0;
  // With K == 0 the operands hold no elements (their data pointer may be
  // null) and C is just the epilogue of a zero accumulator.
  if (!empty && (!C->aligned || (K > 0 && (!A->aligned || !B->aligned))))
    return fail(NOVA_HIP_EINVAL, "gemm: null data pointer");

  GemmProblem p;
  p.batch = batch;
  p.M = M;
  p.N = N;
  p.K = K;
  p.in_dt = in_dt;
  p.out_dt = out_dt;
  p.epi = epi;
  p.bias_dt = bias_dt;
  p.acc_out = (flags & NOVA_HIP_GEMM_ACC_OUT) != 0;
  p.f32_mfma = (flags & NOVA_HIP_GEMM_F32_MFMA) != 0;
  p.acc_c = (flags & NOVA_HIP_GEMM_ACC_C) != 0;
  const int esz = dtype_size(in_dt);
  const int osz = dtype_size(out_dt);
  p.A = data_of(A) + A->offset * esz;
  p.B = data_of(B) + B->offset * esz;
  p.C = const_cast<char *>(data_of(C)) + C->offset * osz;
  p.bias = has_bias ? (const void *)(data_of(bias) + bias->offset * dtype_size(bias_dt)) : nullptr;

  // Each operand is addressed as (unit-stride dim, stride of the other dim).
  // A [M,K]: unit stride on K (row-major) or on M (transposed view).  A
  // dim of extent 1 is never stepped, so its stride does not matter.
  const int64_t a_sm = A->strides[1], a_sk = A->strides[2];
  if (a_sk == 1 || K <= 1) {
    p.a_kcontig = true;
    p.sa_outer = a_sm;
  } else if (a_sm == 1 || M <= 1) {
    p.a_kcontig = false;
    p.sa_outer = a_sk;
  } else {
    return fail(NOVA_HIP_ESTRIDE, "gemm: A strides [%lld,%lld] have no unit stride",
                (long long)a_sm, (long long)a_sk);
  }
  // B [K,N]: unit stride on N (row-major) or on K (transposed view, e.g.
  // nova.transpose of a row-major [N,K] weight).
  const int64_t b_sk = B->strides[1], b_sn = B->strides[2];
  if (b_sn == 1 || N <= 1) {
    p.b_kcontig = false;
    p.sb_outer = b_sk;
  } else if (b_sk == 1 || K <= 1) {
    p.b_kcontig = true;
    p.sb_outer = b_sn;
  } else {
    return fail(NOVA_HIP_ESTRIDE, "gemm: B strides [%lld,%lld] have no unit stride",
                (long long)b_sk, (long long)b_sn);
  }
  if (C->strides[2] != 1 && N > 1) return fail(NOVA_HIP_ESTRIDE, "gemm: C must have unit stride on N");
  if (M > 1 && C->strides[1] < N) return fail(NOVA_HIP_ESTRIDE, "gemm: C rows overlap");
  if (p.sa_outer < 0 || p.sb_outer < 0 || C->strides[1] < 0)
    return fail(NOVA_HIP_ESTRIDE, "gemm: negative strides are not addressed");
  p.sab = (A->sizes[0] == 1) ? 0 : A->strides[0];
  p.sbb = (B->sizes[0] == 1) ? 0 : B->strides[0];
  p.scb = C->strides[0];
  p.scm = C->strides[1];
  if (p.sab < 0 || p.sbb < 0 || p.scb < 0)
    return fail(NOVA_HIP_ESTRIDE, "gemm: negative batch stride");
  if (empty || !launch) return NOVA_HIP_SUCCESS;

  hipStream_t s = current_stream();
  if (p.f32_mfma) {
    // An operand slice beyond the 32-bit buffer range takes the exact kernel.
    rc = launch_gemm_f32_mfma(p, s);
    if (rc != NOVA_HIP_ERANGE) return rc;
    clear_error();
  }
  return (in_dt == NOVA_HIP_DT_F32 || p.acc_out) ? launch_gemm_exact(p, s) : launch_gemm_mfma(p, s);
}

NovaMemRef3D lift(const NovaMemRef2D *d) {
  NovaMemRef3D r;
  r.allocated = d->allocated;
  r.aligned = d->aligned;
  r.offset = d->offset;
  r.sizes[0] = 1;
  r.sizes[1] = d->sizes[0];
  r.sizes[2] = d->sizes[1];
  r.strides[0] = 0;
  r.strides[1] = d->strides[0];
  r.strides[2] = d->strides[1];
  return r;
}

int32_t gemm2d(const NovaMemRef2D *A, const NovaMemRef2D *B, NovaMemRef2D *C,
               const NovaMemRef1D *bias, int32_t flags, bool launch = true) {
  if (!A || !B || !C) {
    clear_error();
    return fail(NOVA_HIP_EINVAL, "gemm: null descriptor");
  }
  NovaMemRef3D a = lift(A), b = lift(B), c = lift(C);
  return gemm_core(&a, &b, &c, bias, flags, launch);
}

NovaMemRef2D transposed(const NovaMemRef2D *d) {
  NovaMemRef2D r = *d;
  r.sizes[0] = d->sizes[1];
  r.sizes[1] = d->sizes[0];
  r.strides[0] = d->strides[1];
  r.strides[1] = d->strides[0];
  return r;
}

// C = A . B into C as laid out: row-major C directly; a transposed view of
// a row-major buffer (unit stride on dim 0) as C^T = B^T . A^T into that
// buffer, since the kernels store rows with unit stride.
int32_t gemm2d_to(const NovaMemRef2D *A, const NovaMemRef2D *B, NovaMemRef2D *C, int32_t flags,
                  bool launch = true) {
  if (C && C->strides[1] != 1 && C->sizes[1] > 1 && (C->strides[0] == 1 || C->sizes[0] <= 1)) {
    NovaMemRef2D at = transposed(A), bt = transposed(B), ct = transposed(C);
    return gemm2d(&bt, &at, &ct, nullptr, flags, launch);
  }
  return gemm2d(A, B, C, nullptr, flags, launch);
}

// Flags of the backward GEMM entry points: dtypes only, no epilogue.
int32_t backward_flags(int32_t flags, int &in_dt, int &out_dt, const char *what) {
  if (flags & (NOVA_HIP_GEMM_ACC_OUT | NOVA_HIP_GEMM_ACC_C))
    return fail(NOVA_HIP_EINVAL, "%s: no narrow-accumulator or accumulate-into form (flags 0x%x)",
                what, flags);
  int epi, bias_dt;
  int32_t rc = decode_flags(flags, in_dt, out_dt, epi, bias_dt);
  if (rc) return rc;
  if (epi != NOVA_HIP_EPI_NONE)
    return fail(NOVA_HIP_EINVAL, "%s: flags carry an epilogue (0x%x)", what, flags);
  return NOVA_HIP_SUCCESS;
}

// Shared validation of the SCE forward entry points (optional softmax and
// fused gradient outputs).
int32_t sce_common(const NovaMemRef2D *logits, const NovaMemRef1D *labels, NovaMemRef1D *loss,
                   NovaMemRef2D *softmax, NovaMemRef2D *grad, const char *what,
                   bool noalloc = false) {
  clear_error();
  if (!logits || !labels || !loss) return fail(NOVA_HIP_EINVAL, "%s: null descriptor", what);
  const int64_t R = logits->sizes[0], C = logits->sizes[1];
  if (R < 0 || C < 0) return fail(NOVA_HIP_ESHAPE, "%s: negative size", what);
  if (labels->sizes[0] != R) return fail(NOVA_HIP_ESHAPE, "%s: labels size != rows", what);
  if (loss->sizes[0] != 1) return fail(NOVA_HIP_ESHAPE, "%s: loss must have shape [1]", what);
  if (softmax && (softmax->sizes[0] != R || softmax->sizes[1] != C))
    return fail(NOVA_HIP_ESHAPE, "%s: softmax shape differs from logits", what);
  if (grad && (grad->sizes[0] != R || grad->sizes[1] != C))
    return fail(NOVA_HIP_ESHAPE, "%s: grad shape differs from logits", what);
  if (C == 0 && R > 0) return fail(NOVA_HIP_ESHAPE, "%s: zero classes", what);
  if ((logits->strides[1] != 1 && C > 1) || (labels->strides[0] != 1 && R > 1) ||
      (softmax && softmax->strides[1] != 1 && C > 1) || (grad && grad->strides[1] != 1 && C > 1))
    return fail(NOVA_HIP_ESTRIDE, "%s: last dim must be contiguous", what);
  if (R > 1 && (logits->strides[0] < C || (softmax && softmax->strides[0] < C) ||
                (grad && grad->strides[0] < C)))
    return fail(NOVA_HIP_ESTRIDE, "%s: rows overlap", what);
  if (!loss->aligned || (R > 0 && (!logits->aligned || !labels->aligned)) ||
      (softmax && !softmax->aligned) || (grad && !grad->aligned))
    return fail(NOVA_HIP_EINVAL, "%s: null data pointer", what);
  SceProblem p;
  p.logits = reinterpret_cast<const float *>(data_of(logits)) + logits->offset;
  p.labels = reinterpret_cast<const int32_t *>(data_of(labels)) + labels->offset;
  p.loss = reinterpret_cast<float *>(const_cast<char *>(data_of(loss))) + loss->offset;
  p.softmax = softmax ? reinterpret_cast<float *>(const_cast<char *>(data_of(softmax))) + softmax->offset : nullptr;
  p.grad = grad ? reinterpret_cast<float *>(const_cast<char *>(data_of(grad))) + grad->offset : nullptr;
  p.rows = R;
  p.C = C;
  p.sx = logits->strides[0];
  p.ssm = softmax ? softmax->strides[0] : 0;
  p.sg = grad ? grad->strides[0] : 0;
  return noalloc ? launch_sce_noalloc(p, current_stream()) : launch_sce(p, current_stream());
}

template <typename D>
float *out_f32(D *d) {
  return reinterpret_cast<float *>(const_cast<char *>(data_of(d))) + d->offset;
}
template <typename D>
const float *in_f32(const D *d) {
  return reinterpret_cast<const float *>(data_of(d)) + d->offset;
}

}  // namespace
}  // namespace nova_hip

using namespace nova_hip;

extern "C" {

int32_t _mlir_ciface_nova_hip_gemm(const NovaMemRef3D *A, const NovaMemRef3D *B,
                                   NovaMemRef3D *C, const NovaMemRef1D *bias,
                                   int32_t flags) {
  return gemm_core(A, B, C, bias, flags);
}

int32_t _mlir_ciface_nova_hip_matmul_f32(const NovaMemRef2D *A, const NovaMemRef2D *B,
                                         NovaMemRef2D *C) {
  return gemm2d(A, B, C, nullptr,
                NOVA_HIP_GEMM_FLAGS(NOVA_HIP_DT_F32, NOVA_HIP_DT_F32, NOVA_HIP_EPI_NONE, 0));
}

int32_t _mlir_ciface_nova_hip_batch_matmul_f32(const NovaMemRef3D *A, const NovaMemRef3D *B,
                                               NovaMemRef3D *C) {
  return gemm_core(A, B, C, nullptr,
                   NOVA_HIP_GEMM_FLAGS(NOVA_HIP_DT_F32, NOVA_HIP_DT_F32, NOVA_HIP_EPI_NONE, 0));
}

int32_t _mlir_ciface_nova_hip_batch_matmul_bf16_f32(const NovaMemRef3D *A,
                                                    const NovaMemRef3D *B,
                                                    NovaMemRef3D *C) {
  return gemm_core(A, B, C, nullptr,
                   NOVA_HIP_GEMM_FLAGS(NOVA_HIP_DT_BF16, NOVA_HIP_DT_F32, NOVA_HIP_EPI_NONE, 0));
}

int32_t _mlir_ciface_nova_hip_batch_matmul_f16_f32(const NovaMemRef3D *A,
                                                   const NovaMemRef3D *B,
                                                   NovaMemRef3D *C) {
  return gemm_core(A, B, C, nullptr,
                   NOVA_HIP_GEMM_FLAGS(NOVA_HIP_DT_F16, NOVA_HIP_DT_F32, NOVA_HIP_EPI_NONE, 0));
}

int32_t _mlir_ciface_nova_hip_matmul_bf16_f32(const NovaMemRef2D *A, const NovaMemRef2D *B,
                                              NovaMemRef2D *C) {
  return gemm2d(A, B, C, nullptr,
                NOVA_HIP_GEMM_FLAGS(NOVA_HIP_DT_BF16, NOVA_HIP_DT_F32, NOVA_HIP_EPI_NONE, 0));
}

int32_t _mlir_ciface_nova_hip_matmul_f16_f32(const NovaMemRef2D *A, const NovaMemRef2D *B,
                                             NovaMemRef2D *C) {
  return gemm2d(A, B, C, nullptr,
                NOVA_HIP_GEMM_FLAGS(NOVA_HIP_DT_F16, NOVA_HIP_DT_F32, NOVA_HIP_EPI_NONE, 0));
}

int32_t _mlir_ciface_nova_hip_linear(const NovaMemRef2D *x, const NovaMemRef2D *weight,
                                     const NovaMemRef1D *bias, NovaMemRef2D *y,
                                     int32_t flags) {
  return gemm2d(x, weight, y, bias, flags);
}

int32_t _mlir_ciface_nova_hip_linear_bf16_bias_gelu(const NovaMemRef2D *x,
                                                    const NovaMemRef2D *weight,
                                                    const NovaMemRef1D *bias,
                                                    NovaMemRef2D *y) {
  return gemm2d(x, weight, y, bias,
                NOVA_HIP_GEMM_FLAGS(NOVA_HIP_DT_BF16, NOVA_HIP_DT_BF16,
                                    NOVA_HIP_EPI_BIAS_GELU, NOVA_HIP_DT_BF16));
}

int32_t _mlir_ciface_nova_hip_layer_norm_f32(const NovaMemRef2D *x, const NovaMemRef1D *gamma,
                                             const NovaMemRef1D *beta, NovaMemRef2D *y,
                                             NovaMemRef1D *mean_sum, NovaMemRef1D *rstd,
                                             float eps) {
  clear_error();
  if (!x || !gamma || !beta || !y) return fail(NOVA_HIP_EINVAL, "layer_norm: null descriptor");
  const int64_t R = x->sizes[0], D = x->sizes[1];
  if (R < 0 || D < 0) return fail(NOVA_HIP_ESHAPE, "layer_norm: negative size");
  if (y->sizes[0] != R || y->sizes[1] != D)
    return fail(NOVA_HIP_ESHAPE, "layer_norm: y shape differs from x");
  if (gamma->sizes[0] != D || beta->sizes[0] != D)
    return fail(NOVA_HIP_ESHAPE, "layer_norm: gamma/beta size != D");
  if (mean_sum && mean_sum->sizes[0] != R) return fail(NOVA_HIP_ESHAPE, "layer_norm: mean_sum size != rows");
  if (rstd && rstd->sizes[0] != R) return fail(NOVA_HIP_ESHAPE, "layer_norm: rstd size != rows");
  if (R == 0) return NOVA_HIP_SUCCESS;
  if (D == 0) return fail(NOVA_HIP_ESHAPE, "layer_norm: empty normalised dim");
  if ((x->strides[1] != 1 && D > 1) || (y->strides[1] != 1 && D > 1) ||
      (gamma->strides[0] != 1 && D > 1) || (beta->strides[0] != 1 && D > 1))
    return fail(NOVA_HIP_ESTRIDE, "layer_norm: last dim must be contiguous");
  if ((mean_sum && mean_sum->strides[0] != 1 && R > 1) || (rstd && rstd->strides[0] != 1 && R > 1))
    return fail(NOVA_HIP_ESTRIDE, "layer_norm: stats must be contiguous");
  if (!x->aligned || !y->aligned || !gamma->aligned || !beta->aligned ||
      (mean_sum && !mean_sum->aligned) || (rstd && !rstd->aligned))
    return fail(NOVA_HIP_EINVAL, "layer_norm: null data pointer");
  if ((R > 1 && (x->strides[0] < D || y->strides[0] < D)))
    return fail(NOVA_HIP_ESTRIDE, "layer_norm: rows overlap");
  LayerNormProblem p;
  p.x = reinterpret_cast<const float *>(data_of(x)) + x->offset;
  p.y = reinterpret_cast<float *>(const_cast<char *>(data_of(y))) + y->offset;
  p.gamma = reinterpret_cast<const float *>(data_of(gamma)) + gamma->offset;
  p.beta = reinterpret_cast<const float *>(data_of(beta)) + beta->offset;
  p.mean_sum = mean_sum ? reinterpret_cast<float *>(const_cast<char *>(data_of(mean_sum))) + mean_sum->offset : nullptr;
  p.rstd = rstd ? reinterpret_cast<float *>(const_cast<char *>(data_of(rstd))) + rstd->offset : nullptr;
  p.rows = R;
  p.D = D;
  p.sx = x->strides[0];
  p.sy = y->strides[0];
  p.eps = eps;
  return launch_layer_norm(p, current_stream());
}

int32_t _mlir_ciface_nova_hip_sce_f32(const NovaMemRef2D *logits, const NovaMemRef1D *labels,
                                      NovaMemRef1D *loss, NovaMemRef2D *softmax) {
  return sce_common(logits, labels, loss, softmax, nullptr, "sce");
}

int32_t _mlir_ciface_nova_hip_sce_f32_noalloc(const NovaMemRef2D *logits,
                                              const NovaMemRef1D *labels, NovaMemRef1D *loss,
                                              NovaMemRef2D *softmax) {
  return sce_common(logits, labels, loss, softmax, nullptr, "sce_noalloc", true);
}

int32_t _mlir_ciface_nova_hip_sce_fwd_bwd_f32(const NovaMemRef2D *logits,
                                              const NovaMemRef1D *labels, NovaMemRef1D *loss,
                                              NovaMemRef2D *grad) {
  if (!grad) {
    clear_error();
    return fail(NOVA_HIP_EINVAL, "sce_fwd_bwd: null grad descriptor");
  }
  return sce_common(logits, labels, loss, nullptr, grad, "sce_fwd_bwd");
}

int32_t _mlir_ciface_nova_hip_sce_backward_f32(const NovaMemRef2D *softmax,
                                               const NovaMemRef1D *labels, NovaMemRef2D *grad) {
  clear_error();
  if (!softmax || !labels || !grad) return fail(NOVA_HIP_EINVAL, "sce_backward: null descriptor");
  const int64_t R = softmax->sizes[0], C = softmax->sizes[1];
  if (R < 0 || C < 0) return fail(NOVA_HIP_ESHAPE, "sce_backward: negative size");
  if (labels->sizes[0] != R) return fail(NOVA_HIP_ESHAPE, "sce_backward: labels size != rows");
  if (grad->sizes[0] != R || grad->sizes[1] != C)
    return fail(NOVA_HIP_ESHAPE, "sce_backward: grad shape differs from softmax");
  if (R == 0 || C == 0) return NOVA_HIP_SUCCESS;
  if ((softmax->strides[1] != 1 && C > 1) || (grad->strides[1] != 1 && C > 1) ||
      (labels->strides[0] != 1 && R > 1))
    return fail(NOVA_HIP_ESTRIDE, "sce_backward: last dim must be contiguous");
  if (R > 1 && (softmax->strides[0] < C || grad->strides[0] < C))
    return fail(NOVA_HIP_ESTRIDE, "sce_backward: rows overlap");
  if (!softmax->aligned || !labels->aligned || !grad->aligned)
    return fail(NOVA_HIP_EINVAL, "sce_backward: null data pointer");
  SceBackwardProblem p;
  p.softmax = in_f32(softmax);
  p.labels = reinterpret_cast<const int32_t *>(data_of(labels)) + labels->offset;
  p.grad = out_f32(grad);
  p.rows = R;
  p.C = C;
  p.ss = softmax->strides[0];
  p.sg = grad->strides[0];
  return launch_sce_backward(p, current_stream());
}

int32_t _mlir_ciface_nova_hip_layer_norm_backward_f32(
    const NovaMemRef2D *grad_y, const NovaMemRef2D *x, const NovaMemRef1D *gamma,
    const NovaMemRef1D *mean_sum, const NovaMemRef1D *rstd, NovaMemRef2D *dx,
    NovaMemRef1D *dgamma, NovaMemRef1D *dbeta) {
  clear_error();
  const char *w = "layer_norm_backward";
  if (!grad_y || !x || !gamma || !mean_sum || !rstd)
    return fail(NOVA_HIP_EINVAL, "%s: null descriptor", w);
  const int64_t R = x->sizes[0], D = x->sizes[1];
  if (R < 0 || D < 0) return fail(NOVA_HIP_ESHAPE, "%s: negative size", w);
  if (grad_y->sizes[0] != R || grad_y->sizes[1] != D || (dx && (dx->sizes[0] != R || dx->sizes[1] != D)))
    return fail(NOVA_HIP_ESHAPE, "%s: grad_y / dx shape differs from x", w);
  if (gamma->sizes[0] != D || (dgamma && dgamma->sizes[0] != D) || (dbeta && dbeta->sizes[0] != D))
    return fail(NOVA_HIP_ESHAPE, "%s: gamma / dgamma / dbeta size != D", w);
  if (mean_sum->sizes[0] != R || rstd->sizes[0] != R)
    return fail(NOVA_HIP_ESHAPE, "%s: mean_sum / rstd size != rows", w);
  if (D == 0) return fail(NOVA_HIP_ESHAPE, "%s: empty normalised dim", w);
  if ((x->strides[1] != 1 && D > 1) || (grad_y->strides[1] != 1 && D > 1) ||
      (dx && dx->strides[1] != 1 && D > 1) || (gamma->strides[0] != 1 && D > 1) ||
      (dgamma && dgamma->strides[0] != 1 && D > 1) || (dbeta && dbeta->strides[0] != 1 && D > 1))
    return fail(NOVA_HIP_ESTRIDE, "%s: last dim must be contiguous", w);
  if ((mean_sum->strides[0] != 1 || rstd->strides[0] != 1) && R > 1)
    return fail(NOVA_HIP_ESTRIDE, "%s: stats must be contiguous", w);
  if (R > 1 && (x->strides[0] < D || grad_y->strides[0] < D || (dx && dx->strides[0] < D)))
    return fail(NOVA_HIP_ESTRIDE, "%s: rows overlap", w);
  if (!gamma->aligned || (dgamma && !dgamma->aligned) || (dbeta && !dbeta->aligned) ||
      (R > 0 && (!x->aligned || !grad_y->aligned || !mean_sum->aligned || !rstd->aligned ||
                 (dx && !dx->aligned))))
    return fail(NOVA_HIP_EINVAL, "%s: null data pointer", w);
  LayerNormBackwardProblem p;
  p.gy = in_f32(grad_y);
  p.x = in_f32(x);
  p.gamma = in_f32(gamma);
  p.mean_sum = in_f32(mean_sum);
  p.rstd = in_f32(rstd);
  p.dx = dx ? out_f32(dx) : nullptr;
  p.dgamma = dgamma ? out_f32(dgamma) : nullptr;
  p.dbeta = dbeta ? out_f32(dbeta) : nullptr;
  p.rows = R;
  p.D = D;
  p.sgy = grad_y->strides[0];
  p.sx = x->strides[0];
  p.sdx = dx ? dx->strides[0] : 0;
  return launch_layer_norm_backward(p, current_stream());
}

int32_t _mlir_ciface_nova_hip_linear_backward(const NovaMemRef2D *grad_out, const NovaMemRef2D *x,
                                              const NovaMemRef2D *weight,
                                              NovaMemRef2D *grad_input,
                                              NovaMemRef2D *grad_weight,
                                              NovaMemRef1D *grad_bias, int32_t flags) {
  clear_error();
  const char *w = "linear_backward";
  if (!grad_out || !x || !weight) return fail(NOVA_HIP_EINVAL, "%s: null descriptor", w);
  int in_dt, out_dt;
  int32_t rc = backward_flags(flags, in_dt, out_dt, w);
  if (rc) return rc;
  const int64_t M = x->sizes[0], K = x->sizes[1], N = weight->sizes[1];
  if (weight->sizes[0] != K || grad_out->sizes[0] != M || grad_out->sizes[1] != N)
    return fail(NOVA_HIP_ESHAPE, "%s: x [%lld,%lld], weight [%lld,%lld], grad_out [%lld,%lld]",
                w, (long long)M, (long long)K, (long long)weight->sizes[0], (long long)N,
                (long long)grad_out->sizes[0], (long long)grad_out->sizes[1]);
  // grad_input [M,K] = grad_out . weight^T  (NovaToLinalgGeneric.cpp:1867-1911)
  // grad_weight [K,N] = x^T . grad_out  (:1913-1968)
  // grad_bias [N] = column sums of grad_out  (:1970-1989)
  // Every requested output is validated before the first launch, so a call
  // that fails writes nothing.
  NovaMemRef2D wt = transposed(weight), xt = transposed(x);
  if (grad_input && (rc = gemm2d_to(grad_out, &wt, grad_input, flags, false))) return rc;
  if (grad_weight && (rc = gemm2d_to(&xt, grad_out, grad_weight, flags, false))) return rc;
  if (grad_bias) {
    clear_error();
    if (grad_bias->sizes[0] != N) return fail(NOVA_HIP_ESHAPE, "%s: grad_bias size != N", w);
    if (grad_bias->strides[0] != 1 && N > 1)
      return fail(NOVA_HIP_ESTRIDE, "%s: grad_bias must be contiguous", w);
    if (grad_out->strides[1] != 1 && N > 1)
      return fail(NOVA_HIP_ESTRIDE, "%s: grad_out must have unit stride on N for grad_bias", w);
    if (M > 1 && grad_out->strides[0] < N) return fail(NOVA_HIP_ESTRIDE, "%s: grad_out rows overlap", w);
    if (N > 0 && (!grad_bias->aligned || (M > 0 && !grad_out->aligned)))
      return fail(NOVA_HIP_EINVAL, "%s: null data pointer", w);
    if (!col_sum_in_range(M, N))
      return fail(NOVA_HIP_ERANGE, "%s: grad_bias of [%lld, %lld] exceeds the column sum's range",
                  w, (long long)M, (long long)N);
  }
  if (grad_input && (rc = gemm2d_to(grad_out, &wt, grad_input, flags))) return rc;
  if (grad_weight && (rc = gemm2d_to(&xt, grad_out, grad_weight, flags))) return rc;
  if (grad_bias) {
    ColSumProblem p;
    p.in = data_of(grad_out) + grad_out->offset * dtype_size(in_dt);
    p.out = const_cast<char *>(data_of(grad_bias)) + grad_bias->offset * dtype_size(out_dt);
    p.rows = M;
    p.cols = N;
    p.ld = grad_out->strides[0];
    p.in_dt = in_dt;
    p.out_dt = out_dt;
    if ((rc = launch_col_sum(p, current_stream()))) return rc;
  }
  return NOVA_HIP_SUCCESS;
}

int32_t _mlir_ciface_nova_hip_matmul_backward(const NovaMemRef2D *grad, const NovaMemRef2D *A,
                                              const NovaMemRef2D *B, NovaMemRef2D *grad_a,
                                              NovaMemRef2D *grad_b, int32_t flags) {
  clear_error();
  const char *w = "matmul_backward";
  if (!grad || !A || !B) return fail(NOVA_HIP_EINVAL, "%s: null descriptor", w);
  int in_dt, out_dt;
  int32_t rc = backward_flags(flags, in_dt, out_dt, w);
  if (rc) return rc;
  const int64_t M = A->sizes[0], K = A->sizes[1], N = B->sizes[1];
  if (B->sizes[0] != K || grad->sizes[0] != M || grad->sizes[1] != N)
    return fail(NOVA_HIP_ESHAPE, "%s: A [%lld,%lld], B [%lld,%lld], grad [%lld,%lld]", w,
                (long long)M, (long long)K, (long long)B->sizes[0], (long long)N,
                (long long)grad->sizes[0], (long long)grad->sizes[1]);
  // grad_a [M,K] = grad . B^T; grad_b [K,N] = A^T . grad
  // (NovaMatmulBackwardPattern, NovaToLinalgGeneric.cpp:160-239), both
  // validated before either is launched.
  NovaMemRef2D bt = transposed(B), at = transposed(A);
  if (grad_a && (rc = gemm2d_to(grad, &bt, grad_a, flags, false))) return rc;
  if (grad_b && (rc = gemm2d_to(&at, grad, grad_b, flags, false))) return rc;
  if (grad_a && (rc = gemm2d_to(grad, &bt, grad_a, flags))) return rc;
  if (grad_b && (rc = gemm2d_to(&at, grad, grad_b, flags))) return rc;
  return NOVA_HIP_SUCCESS;
}

// ---- program glue ---------------------------------------------------------------
namespace {
bool index_dt_ok(int32_t dt) {
  return dt == NOVA_HIP_DT_I16 || dt == NOVA_HIP_DT_I32 || dt == NOVA_HIP_DT_I64;
}
int index_size(int32_t dt) { return dt == NOVA_HIP_DT_I16 ? 2 : dt == NOVA_HIP_DT_I32 ? 4 : 8; }
// A dense 1-D f32 view (unit stride, or a single element).
int32_t dense1(const NovaMemRef1D *d, const char *w, const char *what) {
  if (!d) return fail(NOVA_HIP_EINVAL, "%s: null %s", w, what);
  if (d->sizes[0] < 0) return fail(NOVA_HIP_ESHAPE, "%s: negative size", w);
  if (d->sizes[0] > 1 && d->strides[0] != 1)
    return fail(NOVA_HIP_ESTRIDE, "%s: %s must be dense", w, what);
  if (d->sizes[0] > 0 && !d->aligned) return fail(NOVA_HIP_EINVAL, "%s: null data pointer", w);
  return NOVA_HIP_SUCCESS;
}
}  // namespace

int32_t _mlir_ciface_nova_hip_binary_f32(const NovaMemRef4D *a, const NovaMemRef4D *b,
                                         NovaMemRef4D *c, int32_t op) {
  clear_error();
  const char *w = "binary";
  if (!a || !b || !c) return fail(NOVA_HIP_EINVAL, "%s: null descriptor", w);
  if (op < NOVA_HIP_BIN_ADD || op > NOVA_HIP_BIN_DIV)
    return fail(NOVA_HIP_EINVAL, "%s: unknown op %d", w, op);
  BinaryProblem p;
  int64_t n = 1;
  for (int d = 0; d < 4; ++d) {
    const int64_t m = c->sizes[d];
    if (m < 0 || a->sizes[d] < 0 || b->sizes[d] < 0)
      return fail(NOVA_HIP_ESHAPE, "%s: negative size", w);
    if ((a->sizes[d] != m && a->sizes[d] != 1) || (b->sizes[d] != m && b->sizes[d] != 1))
      return fail(NOVA_HIP_ESHAPE, "%s: dim %d: %lld and %lld do not broadcast to %lld", w, d,
                  (long long)a->sizes[d], (long long)b->sizes[d], (long long)m);
    p.size[d] = m;
    p.sa[d] = a->sizes[d] == 1 ? 0 : a->strides[d];
    p.sb[d] = b->sizes[d] == 1 ? 0 : b->strides[d];
    p.sc[d] = c->strides[d];
    n *= m;
  }
  if (n == 0) return NOVA_HIP_SUCCESS;
  if (!a->aligned || !b->aligned || !c->aligned)
    return fail(NOVA_HIP_EINVAL, "%s: null data pointer", w);
  p.a = in_f32(a);
  p.b = in_f32(b);
  p.c = out_f32(c);
  p.op = op;
  return launch_binary(p, current_stream());
}

int32_t _mlir_ciface_nova_hip_fill_f32(NovaMemRef1D *out, float value) {
  clear_error();
  if (!out) return fail(NOVA_HIP_EINVAL, "fill: null descriptor");
  if (out->sizes[0] < 0) return fail(NOVA_HIP_ESHAPE, "fill: negative size");
  if (out->sizes[0] == 0) return NOVA_HIP_SUCCESS;
  if (!out->aligned) return fail(NOVA_HIP_EINVAL, "fill: null data pointer");
  return launch_fill(out_f32(out), out->sizes[0], out->strides[0], value, current_stream());
}

int32_t _mlir_ciface_nova_hip_gelu_f32(const NovaMemRef1D *x, NovaMemRef1D *y) {
  clear_error();
  int32_t rc;
  if ((rc = dense1(x, "gelu", "x")) || (rc = dense1(y, "gelu", "y"))) return rc;
  if (x->sizes[0] != y->sizes[0]) return fail(NOVA_HIP_ESHAPE, "gelu: sizes differ");
  return launch_gelu(in_f32(x), out_f32(y), x->sizes[0], current_stream());
}

int32_t _mlir_ciface_nova_hip_gelu_backward_f32(const NovaMemRef1D *grad_out,
                                                const NovaMemRef1D *x, NovaMemRef1D *out) {
  clear_error();
  const char *w = "gelu_backward";
  int32_t rc;
  if ((rc = dense1(grad_out, w, "grad_out")) || (rc = dense1(x, w, "x")) ||
      (rc = dense1(out, w, "out")))
    return rc;
  if (x->sizes[0] != grad_out->sizes[0] || x->sizes[0] != out->sizes[0])
    return fail(NOVA_HIP_ESHAPE, "%s: sizes differ", w);
  return launch_gelu_backward(in_f32(grad_out), in_f32(x), out_f32(out), x->sizes[0],
                              current_stream());
}

int32_t _mlir_ciface_nova_hip_gather_f32(const NovaMemRef2D *table, const NovaMemRef1D *idx,
                                         NovaMemRef2D *out, int32_t idx_dt) {
  clear_error();
  const char *w = "gather";
  if (!table || !idx || !out) return fail(NOVA_HIP_EINVAL, "%s: null descriptor", w);
  if (!index_dt_ok(idx_dt)) return fail(NOVA_HIP_EDTYPE, "%s: index dtype %d", w, idx_dt);
  if (!nonneg_sizes(table, 2) || !nonneg_sizes(idx, 1) || !nonneg_sizes(out, 2))
    return fail(NOVA_HIP_ESHAPE, "%s: negative size", w);
  const int64_t n = idx->sizes[0], D = table->sizes[1];
  if (out->sizes[0] != n || out->sizes[1] != D)
    return fail(NOVA_HIP_ESHAPE, "%s: out is [%lld, %lld], want [%lld, %lld]", w,
                (long long)out->sizes[0], (long long)out->sizes[1], (long long)n, (long long)D);
  if (n == 0 || D == 0) return NOVA_HIP_SUCCESS;
  if ((D > 1 && (table->strides[1] != 1 || out->strides[1] != 1)))
    return fail(NOVA_HIP_ESTRIDE, "%s: rows must be contiguous", w);
  if (!table->aligned || !idx->aligned || !out->aligned)
    return fail(NOVA_HIP_EINVAL, "%s: null data pointer", w);
  GatherProblem p;
  p.table = in_f32(table);
  p.idx = data_of(idx) + idx->offset * index_size(idx_dt);
  p.out = out_f32(out);
  p.rows = table->sizes[0];
  p.D = D;
  p.n = n;
  p.st = table->strides[0];
  p.so = out->strides[0];
  p.sidx = idx->strides[0];
  p.idx_dt = idx_dt;
  return launch_gather(p, current_stream());
}

int32_t _mlir_ciface_nova_hip_scatter_add_f32(NovaMemRef2D *out, const NovaMemRef1D *idx,
                                              const NovaMemRef2D *src, int32_t idx_dt) {
  clear_error();
  const char *w = "scatter_add";
  if (!out || !idx || !src) return fail(NOVA_HIP_EINVAL, "%s: null descriptor", w);
  if (!index_dt_ok(idx_dt)) return fail(NOVA_HIP_EDTYPE, "%s: index dtype %d", w, idx_dt);
  if (!nonneg_sizes(out, 2) || !nonneg_sizes(idx, 1) || !nonneg_sizes(src, 2))
    return fail(NOVA_HIP_ESHAPE, "%s: negative size", w);
  const int64_t n = idx->sizes[0], D = out->sizes[1];
  if (src->sizes[0] != n || src->sizes[1] != D)
    return fail(NOVA_HIP_ESHAPE, "%s: src is [%lld, %lld], want [%lld, %lld]", w,
                (long long)src->sizes[0], (long long)src->sizes[1], (long long)n, (long long)D);
  if (n == 0 || D == 0) return NOVA_HIP_SUCCESS;
  if (D > 1 && (out->strides[1] != 1 || src->strides[1] != 1))
    return fail(NOVA_HIP_ESTRIDE, "%s: rows must be contiguous", w);
  if (!out->aligned || !idx->aligned || !src->aligned)
    return fail(NOVA_HIP_EINVAL, "%s: null data pointer", w);
  ScatterAddProblem p;
  p.out = out_f32(out);
  p.idx = data_of(idx) + idx->offset * index_size(idx_dt);
  p.src = in_f32(src);
  p.rows = out->sizes[0];
  p.D = D;
  p.n = n;
  p.so = out->strides[0];
  p.ss = src->strides[0];
  p.sidx = idx->strides[0];
  p.idx_dt = idx_dt;
  return launch_scatter_add(p, current_stream());
}

int32_t _mlir_ciface_nova_hip_reduce_sum_f32(const NovaMemRef3D *x, NovaMemRef2D *out) {
  clear_error();
  const char *w = "reduce_sum";
  if (!x || !out) return fail(NOVA_HIP_EINVAL, "%s: null descriptor", w);
  if (!nonneg_sizes(x, 3) || !nonneg_sizes(out, 2))
    return fail(NOVA_HIP_ESHAPE, "%s: negative size", w);
  if (out->sizes[0] != x->sizes[0] || out->sizes[1] != x->sizes[2])
    return fail(NOVA_HIP_ESHAPE, "%s: out is [%lld, %lld], want [%lld, %lld]", w,
                (long long)out->sizes[0], (long long)out->sizes[1], (long long)x->sizes[0],
                (long long)x->sizes[2]);
  if (x->sizes[0] * x->sizes[2] == 0) return NOVA_HIP_SUCCESS;
  if (!x->aligned || !out->aligned) return fail(NOVA_HIP_EINVAL, "%s: null data pointer", w);
  ReduceSumProblem p;
  p.x = in_f32(x);
  p.out = out_f32(out);
  p.outer = x->sizes[0];
  p.n = x->sizes[1];
  p.inner = x->sizes[2];
  p.so = x->strides[0];
  p.sn = x->strides[1];
  p.si = x->strides[2];
  p.soo = out->strides[0];
  p.soi = out->strides[1];
  return launch_reduce_sum(p, current_stream());
}

int32_t _mlir_ciface_nova_hip_index_to_i32(const NovaMemRef1D *src, NovaMemRef1D *dst,
                                           int32_t src_dt) {
  clear_error();
  const char *w = "index_to_i32";
  if (!src || !dst) return fail(NOVA_HIP_EINVAL, "%s: null descriptor", w);
  if (!index_dt_ok(src_dt)) return fail(NOVA_HIP_EDTYPE, "%s: index dtype %d", w, src_dt);
  int32_t rc;
  if ((rc = dense1(dst, w, "dst"))) return rc;
  if (src->sizes[0] != dst->sizes[0]) return fail(NOVA_HIP_ESHAPE, "%s: sizes differ", w);
  if (src->sizes[0] == 0) return NOVA_HIP_SUCCESS;
  if (!src->aligned) return fail(NOVA_HIP_EINVAL, "%s: null data pointer", w);
  return launch_index_to_i32(data_of(src) + src->offset * index_size(src_dt), src->strides[0],
                             src_dt,
                             reinterpret_cast<int32_t *>(const_cast<char *>(data_of(dst))) +
                                 dst->offset,
                             src->sizes[0], current_stream());
}

void nova_hip_set_stream(void *stream) { t_stream = static_cast<hipStream_t>(stream); }

void *nova_hip_get_stream(void) { return t_stream; }

int32_t nova_hip_synchronize(void) {
  clear_error();
  return check_hip(hipStreamSynchronize(t_stream), "synchronize");
}

const char *nova_hip_last_error(void) { return t_err; }

// ---- Typed aliases for lowered modules --------------------------------------
// A module declares each callee once, with one type; these aliases give the
// generic entry points one name per operand dtype combination.  The flags
// must name the alias's dtypes (the bias dtype only when the epilogue has a
// bias).
#define NOVA_GEMM_ALIAS(SUF, IN, OUT, BIAS)                                                    \
  int32_t _mlir_ciface_nova_hip_gemm_##SUF(const NovaMemRef3D *A, const NovaMemRef3D *B,       \
                                           NovaMemRef3D *C, const NovaMemRef1D *bias,          \
                                           int32_t flags) {                                    \
    const int epi = (flags >> 8) & 0xf;                                                        \
    const bool has_bias = epi == NOVA_HIP_EPI_BIAS || epi == NOVA_HIP_EPI_BIAS_GELU;          \
    if ((flags & 0xf) != (IN) || ((flags >> 4) & 0xf) != (OUT) ||                              \
        (has_bias && ((flags >> 12) & 0xf) != (BIAS))) {                                       \
      clear_error();                                                                           \
      return fail(NOVA_HIP_EINVAL, "gemm_" #SUF ": flags 0x%x name other dtypes", flags);     \
    }                                                                                          \
    return gemm_core(A, B, C, bias, flags);                                                    \
  }
#define NOVA_GEMM_ALIASES_OUT(IS, IN, OS, OUT)               \
  NOVA_GEMM_ALIAS(IS##_##OS##_bf32, IN, OUT, NOVA_HIP_DT_F32) \
  NOVA_GEMM_ALIAS(IS##_##OS##_bbf16, IN, OUT, NOVA_HIP_DT_BF16) \
  NOVA_GEMM_ALIAS(IS##_##OS##_bf16, IN, OUT, NOVA_HIP_DT_F16)
#define NOVA_GEMM_ALIASES_IN(IS, IN)                     \
  NOVA_GEMM_ALIASES_OUT(IS, IN, f32, NOVA_HIP_DT_F32)   \
  NOVA_GEMM_ALIASES_OUT(IS, IN, bf16, NOVA_HIP_DT_BF16) \
  NOVA_GEMM_ALIASES_OUT(IS, IN, f16, NOVA_HIP_DT_F16)
NOVA_GEMM_ALIASES_IN(f32, NOVA_HIP_DT_F32)
NOVA_GEMM_ALIASES_IN(bf16, NOVA_HIP_DT_BF16)
NOVA_GEMM_ALIASES_IN(f16, NOVA_HIP_DT_F16)

#define NOVA_BWD_ALIAS(SUF, IN, OUT)                                                             \
  int32_t _mlir_ciface_nova_hip_linear_backward_##SUF(                                           \
      const NovaMemRef2D *go, const NovaMemRef2D *x, const NovaMemRef2D *w, NovaMemRef2D *gi,    \
      NovaMemRef2D *gw, NovaMemRef1D *gb, int32_t flags) {                                       \
    if ((flags & 0xf) != (IN) || ((flags >> 4) & 0xf) != (OUT)) {                                \
      clear_error();                                                                             \
      return fail(NOVA_HIP_EINVAL, "linear_backward_" #SUF ": flags 0x%x name other dtypes",    \
                  flags);                                                                        \
    }                                                                                            \
    return _mlir_ciface_nova_hip_linear_backward(go, x, w, gi, gw, gb, flags);                  \
  }                                                                                              \
  int32_t _mlir_ciface_nova_hip_matmul_backward_##SUF(const NovaMemRef2D *g,                     \
                                                      const NovaMemRef2D *A,                     \
                                                      const NovaMemRef2D *B, NovaMemRef2D *ga,   \
                                                      NovaMemRef2D *gb, int32_t flags) {         \
    if ((flags & 0xf) != (IN) || ((flags >> 4) & 0xf) != (OUT)) {                                \
      clear_error();                                                                             \
      return fail(NOVA_HIP_EINVAL, "matmul_backward_" #SUF ": flags 0x%x name other dtypes",    \
                  flags);                                                                        \
    }                                                                                            \
    return _mlir_ciface_nova_hip_matmul_backward(g, A, B, ga, gb, flags);                       \
  }
NOVA_BWD_ALIAS(f32_f32, NOVA_HIP_DT_F32, NOVA_HIP_DT_F32)
NOVA_BWD_ALIAS(bf16_f32, NOVA_HIP_DT_BF16, NOVA_HIP_DT_F32)
NOVA_BWD_ALIAS(bf16_bf16, NOVA_HIP_DT_BF16, NOVA_HIP_DT_BF16)
NOVA_BWD_ALIAS(bf16_f16, NOVA_HIP_DT_BF16, NOVA_HIP_DT_F16)
NOVA_BWD_ALIAS(f16_f32, NOVA_HIP_DT_F16, NOVA_HIP_DT_F32)
NOVA_BWD_ALIAS(f16_bf16, NOVA_HIP_DT_F16, NOVA_HIP_DT_BF16)
NOVA_BWD_ALIAS(f16_f16, NOVA_HIP_DT_F16, NOVA_HIP_DT_F16)

int32_t _mlir_ciface_nova_hip_index_to_i32_i16(const NovaMemRef1D *src, NovaMemRef1D *dst,
                                               int32_t src_dt) {
  return _mlir_ciface_nova_hip_index_to_i32(src, dst, src_dt);
}
int32_t _mlir_ciface_nova_hip_index_to_i32_i64(const NovaMemRef1D *src, NovaMemRef1D *dst,
                                               int32_t src_dt) {
  return _mlir_ciface_nova_hip_index_to_i32(src, dst, src_dt);
}

int32_t _mlir_ciface_nova_hip_sce_loss_f32(const NovaMemRef2D *logits,
                                           const NovaMemRef1D *labels, NovaMemRef1D *loss) {
  return sce_common(logits, labels, loss, nullptr, nullptr, "sce");
}

const char *nova_hip_version(void) { return "libnova_hip 0.1.0 (gfx950)"; }

int32_t nova_hip_release_workspace(void) {
  clear_error();
  std::vector<hipStream_t> streams;
  {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    for (auto &kv : g_ws) streams.push_back(kv.first);
  }
  int32_t rc = NOVA_HIP_SUCCESS;
  // Each stream's buffer is freed under that stream's mutex: a call that
  // holds the buffer finishes its launches first.
  for (hipStream_t st : streams) {
    std::lock_guard<std::mutex> stream_lock(stream_mutex(st));
    std::lock_guard<std::mutex> lock(g_ws_mu);
    auto it = g_ws.find(st);
    if (it == g_ws.end()) continue;
    if (it->second.ptr) {
      hipError_t e = hipStreamSynchronize(st);
      if (e == hipSuccess) e = hipFree(it->second.ptr);
      if (e != hipSuccess) rc = check_hip(e, "release_workspace");
    }
    g_ws.erase(it);
  }
  return rc;
}

}  // extern "C"
