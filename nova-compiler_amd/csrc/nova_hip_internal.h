// Internal declarations shared by the libnova_hip translation units.
// Host-side helpers (validation, error text, stream) and the launcher
// signatures each kernel file exports to nova_hip_abi.hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "../../include/nova_hip.h"

namespace nova_hip {

// Error text of the calling thread; returns `code` so call sites can write
// `return fail(NOVA_HIP_ESHAPE, "...")`.
int32_t fail(int32_t code, const char *fmt, ...);
void clear_error();
hipStream_t current_stream();
// Compute units of the current device (cached per device), or 0 if the
// query fails.
int device_cu_count();
// LDS bytes one workgroup may use on the current device (0 if unknown).
int device_lds_per_block();
// Convert a HIP status into NOVA_HIP_EDEVICE with text, or success.
int32_t check_hip(hipError_t e, const char *what);

// Element sizes per dtype code.
inline int dtype_size(int dt) { return dt == NOVA_HIP_DT_F32 ? 4 : 2; }

// ---- GEMM -----------------------------------------------------------------
// A normalised, validated view of one batched contraction.  Strides in
// elements.  `a_kcontig` : A's unit stride is on K (else on M).
// `b_kcontig` : B's unit stride is on K (else on N).
struct GemmProblem {
  const void *A;
  const void *B;
  void *C;
  const void *bias;
  int64_t batch, M, N, K;
  int64_t sab, sa_outer;  // batch stride; stride of the non-unit dim of A
  int64_t sbb, sb_outer;  // batch stride; stride of the non-unit dim of B
  int64_t scb, scm;       // C batch and row strides (unit on N)
  bool a_kcontig, b_kcontig;
  int in_dt, out_dt, bias_dt, epi;
  bool acc_out;  // accumulate in the output dtype (NOVA_HIP_GEMM_ACC_OUT)
  bool f32_mfma;  // f32 on the matrix cores (NOVA_HIP_GEMM_F32_MFMA)
  bool acc_c;     // C holds the accumulator's initial values (NOVA_HIP_GEMM_ACC_C)
};

// Launch the MFMA kernels (bf16/f16 in).  Returns a NOVA_HIP_* status.
int32_t launch_gemm_mfma(const GemmProblem &p, hipStream_t s);
// Launch the exact kernel: f32 in and out, or (acc_out) bf16 / f16 in and
// out with the accumulator in that type.
int32_t launch_gemm_exact(const GemmProblem &p, hipStream_t s);
// f32 in and out on the f32 MFMA (NOVA_HIP_GEMM_F32_MFMA): within the f32
// parity bar, not bit-identical to the sequential-k reference arithmetic.
int32_t launch_gemm_f32_mfma(const GemmProblem &p, hipStream_t s);

// ---- reductions ------------------------------------------------------------
struct LayerNormProblem {
  const float *x;
  const float *gamma;
  const float *beta;
  float *y;
  float *mean_sum;  // may be null
  float *rstd;      // may be null
  int64_t rows, D;
  int64_t sx, sy;   // row strides (elements)
  float eps;
};
int32_t launch_layer_norm(const LayerNormProblem &p, hipStream_t s);

struct SceProblem {
  const float *logits;
  const int32_t *labels;
  float *loss;
  float *softmax;  // may be null
  float *grad;     // may be null: (softmax - onehot) / rows, the fused backward
  int64_t rows, C;
  int64_t sx, ssm, sg;  // row strides (elements)
};
int32_t launch_sce(const SceProblem &p, hipStream_t s);
// The same with the row losses in the library's static per-device array
// (rows <= SCE_NOALLOC_MAX_ROWS): no allocation.
int32_t launch_sce_noalloc(const SceProblem &p, hipStream_t s);

// ---- backward (backward.hip) ------------------------------------------------
struct SceBackwardProblem {
  const float *softmax;
  const int32_t *labels;
  float *grad;
  int64_t rows, C;
  int64_t ss, sg;  // row strides (elements)
};
int32_t launch_sce_backward(const SceBackwardProblem &p, hipStream_t s);

struct LayerNormBackwardProblem {
  const float *gy;
  const float *x;
  const float *gamma;
  const float *mean_sum;
  const float *rstd;
  float *dx;      // may be null
  float *dgamma;  // may be null
  float *dbeta;   // may be null
  int64_t rows, D;
  int64_t sgy, sx, sdx;  // row strides (elements)
};
int32_t launch_layer_norm_backward(const LayerNormBackwardProblem &p, hipStream_t s);

// out[c] = sum_r in[r, c] (rows in order within chunks, chunks in order),
// in of dtype in_dt with row stride ld, out of dtype out_dt.
struct ColSumProblem {
  const void *in;
  void *out;
  int64_t rows, cols, ld;
  int in_dt, out_dt;
};
int32_t launch_col_sum(const ColSumProblem &p, hipStream_t s);
// Whether launch_col_sum takes [rows, cols] (its row chunks and column
// groups index with 32-bit ints and run up to 2^20 past the extents).
bool col_sum_in_range(int64_t rows, int64_t cols);

// ---- program glue (glue.hip) -------------------------------------------------
// c = a (op) b over a [4]-shaped index space; strides in elements, 0 on a
// broadcast dimension.
struct BinaryProblem {
  const float *a;
  const float *b;
  float *c;
  int64_t size[4];
  int64_t sa[4], sb[4], sc[4];
  int op;
};
int32_t launch_binary(const BinaryProblem &p, hipStream_t s);
int32_t launch_fill(float *out, int64_t n, int64_t stride, float v, hipStream_t s);
int32_t launch_gelu(const float *x, float *y, int64_t n, hipStream_t s);
int32_t launch_gelu_backward(const float *go, const float *x, float *out, int64_t n,
                             hipStream_t s);

// out[i, :] = table[idx[i], :] (D columns).
struct GatherProblem {
  const float *table;
  const void *idx;
  float *out;
  int64_t rows, D, n;    // table rows, columns, indices
  int64_t st, so, sidx;  // row strides of table / out, index stride
  int idx_dt;
};
int32_t launch_gather(const GatherProblem &p, hipStream_t s);

// out[idx[i], :] += src[i, :].
struct ScatterAddProblem {
  float *out;
  const void *idx;
  const float *src;
  int64_t rows, D, n;
  int64_t so, ss, sidx;
  int idx_dt;
};
int32_t launch_scatter_add(const ScatterAddProblem &p, hipStream_t s);
int32_t launch_index_to_i32(const void *src, int64_t stride, int dt, int32_t *dst, int64_t n,
                            hipStream_t s);

// out[o, i] = sum_j x[o, j, i].
struct ReduceSumProblem {
  const float *x;
  float *out;
  int64_t outer, n, inner;
  int64_t so, sn, si;  // strides of x
  int64_t soo, soi;    // strides of out
};
int32_t launch_reduce_sum(const ReduceSumProblem &p, hipStream_t s);

// The per-stream device workspace owned by the library, held for one
// call's launches.  acquire() locks the stream's enqueue mutex until the
// lease ends, then returns the stream's buffer grown to at least `bytes`
// (null, with the error text set, when the allocation fails).  Calls made
// on one stream from several threads (every thread that has set no stream
// shares the null stream) therefore enqueue their kernels one call at a
// time: no call's kernels read another call's partials, and the buffer is
// not regrown or released while a call still has launches to make with it.
// A lease must not be acquired on a stream whose lease the thread holds.
class WorkspaceLease {
 public:
  WorkspaceLease() = default;
  WorkspaceLease(hipStream_t s, size_t bytes) { acquire(s, bytes); }
  WorkspaceLease(const WorkspaceLease &) = delete;
  WorkspaceLease &operator=(const WorkspaceLease &) = delete;
  void *acquire(hipStream_t s, size_t bytes);
  void *get() const { return ptr_; }

 private:
  std::unique_lock<std::mutex> lock_;
  void *ptr_ = nullptr;
};

}  // namespace nova_hip
