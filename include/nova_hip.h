/*
 * nova_hip.h -- C ABI of libnova_hip, the MI355X (gfx950) kernels behind
 * Nova's GPU matmul / reduction path.
 *
 * Every compute entry point is named `_mlir_ciface_nova_hip_<op>` and takes
 * pointers to MLIR strided-memref descriptors, so that a lowering which
 * emits
 *     func.func private @nova_hip_<op>(memref<...>, ...) -> i32
 *         attributes {llvm.emit_c_interface}
 *     %rc = func.call @nova_hip_<op>(...) : (...) -> i32
 * links against this library with no glue.  The descriptor layout is the one
 * MLIR's C interface passes (`_mlir_ciface_<fn>(Desc*...)`), exactly what the
 * reference's own host harness builds by hand in robust_driver.cpp:9-23 and
 * driver.cpp:9-17 ({allocated, aligned, offset, sizes[R], strides[R]}).
 *
 * Conventions (all entry points):
 *   - memref data pointers are DEVICE pointers owned by the caller (the
 *     reference's address-space-1 convention, robust_driver.cpp:25-39);
 *     the library never allocates or frees caller buffers.  It owns only a
 *     cached per-stream workspace (SCE row losses, column-sum partials).
 *   - offsets and strides are in elements and are honoured.  The innermost
 *     dimension of every operand must have unit stride, except where a GEMM
 *     operand is a transposed view (its second-to-last stride is 1 instead).
 *   - return value: NOVA_HIP_SUCCESS (0) or a NOVA_HIP_E* code; the text of
 *     the last error on the calling thread is in nova_hip_last_error().
 *     The reference's compiled entry points return void and ignore every
 *     CUDA status (FixGpuLaunch.cpp:49); these report instead.
 *   - launches are asynchronous on the calling thread's stream
 *     (nova_hip_set_stream; default: the null stream).
 */
#ifndef NOVA_HIP_H
#define NOVA_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* MLIR StridedMemRefType<T, R> for R = 1, 2, 3 (element type erased). */
typedef struct NovaMemRef1D {
  void *allocated;
  void *aligned;
  int64_t offset;
  int64_t sizes[1];
  int64_t strides[1];
} NovaMemRef1D;

typedef struct NovaMemRef2D {
  void *allocated;
  void *aligned;
  int64_t offset;
  int64_t sizes[2];
  int64_t strides[2];
} NovaMemRef2D;

typedef struct NovaMemRef3D {
  void *allocated;
  void *aligned;
  int64_t offset;
  int64_t sizes[3];
  int64_t strides[3];
} NovaMemRef3D;

typedef struct NovaMemRef4D {
  void *allocated;
  void *aligned;
  int64_t offset;
  int64_t sizes[4];
  int64_t strides[4];
} NovaMemRef4D;

/* Status codes.  Every entry point checks all of its descriptors before it
 * launches anything, so a call that returns 1-4 has written nothing.  A
 * call with two or three outputs (linear_backward, matmul_backward) may
 * return 5-7 from a later output's launch after an earlier output has
 * been written. */
enum {
  NOVA_HIP_SUCCESS = 0,
  NOVA_HIP_EINVAL = 1,    /* null descriptor / data pointer, bad flag bits  */
  NOVA_HIP_ESHAPE = 2,    /* operand shapes disagree                        */
  NOVA_HIP_ESTRIDE = 3,   /* stride pattern the kernels do not address      */
  NOVA_HIP_EDTYPE = 4,    /* dtype / epilogue combination not provided      */
  NOVA_HIP_ERANGE = 5,    /* size beyond the kernels' index range           */
  NOVA_HIP_EDEVICE = 6,   /* HIP runtime error (details in last_error)      */
  NOVA_HIP_ENOMEM = 7     /* workspace allocation failed                    */
};

/* dtype codes (flags bits 0-3: input, 4-7: output, 12-15: bias; the
 * integer codes name index / label operands of the program-glue ops). */
enum {
  NOVA_HIP_DT_F32 = 0,
  NOVA_HIP_DT_BF16 = 1,
  NOVA_HIP_DT_F16 = 2,
  NOVA_HIP_DT_I32 = 3,
  NOVA_HIP_DT_I64 = 4,
  NOVA_HIP_DT_I16 = 5
};

/* binary op codes of _mlir_ciface_nova_hip_binary_f32. */
enum {
  NOVA_HIP_BIN_ADD = 0,
  NOVA_HIP_BIN_SUB = 1,
  NOVA_HIP_BIN_MUL = 2,
  NOVA_HIP_BIN_DIV = 3
};

/* epilogue codes (flags bits 8-11). */
enum {
  NOVA_HIP_EPI_NONE = 0,
  NOVA_HIP_EPI_BIAS = 1,      /* C = A.B + bias[n]                           */
  NOVA_HIP_EPI_BIAS_GELU = 2, /* C = gelu_tanh(A.B + bias[n])                */
  NOVA_HIP_EPI_GELU = 3       /* C = gelu_tanh(A.B)                          */
};

#define NOVA_HIP_GEMM_FLAGS(in_dt, out_dt, epi, bias_dt)                     \
  ((int32_t)(((in_dt) & 0xf) | (((out_dt) & 0xf) << 4) |                     \
             (((epi) & 0xf) << 8) | (((bias_dt) & 0xf) << 12)))

/* flags bit 16: accumulate in the output dtype.  A linalg.matmul /
 * batch_matmul whose outs is bf16 or f16 runs its body C += A * B in that
 * type (NovaMatmulOpLowering builds one for an f16 x f16 nova.matmul, whose
 * result is f16: NovaToLinalg.cpp:1027-1049, NovaOps.cpp:1198; nova.linear
 * on f16 / bf16 operands likewise, NovaToLinalgGeneric.cpp:1623-1822):
 * every product and partial sum is rounded to it, k ascending, from zero or
 * from the bias (FuseMatmulBias.cpp:184-188).  Needs in == out dtype, bf16
 * or f16, and an epilogue of none or a bias of that dtype.  Without the bit,
 * bf16 / f16 inputs accumulate in f32 (the MFMA kernels). */
#define NOVA_HIP_GEMM_ACC_OUT 0x10000

/* flags bit 17: f32 operands on the f32 matrix cores (v_mfma_f32_32x32x2_f32)
 * instead of the exact kernel.  Products are exact and sums f32, but in the
 * MFMA's and the tile loop's order, not the reference's sequential k: the
 * result is within the f32 parity bar (1e-4 relative), not bit-identical to
 * Nova's CPU pipeline.  Same results on every run.  f32 in and out; the
 * epilogues as for the other kernels.  Also accepted by the backward GEMM
 * entry points. */
#define NOVA_HIP_GEMM_F32_MFMA 0x20000

/* flags bit 18: C holds the accumulator's initial values.  C = C + A . B in
 * place, each element summed k ascending from its own value in C: a
 * linalg.matmul / linalg.batch_matmul whose outs holds data, such as a
 * function argument (test/pipeline-tests/02_matmul_aligned.mlir:15-19,
 * 06_matmul_exact_tile.mlir:17-21, 11_lowering_config.mlir:21-27), runs its body
 * C += A * B from that data where NovaMatmulOpLowering's zero fill
 * (NovaToLinalg.cpp:1031-1049) would start from 0.  The exact kernel only:
 * f32 in and out, or bf16 / f16 in and out with NOVA_HIP_GEMM_ACC_OUT; no
 * epilogue; not with NOVA_HIP_GEMM_F32_MFMA.  C must not overlap A or B. */
#define NOVA_HIP_GEMM_ACC_C 0x40000

/* ------------------------------------------------------------------------
 * GEMM family.
 *
 * General batched contraction C[b,m,n] = epi(sum_k A[b,m,k] * B[b,k,n]),
 * f32 accumulate.  Replaces, for these ops, the LLVMGPU code generation of
 * `nova-gpu-optimized-pipeline` (lib/Transforms/LLVMGPU/Passes.cpp:115-372)
 * applied to the linalg.matmul / linalg.batch_matmul that
 * NovaMatmulOpLowering produces (NovaToLinalg.cpp:874-1051, rank-3 at :1040,
 * rank-2 at :1045), the bias accumulator init of FuseMatmulBias
 * (FuseMatmulBias.cpp:95-199) and the nova.gelu generic
 * (NovaToLinalgGeneric.cpp:1277-1337) that follows nova.linear.
 *
 *   A : [B, M, K]  unit stride on K (row-major) or on M (transposed view);
 *                  batch stride 0 broadcasts a rank-2 operand
 *                  (NovaToLinalg.cpp:992-1025).
 *   B : [B, K, N]  unit stride on N (row-major) or on K (transposed view,
 *                  e.g. nova.transpose of a [N,K] weight).
 *   C : [B, M, N]  unit stride on N.
 *   bias : [N] unit stride, or NULL when the epilogue has no bias.
 *   flags : NOVA_HIP_GEMM_FLAGS(in, out, epilogue, bias dtype).
 * Inputs f32 use an exact f32 kernel (sequential k, unfused multiply-add,
 * the reference's CPU arithmetic); bf16 / f16 inputs use MFMA with f32
 * accumulate, or with NOVA_HIP_GEMM_ACC_OUT the same exact kernel with the
 * accumulator in the input dtype.  Low-precision outputs are rounded to
 * nearest-even.
 * ---------------------------------------------------------------------- */
int32_t _mlir_ciface_nova_hip_gemm(const NovaMemRef3D *A, const NovaMemRef3D *B,
                                   NovaMemRef3D *C, const NovaMemRef1D *bias,
                                   int32_t flags);

/* nova.matmul rank 2, f32 x f32 -> f32 (NovaOps.cpp:1116-1285 result type;
 * linalg.matmul at NovaToLinalg.cpp:1045). */
int32_t _mlir_ciface_nova_hip_matmul_f32(const NovaMemRef2D *A,
                                         const NovaMemRef2D *B,
                                         NovaMemRef2D *C);

/* nova.matmul rank 3 (linalg.batch_matmul, NovaToLinalg.cpp:1040), f32. */
int32_t _mlir_ciface_nova_hip_batch_matmul_f32(const NovaMemRef3D *A,
                                               const NovaMemRef3D *B,
                                               NovaMemRef3D *C);

/* linalg.batch_matmul with bf16 ins and f32 outs (test/pipeline-tests/
 * 03_batch_matmul.mlir:20-26 form; bf16 x bf16 nova.matmul infers f16,
 * NovaOps.cpp:1198, so the f32-accumulate form is spelled in linalg or with
 * nova.cast operands). */
int32_t _mlir_ciface_nova_hip_batch_matmul_bf16_f32(const NovaMemRef3D *A,
                                                    const NovaMemRef3D *B,
                                                    NovaMemRef3D *C);

/* Same, f16 ins and f32 outs. */
int32_t _mlir_ciface_nova_hip_batch_matmul_f16_f32(const NovaMemRef3D *A,
                                                   const NovaMemRef3D *B,
                                                   NovaMemRef3D *C);

/* Rank-2 low-precision forms of the two entry points above. */
int32_t _mlir_ciface_nova_hip_matmul_bf16_f32(const NovaMemRef2D *A,
                                              const NovaMemRef2D *B,
                                              NovaMemRef2D *C);
int32_t _mlir_ciface_nova_hip_matmul_f16_f32(const NovaMemRef2D *A,
                                             const NovaMemRef2D *B,
                                             NovaMemRef2D *C);

/* nova.linear (NovaToLinalgGeneric.cpp:1623-1822; result type
 * NovaOps.cpp:2075-2103) with the bias folded into the accumulator
 * (FuseMatmulBias.cpp:184-188), optionally followed by nova.gelu
 * (NovaToLinalgGeneric.cpp:1277-1337) and nova.cast to the output dtype
 * (NovaToLinalgGeneric.cpp:37-85).
 *   x : [M, K]; weight : [K, N] (a row-major [K,N] tensor, or the
 *   nova.transpose view of a row-major [N,K] tensor: strides {1, K});
 *   bias : [N]; y : [M, N].  flags as for _mlir_ciface_nova_hip_gemm. */
int32_t _mlir_ciface_nova_hip_linear(const NovaMemRef2D *x,
                                     const NovaMemRef2D *weight,
                                     const NovaMemRef1D *bias, NovaMemRef2D *y,
                                     int32_t flags);

/* The config-3 form: bf16 x, bf16 weight view, bf16 bias, GELU(tanh),
 * bf16 y, f32 accumulate. */
int32_t _mlir_ciface_nova_hip_linear_bf16_bias_gelu(const NovaMemRef2D *x,
                                                    const NovaMemRef2D *weight,
                                                    const NovaMemRef1D *bias,
                                                    NovaMemRef2D *y);

/* ------------------------------------------------------------------------
 * Reductions (HBM bound, no MFMA).
 * ---------------------------------------------------------------------- */

/* nova.layer_norm over the last dim (NovaLayerNormPattern,
 * NovaToLinalgGeneric.cpp:1997-2126; results (y, mean_sum, var_sum) of
 * NovaOps.td:1027-1037 where var_sum carries rstd, :2123).
 *   x, y : [R, D] f32; gamma, beta : [D] f32;
 *   mean_sum : [R] f32 row sums S, or NULL;  rstd : [R] f32, or NULL.
 * eps: the op hard-codes 1e-5 (NovaToLinalgGeneric.cpp:2025). */
int32_t _mlir_ciface_nova_hip_layer_norm_f32(const NovaMemRef2D *x,
                                             const NovaMemRef1D *gamma,
                                             const NovaMemRef1D *beta,
                                             NovaMemRef2D *y,
                                             NovaMemRef1D *mean_sum,
                                             NovaMemRef1D *rstd, float eps);

/* nova.sce (NovaSceForwardLowering, NovaToLinalgGeneric.cpp:801-1010;
 * results (softmax, loss[1]) of NovaOps.td:880-896) with the mean of
 * lowerFullReduceMeanToSCF (NovaToLinalg.cpp:1974-2126).
 *   logits : [R, C] f32; labels : [R] i32 in [0, C);
 *   loss : [1] f32; softmax : [R, C] f32, or NULL when unused.
 * A label outside [0, C) makes that row's loss, and so the mean, NaN. */
int32_t _mlir_ciface_nova_hip_sce_f32(const NovaMemRef2D *logits,
                                      const NovaMemRef1D *labels,
                                      NovaMemRef1D *loss,
                                      NovaMemRef2D *softmax);

/* _mlir_ciface_nova_hip_sce_f32 for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference.  Same arguments,
 * kernels and results; the per-row losses go to a static array the library
 * holds per GPU for the life of the process (SCE_NOALLOC_MAX_ROWS floats,
 * 1 MiB) instead of a hipMalloc'd workspace, and the call makes no
 * allocation.  More than SCE_NOALLOC_MAX_ROWS rows: NOVA_HIP_ERANGE.
 * Calls on one GPU share the array: calls that overlap on one GPU (other
 * streams, other threads) race and must be serialised by the caller. */
#define SCE_NOALLOC_MAX_ROWS 262144
int32_t _mlir_ciface_nova_hip_sce_f32_noalloc(const NovaMemRef2D *logits,
                                              const NovaMemRef1D *labels,
                                              NovaMemRef1D *loss,
                                              NovaMemRef2D *softmax);

/* nova.sce forward and nova.sce_backward fused: the loss as
 * _mlir_ciface_nova_hip_sce_f32 computes it, and grad [R, C] f32 =
 * (softmax - onehot(labels)) * f32(1/R), bit-identical to feeding this
 * library's softmax to _mlir_ciface_nova_hip_sce_backward_f32 but without
 * writing and re-reading the softmax.  No reference counterpart as one op:
 * it is the pair nova.sce (NovaToLinalgGeneric.cpp:801-1010) then
 * nova.sce_backward (:1012-1137) on the sce's softmax result. */
int32_t _mlir_ciface_nova_hip_sce_fwd_bwd_f32(const NovaMemRef2D *logits,
                                              const NovaMemRef1D *labels,
                                              NovaMemRef1D *loss,
                                              NovaMemRef2D *grad);
/* ------------------------------------------------------------------------
 * Backward ops.
 * ---------------------------------------------------------------------- */
/* nova.sce_backward (NovaSceBackwardLowering, NovaToLinalgGeneric.cpp:
 * 1012-1137), class dim last:
 *   grad = (softmax + scatter(-1.0 at (r, labels[r]))) * f32(1.0 / R)
 * (one multiply by the f32-rounded reciprocal, :1121-1128).
 *   softmax, grad : [R, C] f32; labels : [R] i32.
 * A label outside [0, C) makes that row's gradient NaN (the reference's
 * scatter writes outside the row). */
int32_t _mlir_ciface_nova_hip_sce_backward_f32(const NovaMemRef2D *softmax,
                                               const NovaMemRef1D *labels,
                                               NovaMemRef2D *grad);
/* nova.layer_norm_backward (NovaLayerNormBackwardPattern,
 * NovaToLinalgGeneric.cpp:2128-2371) with the forward's saved stats:
 *   grad_y, x, dx : [R, D] f32; gamma, dgamma, dbeta : [D] f32;
 *   mean_sum, rstd : [R] f32 (the forward's second and third results).
 *   dx = ((gy*gamma - s1/D) - xhat * s2/D) * rstd, xhat = (x - S/D) * rstd,
 *   s1 = sum_d gy*gamma, s2 = sum_d gy*gamma*xhat;
 *   dgamma = sum_r gy*xhat, dbeta = sum_r gy.
 * dx, dgamma, dbeta may each be NULL.  D <= 8192.  The column sums are
 * deterministic (row blocks in order, then the blocks in order). */
int32_t _mlir_ciface_nova_hip_layer_norm_backward_f32(
    const NovaMemRef2D *grad_y, const NovaMemRef2D *x, const NovaMemRef1D *gamma,
    const NovaMemRef1D *mean_sum, const NovaMemRef1D *rstd, NovaMemRef2D *dx,
    NovaMemRef1D *dgamma, NovaMemRef1D *dbeta);
/* nova.linear_backward (NovaLinearBackwardPattern, NovaToLinalgGeneric.cpp:
 * 1824-1996) for weight [K, N] (the nova.linear convention):
 *   grad_input [M, K] = grad_out [M, N] . weight^T        (:1867-1911)
 *   grad_weight [K, N] = x^T . grad_out                    (:1913-1968)
 *   grad_bias [N] = sum_m grad_out[m, :]                   (:1970-1989)
 * Rank-3 inputs are passed flattened to [B*M, .], as the reference itself
 * collapses them for grad_weight.  weight may be a transposed view
 * (strides {1, K}); grad_weight may be a transposed view of a row-major
 * [N, K] buffer, which is then written as grad_out^T . x.  Any of the three
 * outputs may be NULL.  flags = NOVA_HIP_GEMM_FLAGS(in, out, NONE, 0): f32
 * in -> exact f32 kernel; bf16/f16 in -> MFMA, f32 accumulate, outputs (and
 * grad_bias) in the out dtype. */
int32_t _mlir_ciface_nova_hip_linear_backward(const NovaMemRef2D *grad_out,
                                              const NovaMemRef2D *x,
                                              const NovaMemRef2D *weight,
                                              NovaMemRef2D *grad_input,
                                              NovaMemRef2D *grad_weight,
                                              NovaMemRef1D *grad_bias,
                                              int32_t flags);
/* nova.matmul_backward (NovaMatmulBackwardPattern, NovaToLinalgGeneric.cpp:
 * 160-239), rank 2: grad_a [M, K] = grad [M, N] . B^T, grad_b [K, N] =
 * A^T . grad.  Outputs may be NULL or transposed views as above; flags as
 * for _mlir_ciface_nova_hip_linear_backward. */
int32_t _mlir_ciface_nova_hip_matmul_backward(const NovaMemRef2D *grad,
                                              const NovaMemRef2D *A,
                                              const NovaMemRef2D *B,
                                              NovaMemRef2D *grad_a,
                                              NovaMemRef2D *grad_b,
                                              int32_t flags);
/* ------------------------------------------------------------------------
 * Program glue: the elementwise, index and reduction ops a whole training
 * step needs around the GEMMs and row reductions (the reference's GPT step
 * ltest/test.mlir uses each of them), so that libnova_run can execute such
 * programs end to end.  All f32; dense operands read and written with
 * 16-byte accesses where aligned.
 * ---------------------------------------------------------------------- */
/* nova.add / nova.sub / nova.mul / nova.div (Nova_BinaryOp,
 * NovaOps.td:600-700; one IEEE operation per element, numpy-style
 * broadcasting): c = a (op) b over c's [4]-shaped index space, op a
 * NOVA_HIP_BIN_* code.  a and b give stride 0 on a broadcast dimension
 * (size 1 in the operand); c may alias a or b element for element (the
 * reference's in_place form). */
int32_t _mlir_ciface_nova_hip_binary_f32(const NovaMemRef4D *a, const NovaMemRef4D *b,
                                         NovaMemRef4D *c, int32_t op);
/* A splat nova.constant (NovaOps.td:331): out[i] = value for all i. */
int32_t _mlir_ciface_nova_hip_fill_f32(NovaMemRef1D *out, float value);
/* nova.gelu on its own (NovaGeluForwardPattern, NovaToLinalgGeneric.cpp:
 * 1277-1337), when its input has other uses and it cannot fold into the
 * GEMM epilogue: y = (0.5 x)(1 + tanh(0.7978845608028654 (x + 0.044715 x^3)))
 * in the reference's operation order.  x, y : [n], dense. */
int32_t _mlir_ciface_nova_hip_gelu_f32(const NovaMemRef1D *x, NovaMemRef1D *y);
/* nova.gelu_backward (NovaGeluBackwardPattern, NovaToLinalgGeneric.cpp:
 * 1339-1425): out = grad_out * (0.5 (1 + tanh(g)) + 0.5 x (1 - tanh(g)^2) g'),
 * g = 0.797884583 (x + 0.044715 x^3), g' = (1 + 0.134145 x^2) 0.797884583,
 * in the reference's operation order.  All [n], dense. */
int32_t _mlir_ciface_nova_hip_gelu_backward_f32(const NovaMemRef1D *grad_out,
                                                const NovaMemRef1D *x, NovaMemRef1D *out);
/* nova.gather along axis 0 (NovaGatherOpLowering, NovaToLinalgGeneric.cpp:
 * 2372-2471), the embedding lookup: out[i, :] = table[idx[i], :].
 *   table : [V, D] f32; idx : [n] of idx_dt (NOVA_HIP_DT_I16, zero-extended
 *   as the reference's ExtUIOp, :2434-2449; NOVA_HIP_DT_I32; NOVA_HIP_DT_I64);
 *   out : [n, D] f32.  An index outside [0, V) gives a NaN row. */
int32_t _mlir_ciface_nova_hip_gather_f32(const NovaMemRef2D *table, const NovaMemRef1D *idx,
                                         NovaMemRef2D *out, int32_t idx_dt);
/* nova.scatter_add along axis 0 (NovaScatterAddOpLowering, NovaToLinalg.cpp:
 * 1086-1290), in place: out[idx[i], :] += src[i, :] by f32 atomic adds, the
 * reference's memref.atomic_rmw addf; indices outside [0, V) are skipped as
 * its bounds check does.  The order of adds into one row is not fixed.
 *   out : [V, D] f32 (holds the op's `input` on entry); idx : [n] as for
 *   gather; src : [n, D] f32.  out must be device memory from hipMalloc
 *   (coarse-grained): the hardware f32 atomics are not defined on
 *   fine-grained host memory. */
int32_t _mlir_ciface_nova_hip_scatter_add_f32(NovaMemRef2D *out, const NovaMemRef1D *idx,
                                              const NovaMemRef2D *src, int32_t idx_dt);
/* nova.reduce<sum> over one dimension (Nova_ReduceOp, NovaOps.td:191-230):
 * x viewed as [outer, n, inner], out[o, i] = sum_j x[o, j, i] with j
 * ascending (one sequential sum per output, the linalg.reduce order). */
int32_t _mlir_ciface_nova_hip_reduce_sum_f32(const NovaMemRef3D *x, NovaMemRef2D *out);
/* Labels / indices to i32: NovaSceForwardLowering zero-extends non-i32
 * labels (NovaToLinalgGeneric.cpp:801-1010); narrow integers are
 * zero-extended, i64 truncated.  src : [n] of src_dt; dst : [n] i32. */
int32_t _mlir_ciface_nova_hip_index_to_i32(const NovaMemRef1D *src, NovaMemRef1D *dst,
                                           int32_t src_dt);
/* ------------------------------------------------------------------------
 * Typed aliases for lowered modules (nova-compiler_amd/mlir/
 * NovaHipLowering.cpp).  An MLIR module declares each callee once, with one
 * type, so the generic entry points above get one name per operand dtype
 * combination; the flags must name the same dtypes (NOVA_HIP_EINVAL
 * otherwise).  No reference counterpart: they are the symbols the lowering
 * emits in place of the NVPTX code generation of Passes.cpp:115-372.
 *   _mlir_ciface_nova_hip_gemm_<in>_<out>_b<bias>   (as _mlir_ciface_nova_hip_gemm)
 *   _mlir_ciface_nova_hip_linear_backward_<in>_<out>, _matmul_backward_<in>_<out>
 * with <in>, <out>, <bias> one of f32, bf16, f16 (backward: f32_f32 or a
 * 16-bit input with any output). */
#define NOVA_HIP_DECLARE_GEMM_ALIAS(SUF)                                          \
  int32_t _mlir_ciface_nova_hip_gemm_##SUF(const NovaMemRef3D *A,                 \
                                           const NovaMemRef3D *B, NovaMemRef3D *C, \
                                           const NovaMemRef1D *bias, int32_t flags);
#define NOVA_HIP_DECLARE_GEMM_ALIASES_OUT(I, O) \
  NOVA_HIP_DECLARE_GEMM_ALIAS(I##_##O##_bf32)   \
  NOVA_HIP_DECLARE_GEMM_ALIAS(I##_##O##_bbf16)  \
  NOVA_HIP_DECLARE_GEMM_ALIAS(I##_##O##_bf16)
#define NOVA_HIP_DECLARE_GEMM_ALIASES_IN(I)     \
  NOVA_HIP_DECLARE_GEMM_ALIASES_OUT(I, f32)     \
  NOVA_HIP_DECLARE_GEMM_ALIASES_OUT(I, bf16)    \
  NOVA_HIP_DECLARE_GEMM_ALIASES_OUT(I, f16)
NOVA_HIP_DECLARE_GEMM_ALIASES_IN(f32)
NOVA_HIP_DECLARE_GEMM_ALIASES_IN(bf16)
NOVA_HIP_DECLARE_GEMM_ALIASES_IN(f16)
#define NOVA_HIP_DECLARE_BWD_ALIAS(SUF)                                                       \
  int32_t _mlir_ciface_nova_hip_linear_backward_##SUF(                                        \
      const NovaMemRef2D *grad_out, const NovaMemRef2D *x, const NovaMemRef2D *weight,        \
      NovaMemRef2D *grad_input, NovaMemRef2D *grad_weight, NovaMemRef1D *grad_bias,          \
      int32_t flags);                                                                         \
  int32_t _mlir_ciface_nova_hip_matmul_backward_##SUF(                                        \
      const NovaMemRef2D *grad, const NovaMemRef2D *A, const NovaMemRef2D *B,                 \
      NovaMemRef2D *grad_a, NovaMemRef2D *grad_b, int32_t flags);
NOVA_HIP_DECLARE_BWD_ALIAS(f32_f32)
NOVA_HIP_DECLARE_BWD_ALIAS(bf16_f32)
NOVA_HIP_DECLARE_BWD_ALIAS(bf16_bf16)
NOVA_HIP_DECLARE_BWD_ALIAS(bf16_f16)
NOVA_HIP_DECLARE_BWD_ALIAS(f16_f32)
NOVA_HIP_DECLARE_BWD_ALIAS(f16_bf16)
NOVA_HIP_DECLARE_BWD_ALIAS(f16_f16)
/* _mlir_ciface_nova_hip_index_to_i32 by source element type (i16, i64). */
int32_t _mlir_ciface_nova_hip_index_to_i32_i16(const NovaMemRef1D *src, NovaMemRef1D *dst,
                                               int32_t src_dt);
int32_t _mlir_ciface_nova_hip_index_to_i32_i64(const NovaMemRef1D *src, NovaMemRef1D *dst,
                                               int32_t src_dt);
/* nova.sce whose softmax is unused (the op is Pure): the loss alone, as
 * _mlir_ciface_nova_hip_sce_f32 with a NULL softmax (a lowered module cannot
 * pass a null descriptor). */
int32_t _mlir_ciface_nova_hip_sce_loss_f32(const NovaMemRef2D *logits,
                                           const NovaMemRef1D *labels, NovaMemRef1D *loss);

/* ------------------------------------------------------------------------
 * Runtime.  The reference's host runtime is libmlir_cuda_runtime's mgpu*
 * calls plus cudaMallocAsync / cudaMemcpyAsync declared by FixGpuLaunch.cpp
 * (:49, :214); this library needs only a stream to launch on.
 * ---------------------------------------------------------------------- */

/* Stream (a hipStream_t) used by the calling thread's later launches. */
void nova_hip_set_stream(void *stream);
void *nova_hip_get_stream(void);
/* Wait for the calling thread's stream. */
int32_t nova_hip_synchronize(void);
/* Text of the calling thread's last error ("" if none). */
const char *nova_hip_last_error(void);
/* Library version string. */
const char *nova_hip_version(void);
/* Release the cached workspaces (e.g. before a process-level teardown). */
int32_t nova_hip_release_workspace(void);

#ifdef __cplusplus
}
#endif

#endif /* NOVA_HIP_H */
