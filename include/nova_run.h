/*
 * nova_run.h -- C ABI of libnova_run, an MLIR-free op->kernel planner and
 * executor for Nova programs written in the op surface this path serves.
 *
 * It reads the textual form nova-opt consumes (func.func bodies of
 * nova.matmul / nova.linear / nova.gelu / nova.cast / nova.transpose /
 * nova.layer_norm / nova.sce and their backward ops, linalg.matmul and
 * linalg.batch_matmul over a zero fill, tensor.empty, arith.constant, and
 * the bufferization.to_tensor / materialize_in_destination pair of
 * memref-argument entry functions such as ltest/test_gpu.mlir:1-9), plans
 * each op onto a libnova_hip entry point -- folding widening casts and
 * transposes into GEMM operands, and a following nova.gelu and narrowing
 * nova.cast into the GEMM epilogue -- and runs the plan on the GPU.  It is
 * the host side the reference's compiled modules get from
 * AddGpuMemoryCopies / ConvertMemRefToGpu / FixGpuLaunch plus its own
 * drivers (driver.cpp, robust_driver.cpp): device buffers, host<->device
 * copies, launches, one synchronisation at the end.  Ops outside the path
 * are refused with an error naming the op and line.
 *
 * dtype codes: 0 f32, 1 bf16, 2 f16 (as nova_hip.h), 3 i32, 4 i64.
 * Return value: 0 or a NOVA_HIP_E* code; text in nova_run_last_error().
 */
#ifndef NOVA_RUN_H
#define NOVA_RUN_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

typedef struct NovaRunProgram NovaRunProgram;

/* Parse a module's text; NULL on a syntax or type error. */
NovaRunProgram *nova_run_parse(const char *text);
void nova_run_free(NovaRunProgram *p);
const char *nova_run_last_error(void);

int32_t nova_run_num_funcs(const NovaRunProgram *p);
const char *nova_run_func_name(const NovaRunProgram *p, int32_t i);

/* Arguments and results of `func` (results in `return` order).  An
 * argument given as a writable memref output (bufferization
 * materialize_in_destination target) counts as an argument and is filled by
 * nova_run_execute. */
int32_t nova_run_num_args(const NovaRunProgram *p, const char *func);
int32_t nova_run_num_results(const NovaRunProgram *p, const char *func);
/* dtype code, rank and up to 8 dims of argument / result i. */
int32_t nova_run_arg_info(const NovaRunProgram *p, const char *func, int32_t i, int32_t *dtype,
                          int32_t *rank, int64_t *shape);
int32_t nova_run_result_info(const NovaRunProgram *p, const char *func, int32_t i,
                             int32_t *dtype, int32_t *rank, int64_t *shape);

/* The plan of `func` as text (one line per launch or view), written to buf
 * (truncated to len); needs no GPU.  Returns 0 or the error code. */
int32_t nova_run_plan(const NovaRunProgram *p, const char *func, char *buf, size_t len);

/* Run `func`: host_args[i] points to argument i's dense row-major host data,
 * host_results[i] to room for result i.  Copies in, launches on the calling
 * thread's libnova_hip stream, synchronises, copies out.  The device buffers
 * stay with the program and are reused by the next execution of the same
 * function (a training loop's repeated step); nova_run_free releases them.
 * Executions of one program are serialised. */
int32_t nova_run_execute(const NovaRunProgram *p, const char *func, const void *const *host_args,
                         void *const *host_results);

/* The reference's compiled entry points take memref arguments in address
 * space 1: device memory the caller allocated (ltest/test_gpu.mlir:2,
 * robust_driver.cpp:17-39, the packed _mlir_ciface_main(result, args) form
 * of GenerateDynamicWrapper.cpp:61-95).  This is that contract: dev_args[i]
 * is argument i's dense row-major data in device memory (a writable memref
 * argument is written in place), dev_results[i] device memory with room for
 * result i, which receives it.  Nothing is copied to or from the host;
 * launches are queued on the calling thread's libnova_hip stream and the
 * call returns without synchronising (nova_hip_synchronize waits).
 * Intermediates live in device buffers the program keeps and reuses on the
 * next execution, as for nova_run_execute.  Executions of one function share
 * those buffers, so each waits on the device (hipStreamWaitEvent, not on
 * the host) for the previous one to finish, whatever stream that ran on:
 * executions on several streams are ordered, never concurrent.  A plan
 * whose buffer sizes changed frees the old buffers only after the previous
 * execution has completed. */
int32_t nova_run_execute_device(const NovaRunProgram *p, const char *func,
                                void *const *dev_args, void *const *dev_results);

/* How f32 GEMMs (nova.matmul / nova.linear / linalg.matmul on f32 and their
 * backward ops) are planned.  EXACT (the default): sequential k with
 * separately rounded multiply and add, bit-identical to Nova's CPU pipeline
 * (Pipeline.cpp:61-187).  MFMA: the f32 matrix cores
 * (NOVA_HIP_GEMM_F32_MFMA of nova_hip.h), within the f32 parity bar (1e-4
 * relative) but not bit-identical, several times faster. */
enum { NOVA_RUN_F32_GEMM_EXACT = 0, NOVA_RUN_F32_GEMM_MFMA = 1 };
int32_t nova_run_set_f32_gemm(NovaRunProgram *p, int32_t mode);

#ifdef __cplusplus
}
#endif
#endif /* NOVA_RUN_H */
