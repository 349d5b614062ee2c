"""ctypes binding of libnova_run (include/nova_run.h): parse a Nova program
written in the op surface of this path, print its launch plan, and run it
on the GPU through libnova_hip.

    import nova_run
    prog = nova_run.Program(open("model.mlir").read())
    print(prog.plan("linear_gelu"))
    outs = prog.run("linear_gelu", x_bits, w_bits, b_bits)   # numpy in, numpy out

Arrays are dense row-major numpy arrays: float32 for f32, uint16 bit
patterns for bf16 / f16, int32 / int64 for integer tensors.  There is no
fallback: a missing library or a refused op raises.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libnova_run.so")
NP_DTYPE = {0: np.float32, 1: np.uint16, 2: np.uint16, 3: np.int32, 4: np.int64, 5: np.int16}
DT_NAME = {0: "f32", 1: "bf16", 2: "f16", 3: "i32", 4: "i64", 5: "i16"}
F32_GEMM_EXACT, F32_GEMM_MFMA = 0, 1  # nova_run_set_f32_gemm modes


class _TorchDtypes(dict):
    def __missing__(self, dt):
        import torch
        self.update({0: torch.float32, 1: torch.bfloat16, 2: torch.float16, 3: torch.int32,
                     4: torch.int64, 5: torch.int16})
        return self[dt]


TORCH_DTYPE = _TorchDtypes()

_lib = None


class NovaRunError(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `make -C nova-compiler_amd`")
        L = ctypes.CDLL(LIB_PATH)
        P, S, I32 = ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int32
        L.nova_run_parse.argtypes = [S]
        L.nova_run_parse.restype = P
        L.nova_run_free.argtypes = [P]
        L.nova_run_last_error.restype = S
        L.nova_run_num_funcs.argtypes = [P]
        L.nova_run_num_funcs.restype = I32
        L.nova_run_func_name.argtypes = [P, I32]
        L.nova_run_func_name.restype = S
        for n in ("nova_run_num_args", "nova_run_num_results"):
            getattr(L, n).argtypes = [P, S]
            getattr(L, n).restype = I32
        for n in ("nova_run_arg_info", "nova_run_result_info"):
            getattr(L, n).argtypes = [P, S, I32, ctypes.POINTER(I32), ctypes.POINTER(I32),
                                      ctypes.POINTER(ctypes.c_int64)]
            getattr(L, n).restype = I32
        L.nova_run_plan.argtypes = [P, S, ctypes.c_char_p, ctypes.c_size_t]
        L.nova_run_plan.restype = I32
        L.nova_run_execute.argtypes = [P, S, ctypes.POINTER(P), ctypes.POINTER(P)]
        L.nova_run_execute.restype = I32
        L.nova_run_execute_device.argtypes = [P, S, ctypes.POINTER(P), ctypes.POINTER(P)]
        L.nova_run_execute_device.restype = I32
        L.nova_run_set_f32_gemm.argtypes = [P, I32]
        L.nova_run_set_f32_gemm.restype = I32
        _lib = L
    return _lib


def _err(what: str):
    raise NovaRunError(f"{what}: {lib().nova_run_last_error().decode()}")


class Program:
    def __init__(self, text: str):
        self._p = lib().nova_run_parse(text.encode())
        if not self._p:
            _err("parse")

    def __del__(self):
        if getattr(self, "_p", None):
            lib().nova_run_free(self._p)
            self._p = None

    def funcs(self):
        L = lib()
        return [L.nova_run_func_name(self._p, i).decode()
                for i in range(L.nova_run_num_funcs(self._p))]

    def _info(self, fn, func, i):
        dt, rank = ctypes.c_int32(), ctypes.c_int32()
        shape = (ctypes.c_int64 * 8)()
        if fn(self._p, func.encode(), i, ctypes.byref(dt), ctypes.byref(rank), shape):
            _err(f"@{func}")
        return dt.value, tuple(shape[d] for d in range(rank.value))

    def args(self, func: str):
        n = lib().nova_run_num_args(self._p, func.encode())
        if n < 0:
            _err(f"@{func}")
        return [self._info(lib().nova_run_arg_info, func, i) for i in range(n)]

    def results(self, func: str):
        n = lib().nova_run_num_results(self._p, func.encode())
        if n < 0:
            _err(f"@{func}")
        return [self._info(lib().nova_run_result_info, func, i) for i in range(n)]

    def plan(self, func: str) -> str:
        buf = ctypes.create_string_buffer(1 << 16)
        if lib().nova_run_plan(self._p, func.encode(), buf, len(buf)):
            _err(f"@{func}")
        return buf.value.decode()

    def set_f32_gemm(self, mode: int) -> None:
        """F32_GEMM_EXACT (bit-identical to the reference's CPU arithmetic) or
        F32_GEMM_MFMA (the f32 matrix cores, within 1e-4)."""
        if lib().nova_run_set_f32_gemm(self._p, mode):
            _err("set_f32_gemm")

    def run_device(self, func: str, *tensors, results=None):
        """Run `func` on torch device tensors through nova_run_execute_device:
        no host copies, launches queued on torch's current stream, no
        synchronisation.  Returns the result tensors (allocated here unless
        ``results`` gives them)."""
        import torch
        import nova_hip
        spec = self.args(func)
        if len(tensors) != len(spec):
            raise ValueError(f"@{func} takes {len(spec)} arguments, got {len(tensors)}")
        for t, (dt, shape) in zip(tensors, spec):
            if (tuple(t.shape) != shape or t.dtype != TORCH_DTYPE[dt] or not t.is_contiguous()
                    or not t.is_cuda):
                raise ValueError(f"argument needs a contiguous {DT_NAME[dt]} device tensor "
                                 f"of shape {shape}")
        rspec = self.results(func)
        if results is None:
            dev = tensors[0].device if tensors else torch.device("cuda", torch.cuda.current_device())
            results = [torch.empty(shape, dtype=TORCH_DTYPE[dt], device=dev) for dt, shape in rspec]
        else:
            # The kernels write each planned result's full byte size at its
            # data pointer: the tensors must be exactly the planned results.
            results = list(results)
            if len(results) != len(rspec):
                raise ValueError(f"@{func} has {len(rspec)} results, got {len(results)}")
            for r, (dt, shape) in zip(results, rspec):
                if (tuple(r.shape) != shape or r.dtype != TORCH_DTYPE[dt]
                        or not r.is_contiguous() or not r.is_cuda):
                    raise ValueError(f"result needs a contiguous {DT_NAME[dt]} device tensor "
                                     f"of shape {shape}")
        nova_hip._bind_stream()
        pin = (ctypes.c_void_p * max(len(tensors), 1))(*[t.data_ptr() for t in tensors])
        pout = (ctypes.c_void_p * max(len(results), 1))(*[r.data_ptr() for r in results])
        if lib().nova_run_execute_device(self._p, func.encode(), pin, pout):
            _err(f"@{func}")
        return results

    def run(self, func: str, *arrays):
        """Run `func` on host arrays; returns its results as numpy arrays.
        Writable memref arguments are filled in place."""
        spec = self.args(func)
        if len(arrays) != len(spec):
            raise ValueError(f"@{func} takes {len(spec)} arguments, got {len(arrays)}")
        ins = []
        for a, (dt, shape) in zip(arrays, spec):
            a = np.asarray(a)
            if a.shape != shape or a.dtype != NP_DTYPE[dt] or not a.flags.c_contiguous:
                raise ValueError(f"argument needs a contiguous {DT_NAME[dt]} array of shape {shape}")
            ins.append(a)
        outs = [np.empty(shape, NP_DTYPE[dt]) for dt, shape in self.results(func)]
        pin = (ctypes.c_void_p * max(len(ins), 1))(*[a.ctypes.data for a in ins])
        pout = (ctypes.c_void_p * max(len(outs), 1))(*[o.ctypes.data for o in outs])
        if lib().nova_run_execute(self._p, func.encode(), pin, pout):
            _err(f"@{func}")
        return outs
