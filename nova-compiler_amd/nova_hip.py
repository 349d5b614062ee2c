"""Python binding of libnova_hip (the C ABI in include/nova_hip.h).

Mirrors the Nova op surface the GPU path serves -- ``matmul`` (rank 2 and 3,
i.e. batch matmul), ``linear`` (+ GELU epilogue), ``layer_norm`` and ``sce``
-- with the reference's result conventions:

* ``layer_norm`` returns ``(y, mean_sum, rstd)``: NovaOps.td:1027-1037 names
  the results (output, mean_sum, var_sum) and the lowering puts rstd in the
  third (NovaToLinalgGeneric.cpp:2123).
* ``sce`` returns ``(softmax, loss)`` with ``loss`` of shape [1]
  (NovaOps.td:880-896, NovaToLinalgGeneric.cpp:1008).

Tensors are torch tensors on the GPU; each call passes MLIR strided-memref
descriptors built from the tensors' data pointers, sizes and strides, and
launches on torch's current stream.  There is no fallback: if the library is
missing or a call fails, an exception says so.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Tuple

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libnova_hip.so")

DT_F32, DT_BF16, DT_F16 = 0, 1, 2
DT_I32, DT_I64, DT_I16 = 3, 4, 5          # index / label operands of the glue ops
BIN_ADD, BIN_SUB, BIN_MUL, BIN_DIV = 0, 1, 2, 3
EPI_NONE, EPI_BIAS, EPI_BIAS_GELU, EPI_GELU = 0, 1, 2, 3

STATUS = {
    0: "SUCCESS", 1: "EINVAL", 2: "ESHAPE", 3: "ESTRIDE", 4: "EDTYPE",
    5: "ERANGE", 6: "EDEVICE", 7: "ENOMEM",
}

# Every symbol include/nova_hip.h declares.
EXPORTS = (
    "_mlir_ciface_nova_hip_gemm",
    "_mlir_ciface_nova_hip_matmul_f32",
    "_mlir_ciface_nova_hip_batch_matmul_f32",
    "_mlir_ciface_nova_hip_batch_matmul_bf16_f32",
    "_mlir_ciface_nova_hip_batch_matmul_f16_f32",
    "_mlir_ciface_nova_hip_matmul_bf16_f32",
    "_mlir_ciface_nova_hip_matmul_f16_f32",
    "_mlir_ciface_nova_hip_linear",
    "_mlir_ciface_nova_hip_linear_bf16_bias_gelu",
    "_mlir_ciface_nova_hip_layer_norm_f32",
    "_mlir_ciface_nova_hip_sce_f32",
    "_mlir_ciface_nova_hip_sce_f32_noalloc",
    "_mlir_ciface_nova_hip_sce_loss_f32",
    "_mlir_ciface_nova_hip_index_to_i32_i16",
    "_mlir_ciface_nova_hip_index_to_i32_i64",
    "_mlir_ciface_nova_hip_sce_fwd_bwd_f32",
    "_mlir_ciface_nova_hip_sce_backward_f32",
    "_mlir_ciface_nova_hip_layer_norm_backward_f32",
    "_mlir_ciface_nova_hip_linear_backward",
    "_mlir_ciface_nova_hip_matmul_backward",
    "_mlir_ciface_nova_hip_binary_f32",
    "_mlir_ciface_nova_hip_fill_f32",
    "_mlir_ciface_nova_hip_gelu_f32",
    "_mlir_ciface_nova_hip_gelu_backward_f32",
    "_mlir_ciface_nova_hip_gather_f32",
    "_mlir_ciface_nova_hip_scatter_add_f32",
    "_mlir_ciface_nova_hip_reduce_sum_f32",
    "_mlir_ciface_nova_hip_index_to_i32",
    "nova_hip_set_stream",
    "nova_hip_get_stream",
    "nova_hip_synchronize",
    "nova_hip_last_error",
    "nova_hip_version",
    "nova_hip_release_workspace",
)


GEMM_ACC_OUT = 0x10000  # NOVA_HIP_GEMM_ACC_OUT
GEMM_F32_MFMA = 0x20000  # NOVA_HIP_GEMM_F32_MFMA
GEMM_ACC_C = 0x40000  # NOVA_HIP_GEMM_ACC_C


def gemm_flags(in_dt: int, out_dt: int, epi: int = EPI_NONE, bias_dt: int = 0) -> int:
    """NOVA_HIP_GEMM_FLAGS of include/nova_hip.h."""
    return (in_dt & 0xF) | ((out_dt & 0xF) << 4) | ((epi & 0xF) << 8) | ((bias_dt & 0xF) << 12)


def _memref_type(rank: int):
    class MemRef(ctypes.Structure):
        _fields_ = [
            ("allocated", ctypes.c_void_p),
            ("aligned", ctypes.c_void_p),
            ("offset", ctypes.c_int64),
            ("sizes", ctypes.c_int64 * rank),
            ("strides", ctypes.c_int64 * rank),
        ]
    MemRef.__name__ = f"NovaMemRef{rank}D"
    return MemRef


MemRef1D = _memref_type(1)
MemRef2D = _memref_type(2)
MemRef3D = _memref_type(3)
MemRef4D = _memref_type(4)
_MEMREF = {1: MemRef1D, 2: MemRef2D, 3: MemRef3D, 4: MemRef4D}


def make_memref(ptr: int, sizes, strides, offset: int = 0):
    """Descriptor over raw memory (element offsets and strides)."""
    rank = len(sizes)
    d = _MEMREF[rank]()
    d.allocated = ptr
    d.aligned = ptr
    d.offset = offset
    for i in range(rank):
        d.sizes[i] = int(sizes[i])
        d.strides[i] = int(strides[i])
    return d


class NovaHipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"libnova_hip {STATUS.get(code, code)}: {msg}")
        self.code = code


_lib = None


def lib() -> ctypes.CDLL:
    """Load libnova_hip.so (built in-tree by the package Makefile)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `make -C nova-compiler_amd` "
            "(or __graft_entry__.build()); there is no fallback path")
    L = ctypes.CDLL(LIB_PATH)
    P = ctypes.c_void_p
    for name in EXPORTS:
        getattr(L, name)  # raises AttributeError if not exported
    L._mlir_ciface_nova_hip_gemm.argtypes = [P, P, P, P, ctypes.c_int32]
    L._mlir_ciface_nova_hip_linear.argtypes = [P, P, P, P, ctypes.c_int32]
    L._mlir_ciface_nova_hip_linear_bf16_bias_gelu.argtypes = [P, P, P, P]
    for n in ("matmul_f32", "batch_matmul_f32", "batch_matmul_bf16_f32",
              "batch_matmul_f16_f32", "matmul_bf16_f32", "matmul_f16_f32"):
        getattr(L, "_mlir_ciface_nova_hip_" + n).argtypes = [P, P, P]
    L._mlir_ciface_nova_hip_layer_norm_f32.argtypes = [P, P, P, P, P, P, ctypes.c_float]
    L._mlir_ciface_nova_hip_sce_f32.argtypes = [P, P, P, P]
    L._mlir_ciface_nova_hip_sce_fwd_bwd_f32.argtypes = [P, P, P, P]
    L._mlir_ciface_nova_hip_sce_backward_f32.argtypes = [P, P, P]
    L._mlir_ciface_nova_hip_layer_norm_backward_f32.argtypes = [P, P, P, P, P, P, P, P]
    L._mlir_ciface_nova_hip_linear_backward.argtypes = [P, P, P, P, P, P, ctypes.c_int32]
    L._mlir_ciface_nova_hip_matmul_backward.argtypes = [P, P, P, P, P, ctypes.c_int32]
    L._mlir_ciface_nova_hip_binary_f32.argtypes = [P, P, P, ctypes.c_int32]
    L._mlir_ciface_nova_hip_fill_f32.argtypes = [P, ctypes.c_float]
    L._mlir_ciface_nova_hip_gelu_f32.argtypes = [P, P]
    L._mlir_ciface_nova_hip_gelu_backward_f32.argtypes = [P, P, P]
    L._mlir_ciface_nova_hip_gather_f32.argtypes = [P, P, P, ctypes.c_int32]
    L._mlir_ciface_nova_hip_scatter_add_f32.argtypes = [P, P, P, ctypes.c_int32]
    L._mlir_ciface_nova_hip_reduce_sum_f32.argtypes = [P, P]
    L._mlir_ciface_nova_hip_index_to_i32.argtypes = [P, P, ctypes.c_int32]
    for name in EXPORTS:
        if name.startswith("_mlir_ciface_"):
            getattr(L, name).restype = ctypes.c_int32
    L.nova_hip_set_stream.argtypes = [P]
    L.nova_hip_set_stream.restype = None
    L.nova_hip_get_stream.restype = P
    L.nova_hip_synchronize.restype = ctypes.c_int32
    L.nova_hip_last_error.restype = ctypes.c_char_p
    L.nova_hip_version.restype = ctypes.c_char_p
    L.nova_hip_release_workspace.restype = ctypes.c_int32
    _lib = L
    return L


def check(rc: int) -> None:
    if rc != 0:
        raise NovaHipError(rc, lib().nova_hip_last_error().decode())


def ref(d):
    """Pointer argument to descriptor d (None passes NULL).  ctypes.byref is
    accepted for the c_void_p parameters and costs ~0.1 us against ~3 us
    for cast(pointer(d)); it keeps d alive for the call."""
    return None if d is None else ctypes.byref(d)


# --------------------------------------------------------------------------
# torch-facing wrappers
# --------------------------------------------------------------------------

def _torch():
    import torch
    return torch


def _dt(t) -> int:
    torch = _torch()
    if t.dtype == torch.float32:
        return DT_F32
    if t.dtype == torch.bfloat16:
        return DT_BF16
    if t.dtype == torch.float16:
        return DT_F16
    raise NovaHipError(4, f"unsupported dtype {t.dtype}")


def _torch_dtype(dt: int):
    torch = _torch()
    return {DT_F32: torch.float32, DT_BF16: torch.bfloat16, DT_F16: torch.float16}[dt]


def memref_of(t):
    """Descriptor of a torch tensor (element strides, offset folded into ptr)."""
    return make_memref(t.data_ptr(), tuple(t.shape), tuple(t.stride()), 0)


def _bind_stream() -> None:
    torch = _torch()
    lib().nova_hip_set_stream(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


def _as3(t):
    return t if t.dim() == 3 else t.unsqueeze(0)


def gemm(A, B, out=None, *, bias=None, epilogue: int = EPI_NONE, out_dtype=None,
         acc_out: bool = False, f32_mfma: bool = False, acc_c: bool = False):
    """Batched GEMM through _mlir_ciface_nova_hip_gemm.

    A [Bt,M,K] or [M,K]; B [Bt,K,N] or [K,N] (any unit-stride layout,
    transposed views included); returns C [Bt,M,N] (or [M,N] for rank-2
    inputs) in ``out_dtype`` (f32 by default).  ``acc_out``: accumulate in
    the output dtype (NOVA_HIP_GEMM_ACC_OUT; bf16 / f16 in and out).
    ``f32_mfma``: f32 operands on the f32 matrix cores (NOVA_HIP_GEMM_F32_MFMA;
    within 1e-4, not bit-identical to the sequential-k reference).
    ``acc_c``: ``out`` holds the accumulators' initial values and receives
    out + A . B in place (NOVA_HIP_GEMM_ACC_C, linalg.matmul on data-holding
    outs; f32, or 16-bit with ``acc_out``).
    """
    torch = _torch()
    in_dt = _dt(A)
    if acc_c and out is None:
        raise NovaHipError(1, "acc_c accumulates into a given out tensor")
    if _dt(B) != in_dt:
        raise NovaHipError(4, "A and B must share a dtype")
    rank2 = A.dim() == 2 and B.dim() == 2
    A3, B3 = _as3(A), _as3(B)
    batch = max(A3.shape[0], B3.shape[0])
    od = DT_F32 if out_dtype is None else _dt(torch.empty(0, dtype=out_dtype))
    if out is None:
        out = torch.empty((batch, A3.shape[1], B3.shape[2]), dtype=_torch_dtype(od),
                          device=A.device)
        C3 = out
    else:
        od = _dt(out)
        C3 = _as3(out)
    bias_dt = _dt(bias) if bias is not None else 0
    flags = (gemm_flags(in_dt, od, epilogue, bias_dt) | (GEMM_ACC_OUT if acc_out else 0)
             | (GEMM_F32_MFMA if f32_mfma else 0) | (GEMM_ACC_C if acc_c else 0))
    dA, dB, dC = memref_of(A3), memref_of(B3), memref_of(C3)
    dbias = memref_of(bias) if bias is not None else None
    _bind_stream()
    check(lib()._mlir_ciface_nova_hip_gemm(ref(dA), ref(dB), ref(dC), ref(dbias), flags))
    return out[0] if (rank2 and out.dim() == 3) else out


def matmul(A, B, out=None):
    """nova.matmul (rank 2 or 3) with f32 accumulate and f32 result."""
    return gemm(A, B, out)


def batch_matmul(A, B, out=None):
    return gemm(A, B, out)


def linear(x, weight, bias, *, gelu: bool = False, out_dtype=None):
    """nova.linear: x [M,K] . weight [K,N] + bias [N] (weight may be a
    transposed view of a row-major [N,K] tensor), optional GELU(tanh)."""
    torch = _torch()
    od = out_dtype if out_dtype is not None else x.dtype
    y = torch.empty((x.shape[0], weight.shape[1]), dtype=od, device=x.device)
    epi = EPI_BIAS_GELU if gelu else EPI_BIAS
    flags = gemm_flags(_dt(x), _dt(y), epi, _dt(bias))
    dx, dw, db, dy = memref_of(x), memref_of(weight), memref_of(bias), memref_of(y)
    _bind_stream()
    check(lib()._mlir_ciface_nova_hip_linear(ref(dx), ref(dw), ref(db), ref(dy), flags))
    return y


def layer_norm(x, gamma, beta, eps: float = 1e-5, *, y=None, mean_sum=None, rstd=None):
    """nova.layer_norm over the last dim: returns (y, mean_sum, rstd)."""
    torch = _torch()
    shape = x.shape
    x2 = x.reshape(-1, shape[-1])
    if y is None:
        y = torch.empty_like(x2)
    if mean_sum is None:
        mean_sum = torch.empty(x2.shape[0], dtype=torch.float32, device=x.device)
    if rstd is None:
        rstd = torch.empty(x2.shape[0], dtype=torch.float32, device=x.device)
    d = [memref_of(t) for t in (x2, gamma, beta, y, mean_sum, rstd)]
    _bind_stream()
    check(lib()._mlir_ciface_nova_hip_layer_norm_f32(*[ref(v) for v in d], ctypes.c_float(eps)))
    return y.reshape(shape), mean_sum.reshape(shape[:-1]), rstd.reshape(shape[:-1])


def sce(logits, labels, *, softmax: bool = False, loss=None, noalloc: bool = False, sm=None):
    """nova.sce: returns (softmax or None, loss[1]).  ``noalloc``: through
    _mlir_ciface_nova_hip_sce_f32_noalloc (row losses in the library's static
    per-GPU array; at most SCE_NOALLOC_MAX_ROWS rows)."""
    torch = _torch()
    if loss is None:
        loss = torch.empty(1, dtype=torch.float32, device=logits.device)
    if sm is None and softmax:
        sm = torch.empty_like(logits)
    dl, dt, dloss = memref_of(logits), memref_of(labels), memref_of(loss)
    dsm = memref_of(sm) if sm is not None else None
    _bind_stream()
    fn = (lib()._mlir_ciface_nova_hip_sce_f32_noalloc if noalloc
          else lib()._mlir_ciface_nova_hip_sce_f32)
    check(fn(ref(dl), ref(dt), ref(dloss), ref(dsm)))
    return sm, loss


def synchronize() -> None:
    _bind_stream()
    check(lib().nova_hip_synchronize())


def version() -> str:
    return lib().nova_hip_version().decode()


def sce_fwd_bwd(logits, labels, *, loss=None, grad=None):
    """nova.sce then nova.sce_backward in one pass: returns (loss[1], grad)."""
    torch = _torch()
    if loss is None:
        loss = torch.empty(1, dtype=torch.float32, device=logits.device)
    if grad is None:
        grad = torch.empty_like(logits)
    d = [memref_of(t) for t in (logits, labels, loss, grad)]
    _bind_stream()
    check(lib()._mlir_ciface_nova_hip_sce_fwd_bwd_f32(*[ref(v) for v in d]))
    return loss, grad


def sce_backward(softmax, labels, *, grad=None):
    """nova.sce_backward: (softmax - onehot(labels)) * f32(1 / rows)."""
    torch = _torch()
    if grad is None:
        grad = torch.empty_like(softmax)
    d = [memref_of(t) for t in (softmax, labels, grad)]
    _bind_stream()
    check(lib()._mlir_ciface_nova_hip_sce_backward_f32(*[ref(v) for v in d]))
    return grad


def layer_norm_backward(grad_y, x, gamma, mean_sum, rstd, *, dx=None, dgamma=None, dbeta=None,
                        want=(True, True, True)):
    """nova.layer_norm_backward: returns (dx, dgamma, dbeta); an output
    whose ``want`` flag is False is not computed (None)."""
    torch = _torch()
    shape = x.shape
    x2, g2 = x.reshape(-1, shape[-1]), grad_y.reshape(-1, shape[-1])
    if dx is None and want[0]:
        dx = torch.empty_like(x2)
    if dgamma is None and want[1]:
        dgamma = torch.empty(shape[-1], dtype=torch.float32, device=x.device)
    if dbeta is None and want[2]:
        dbeta = torch.empty(shape[-1], dtype=torch.float32, device=x.device)
    d = [memref_of(t) if t is not None else None
         for t in (g2, x2, gamma, mean_sum.reshape(-1), rstd.reshape(-1), dx, dgamma, dbeta)]
    _bind_stream()
    check(lib()._mlir_ciface_nova_hip_layer_norm_backward_f32(*[ref(v) for v in d]))
    return (dx.reshape(shape) if dx is not None else None), dgamma, dbeta


def linear_backward(grad_out, x, weight, *, out_dtype=None, grad_input=None, grad_weight=None,
                    grad_bias=None, want=(True, True, True), f32_mfma: bool = False):
    """nova.linear_backward for weight [K, N]: returns (grad_input [M,K],
    grad_weight [K,N], grad_bias [N]).  ``grad_weight`` may be passed as a
    transposed view of a row-major [N, K] tensor."""
    torch = _torch()
    od = out_dtype if out_dtype is not None else torch.float32
    M, K, N = x.shape[0], x.shape[1], weight.shape[1]
    if grad_input is None and want[0]:
        grad_input = torch.empty((M, K), dtype=od, device=x.device)
    if grad_weight is None and want[1]:
        grad_weight = torch.empty((K, N), dtype=od, device=x.device)
    if grad_bias is None and want[2]:
        grad_bias = torch.empty(N, dtype=od, device=x.device)
    flags = gemm_flags(_dt(x), _dt(torch.empty(0, dtype=od))) | (GEMM_F32_MFMA if f32_mfma else 0)
    d = [memref_of(t) if t is not None else None
         for t in (grad_out, x, weight, grad_input, grad_weight, grad_bias)]
    _bind_stream()
    check(lib()._mlir_ciface_nova_hip_linear_backward(*[ref(v) for v in d], flags))
    return grad_input, grad_weight, grad_bias


def matmul_backward(grad, A, B, *, out_dtype=None, grad_a=None, grad_b=None,
                    f32_mfma: bool = False):
    """nova.matmul_backward (rank 2): returns (grad . B^T, A^T . grad)."""
    torch = _torch()
    od = out_dtype if out_dtype is not None else torch.float32
    if grad_a is None:
        grad_a = torch.empty(tuple(A.shape), dtype=od, device=A.device)
    if grad_b is None:
        grad_b = torch.empty(tuple(B.shape), dtype=od, device=A.device)
    flags = gemm_flags(_dt(A), _dt(torch.empty(0, dtype=od))) | (GEMM_F32_MFMA if f32_mfma else 0)
    d = [memref_of(t) for t in (grad, A, B, grad_a, grad_b)]
    _bind_stream()
    check(lib()._mlir_ciface_nova_hip_matmul_backward(*[ref(v) for v in d], flags))
    return grad_a, grad_b


# --------------------------------------------------------------------------
# program glue (nova.add / mul / ..., constant, gelu, gelu_backward, gather,
# scatter_add, reduce<sum>, label widening)
# --------------------------------------------------------------------------

def _index_dt(t) -> int:
    torch = _torch()
    m = {torch.int16: DT_I16, torch.int32: DT_I32, torch.int64: DT_I64}
    if t.dtype not in m:
        raise NovaHipError(4, f"unsupported index dtype {t.dtype}")
    return m[t.dtype]


def _memref4(t, shape):
    """4-D descriptor of t broadcast (right-aligned) to `shape`: stride 0 on
    the dims t lacks or has as 1."""
    pad = 4 - len(shape)
    full = (1,) * pad + tuple(shape)
    ts = (1,) * (4 - t.dim()) + tuple(t.shape)
    st = (0,) * (4 - t.dim()) + tuple(t.stride())
    return make_memref(t.data_ptr(), full, [0 if ts[i] == 1 else st[i] for i in range(4)], 0)


def binary(a, b, op: int, out=None):
    """nova.add / sub / mul / div with numpy-style broadcasting (f32)."""
    torch = _torch()
    shape = torch.broadcast_shapes(a.shape, b.shape)
    if len(shape) > 4:
        raise NovaHipError(2, "binary: rank above 4")
    if out is None:
        out = torch.empty(shape, dtype=torch.float32, device=a.device)
    d = [_memref4(a, shape), _memref4(b, shape), _memref4(out, shape)]
    _bind_stream()
    check(lib()._mlir_ciface_nova_hip_binary_f32(*[ref(v) for v in d], op))
    return out


def fill(out, value: float):
    """A splat nova.constant written into `out` (dense f32)."""
    d = make_memref(out.data_ptr(), (out.numel(),), (1,), 0)
    _bind_stream()
    check(lib()._mlir_ciface_nova_hip_fill_f32(ref(d), float(value)))
    return out


def gelu(x, out=None):
    """nova.gelu on its own (the reference's tanh form)."""
    torch = _torch()
    if out is None:
        out = torch.empty_like(x)
    d = [make_memref(t.data_ptr(), (t.numel(),), (1,), 0) for t in (x, out)]
    _bind_stream()
    check(lib()._mlir_ciface_nova_hip_gelu_f32(*[ref(v) for v in d]))
    return out


def gelu_backward(grad_out, x, out=None):
    """nova.gelu_backward(grad_out, input)."""
    torch = _torch()
    if out is None:
        out = torch.empty_like(x)
    d = [make_memref(t.data_ptr(), (t.numel(),), (1,), 0) for t in (grad_out, x, out)]
    _bind_stream()
    check(lib()._mlir_ciface_nova_hip_gelu_backward_f32(*[ref(v) for v in d]))
    return out


def gather(table, idx, out=None):
    """nova.gather along axis 0: table[idx] (idx of any shape; i16 / i32 /
    i64, narrow types zero-extended)."""
    torch = _torch()
    flat = idx.reshape(-1)
    if out is None:
        out = torch.empty((flat.numel(), table.shape[1]), dtype=torch.float32,
                          device=table.device)
    d = [memref_of(table), memref_of(flat), memref_of(out.reshape(-1, table.shape[1]))]
    _bind_stream()
    check(lib()._mlir_ciface_nova_hip_gather_f32(*[ref(v) for v in d], _index_dt(idx)))
    return out.reshape(tuple(idx.shape) + (table.shape[1],))


def scatter_add(base, idx, src, out=None):
    """nova.scatter_add along axis 0: a copy of base with src[i] added into
    row idx[i] (f32 atomics; in place when out is base)."""
    if out is None:
        out = base.clone()
    elif out.data_ptr() != base.data_ptr():
        out.copy_(base)
    flat = idx.reshape(-1)
    d = [memref_of(out), memref_of(flat), memref_of(src.reshape(flat.numel(), -1))]
    _bind_stream()
    check(lib()._mlir_ciface_nova_hip_scatter_add_f32(*[ref(v) for v in d], _index_dt(idx)))
    return out


def reduce_sum(x, dim: int, out=None):
    """nova.reduce<sum> over one dimension (keepdims false)."""
    torch = _torch()
    dim = dim % x.dim()
    outer = 1
    for s in x.shape[:dim]:
        outer *= s
    inner = 1
    for s in x.shape[dim + 1:]:
        inner *= s
    rshape = tuple(x.shape[:dim]) + tuple(x.shape[dim + 1:])
    if out is None:
        out = torch.empty(rshape, dtype=torch.float32, device=x.device)
    xc = x.contiguous()
    dx = make_memref(xc.data_ptr(), (outer, x.shape[dim], inner),
                     (x.shape[dim] * inner, inner, 1), 0)
    do = make_memref(out.data_ptr(), (outer, inner), (inner, 1), 0)
    _bind_stream()
    check(lib()._mlir_ciface_nova_hip_reduce_sum_f32(ref(dx), ref(do)))
    return out


def index_to_i32(idx, out=None):
    """Labels / indices widened (narrow: zero-extended) or truncated to i32."""
    torch = _torch()
    flat = idx.reshape(-1)
    if out is None:
        out = torch.empty(flat.numel(), dtype=torch.int32, device=idx.device)
    d = [memref_of(flat), memref_of(out)]
    _bind_stream()
    check(lib()._mlir_ciface_nova_hip_index_to_i32(*[ref(v) for v in d], _index_dt(idx)))
    return out.reshape(idx.shape)
