"""ctypes binding of the CPU oracle (oracle/nova_cpu_ref.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
bench's cpu_baseline leg, as the checker or the timed CPU baseline.  Never
used by the product path.  Function semantics and their reference citations
are documented in nova_cpu_ref.c.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libnova_cpu_ref.so")
F32, BF16, F16 = 0, 1, 2
EPI_NONE, EPI_BIAS, EPI_BIAS_GELU, EPI_GELU = 0, 1, 2, 3

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.nova_ref_gemm.argtypes = [P, I, I64, I64, I64, P, I, I64, I64, I64, P, I, I, P, I,
                                    I64, I64, I64, I64]
        L.nova_ref_gemm.restype = I
        L.nova_ref_gemm_sampled.argtypes = [P, I, I64, I64, I64, P, I, I64, I64, I64, P, I, I,
                                            I, I64, P, I64, P]
        L.nova_ref_gemm_sampled.restype = I
        L.nova_ref_gemm_accumulate.argtypes = [P, I, I64, I64, I64, P, I, I64, I64, I64, P, I,
                                               I64, I64, I64, I64]
        L.nova_ref_gemm_accumulate.restype = I
        L.nova_ref_gelu_f32.argtypes = [ctypes.c_float]
        L.nova_ref_gelu_f32.restype = ctypes.c_float
        L.nova_ref_gelu_array.argtypes = [P, P, I64]
        L.nova_ref_layer_norm_f32.argtypes = [P, P, P, P, P, P, I64, I64, ctypes.c_float]
        L.nova_ref_layer_norm_f32.restype = I
        L.nova_ref_mean_f32.argtypes = [P, I64]
        L.nova_ref_mean_f32.restype = ctypes.c_float
        L.nova_ref_sce_f32.argtypes = [P, P, I64, I64, P, P, P]
        L.nova_ref_sce_f32.restype = I
        L.nova_ref_sce_backward_f32.argtypes = [P, P, I64, I64, P]
        L.nova_ref_sce_backward_f32.restype = I
        L.nova_ref_layer_norm_backward_f32.argtypes = [P, P, P, P, P, P, P, P, I64, I64]
        L.nova_ref_layer_norm_backward_f32.restype = I
        L.nova_ref_col_sum.argtypes = [P, I, I64, I64, I64, P]
        L.nova_ref_col_sum.restype = I
        L.nova_ref_f32_to_bf16.argtypes = [ctypes.c_float]
        L.nova_ref_f32_to_bf16.restype = ctypes.c_uint16
        L.nova_ref_f32_to_f16.argtypes = [ctypes.c_float]
        L.nova_ref_f32_to_f16.restype = ctypes.c_uint16
        L.nova_ref_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.nova_ref_bf16_to_f32.restype = ctypes.c_float
        L.nova_ref_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.nova_ref_f16_to_f32.restype = ctypes.c_float
        L.nova_ref_binary_f32.argtypes = [P, P, P, I64, I]
        L.nova_ref_binary_f32.restype = I
        L.nova_ref_gemm_acc_out.argtypes = [P, P, I64, I64, I64, I64, I64, I64, P, I, P, I,
                                            I64, I64, I64, I64]
        L.nova_ref_gemm_acc_out.restype = I
        L.nova_ref_gelu_backward_f32.argtypes = [ctypes.c_float, ctypes.c_float]
        L.nova_ref_gelu_backward_f32.restype = ctypes.c_float
        L.nova_ref_gelu_backward_array.argtypes = [P, P, P, I64]
        L.nova_ref_gather_f32.argtypes = [P, I64, I64, P, I, I64, P]
        L.nova_ref_gather_f32.restype = I
        L.nova_ref_scatter_add_f32.argtypes = [P, I64, I64, P, I, I64, P]
        L.nova_ref_scatter_add_f32.restype = I
        L.nova_ref_reduce_sum_f32.argtypes = [P, I64, I64, I64, P]
        L.nova_ref_reduce_sum_f32.restype = I
        L.nova_ref_index_to_i32.argtypes = [P, I, I64, P]
        L.nova_ref_index_to_i32.restype = I
        _lib = L
    return _lib


def _dtcode(a: np.ndarray, dt: int | None) -> int:
    if dt is not None:
        return dt
    if a.dtype == np.float32:
        return F32
    raise ValueError("uint16 arrays need an explicit dtype code (BF16 or F16)")


def _strides(a: np.ndarray):
    return [s // a.itemsize for s in a.strides]


def _gemm_args(A, B, adt, bdt):
    """(A ptr, dt, sab, sam, sak, B ptr, dt, sbb, sbk, sbn, batch, M, N, K) for
    A [Bt,M,K] / [M,K] and B [Bt,K,N] / [K,N] numpy views (any strides)."""
    A3 = A if A.ndim == 3 else A[None]
    B3 = B if B.ndim == 3 else B[None]
    sa, sb = _strides(A3), _strides(B3)
    if A3.shape[0] == 1:
        sa[0] = 0
    if B3.shape[0] == 1:
        sb[0] = 0
    batch = max(A3.shape[0], B3.shape[0])
    M, K = A3.shape[1], A3.shape[2]
    N = B3.shape[2]
    assert B3.shape[1] == K
    return (A3.ctypes.data, _dtcode(A, adt), sa[0], sa[1], sa[2],
            B3.ctypes.data, _dtcode(B, bdt), sb[0], sb[1], sb[2], batch, M, N, K)


def gemm(A, B, *, adt=None, bdt=None, bias=None, biasdt=None, epilogue=EPI_NONE,
         cdt=F32) -> np.ndarray:
    """Reference GEMM; returns C [Bt,M,N] (f32, or uint16 bits for bf16/f16)."""
    (pa, da, sab, sam, sak, pb, db, sbb, sbk, sbn, batch, M, N, K) = _gemm_args(A, B, adt, bdt)
    C = np.empty((batch, M, N), dtype=np.float32 if cdt == F32 else np.uint16)
    pbias = bias.ctypes.data if bias is not None else None
    bdtc = _dtcode(bias, biasdt) if bias is not None else 0
    rc = lib().nova_ref_gemm(pa, da, sab, sam, sak, pb, db, sbb, sbk, sbn, pbias, bdtc,
                             epilogue, C.ctypes.data, cdt, batch, M, N, K)
    assert rc == 0, rc
    return C


def gemm_acc_out(A, B, *, dt, bias=None) -> np.ndarray:
    """linalg.matmul with bf16 / f16 outs: the accumulator in dtype dt
    (inputs of that dtype as uint16 bits); returns C [Bt,M,N] uint16 bits."""
    (pa, da, sab, sam, sak, pb, db, sbb, sbk, sbn, batch, M, N, K) = _gemm_args(A, B, dt, dt)
    C = np.empty((batch, M, N), dtype=np.uint16)
    pbias = bias.ctypes.data if bias is not None else None
    rc = lib().nova_ref_gemm_acc_out(pa, pb, sab, sam, sak, sbb, sbk, sbn, pbias,
                                     EPI_BIAS if bias is not None else EPI_NONE,
                                     C.ctypes.data, dt, batch, M, N, K)
    assert rc == 0, rc
    return C


def gemm_accumulate(A, B, C0, *, adt=None, bdt=None, cdt=F32) -> np.ndarray:
    """linalg.matmul / batch_matmul on data-holding outs: C0 + A . B with
    each sum starting from C0's element, k ascending; C0 [Bt,M,N] (f32, or
    uint16 bits when cdt is bf16 / f16, then equal to adt and bdt).
    Returns a new array; C0 is not modified."""
    (pa, da, sab, sam, sak, pb, db, sbb, sbk, sbn, batch, M, N, K) = _gemm_args(A, B, adt, bdt)
    C = np.array(C0, dtype=np.float32 if cdt == F32 else np.uint16, copy=True).reshape(batch, M, N)
    C = np.ascontiguousarray(C)
    rc = lib().nova_ref_gemm_accumulate(pa, da, sab, sam, sak, pb, db, sbb, sbk, sbn,
                                        C.ctypes.data, cdt, batch, M, N, K)
    assert rc == 0, rc
    return C


def gemm_sampled(A, B, idx: np.ndarray, *, adt=None, bdt=None, bias=None, biasdt=None,
                 epilogue=EPI_NONE, cdt=F32) -> np.ndarray:
    """Reference values at idx[t] = (b, i, j), as f32 (already rounded to cdt)."""
    (pa, da, sab, sam, sak, pb, db, sbb, sbk, sbn, batch, M, N, K) = _gemm_args(A, B, adt, bdt)
    idx = np.ascontiguousarray(idx, dtype=np.int64)
    out = np.empty(idx.shape[0], dtype=np.float32)
    pbias = bias.ctypes.data if bias is not None else None
    bdtc = _dtcode(bias, biasdt) if bias is not None else 0
    rc = lib().nova_ref_gemm_sampled(pa, da, sab, sam, sak, pb, db, sbb, sbk, sbn, pbias, bdtc,
                                     epilogue, cdt, K, idx.ctypes.data, idx.shape[0],
                                     out.ctypes.data)
    assert rc == 0, rc
    return out


def gelu(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().nova_ref_gelu_array(x.ctypes.data, y.ctypes.data, x.size)
    return y


def layer_norm(x: np.ndarray, gamma: np.ndarray, beta: np.ndarray, eps: float = 1e-5):
    """Returns (y, mean_sum, rstd) like nova.layer_norm."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    R, D = x.shape
    y = np.empty_like(x)
    s = np.empty(R, dtype=np.float32)
    r = np.empty(R, dtype=np.float32)
    g = np.ascontiguousarray(gamma, dtype=np.float32)
    b = np.ascontiguousarray(beta, dtype=np.float32)
    rc = lib().nova_ref_layer_norm_f32(x.ctypes.data, g.ctypes.data, b.ctypes.data,
                                       y.ctypes.data, s.ctypes.data, r.ctypes.data, R, D,
                                       ctypes.c_float(eps))
    assert rc == 0
    return y, s, r


def mean(v: np.ndarray) -> np.float32:
    v = np.ascontiguousarray(v, dtype=np.float32)
    return np.float32(lib().nova_ref_mean_f32(v.ctypes.data, v.size))


def sce(logits: np.ndarray, labels: np.ndarray, softmax: bool = False):
    """Returns (softmax or None, loss[1], per-row loss)."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    t = np.ascontiguousarray(labels, dtype=np.int32)
    R, C = x.shape
    sm = np.empty_like(x) if softmax else None
    lr = np.empty(R, dtype=np.float32)
    loss = np.empty(1, dtype=np.float32)
    rc = lib().nova_ref_sce_f32(x.ctypes.data, t.ctypes.data, R, C,
                                sm.ctypes.data if sm is not None else None,
                                lr.ctypes.data, loss.ctypes.data)
    if rc == -2:
        raise ValueError("label outside [0, C)")
    assert rc == 0
    return sm, loss, lr


def sce_backward(softmax: np.ndarray, labels: np.ndarray) -> np.ndarray:
    """nova.sce_backward: (softmax - onehot(labels)) * float(1/rows)."""
    sm = np.ascontiguousarray(softmax, dtype=np.float32)
    t = np.ascontiguousarray(labels, dtype=np.int32)
    R, C = sm.shape
    g = np.empty_like(sm)
    rc = lib().nova_ref_sce_backward_f32(sm.ctypes.data, t.ctypes.data, R, C, g.ctypes.data)
    if rc == -2:
        raise ValueError("label outside [0, C)")
    assert rc == 0
    return g


def layer_norm_backward(gy, x, gamma, mean_sum, rstd):
    """nova.layer_norm_backward: returns (dx, dgamma, dbeta)."""
    gy = np.ascontiguousarray(gy, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    g = np.ascontiguousarray(gamma, dtype=np.float32)
    S = np.ascontiguousarray(mean_sum, dtype=np.float32)
    r = np.ascontiguousarray(rstd, dtype=np.float32)
    R, D = x.shape
    dx = np.empty_like(x)
    dg = np.empty(D, dtype=np.float32)
    db = np.empty(D, dtype=np.float32)
    rc = lib().nova_ref_layer_norm_backward_f32(gy.ctypes.data, x.ctypes.data, g.ctypes.data,
                                                S.ctypes.data, r.ctypes.data, dx.ctypes.data,
                                                dg.ctypes.data, db.ctypes.data, R, D)
    assert rc == 0
    return dx, dg, db


def col_sum(a: np.ndarray, dt=None) -> np.ndarray:
    """Sequential column sums of a 2-D array (f32, or uint16 bits with dt)."""
    a = np.ascontiguousarray(a)
    R, C = a.shape
    out = np.empty(C, dtype=np.float32)
    rc = lib().nova_ref_col_sum(a.ctypes.data, _dtcode(a, dt), R, C, C, out.ctypes.data)
    assert rc == 0
    return out


def linear_backward(grad_out, x, weight, *, dt=None):
    """nova.linear_backward with weight [K, N]: returns (grad_input [M,K],
    grad_weight [K,N], grad_bias [N]) in f32 (inputs f32, or uint16 bits with
    dt = BF16 / F16; f32 accumulate)."""
    gi = gemm(grad_out, weight.T, adt=dt, bdt=dt)[0]
    gw = gemm(x.T, grad_out, adt=dt, bdt=dt)[0]
    gb = col_sum(grad_out, dt)
    return gi, gw, gb


def matmul_backward(grad, A, B, *, dt=None):
    """nova.matmul_backward (rank 2): returns (grad_a = grad . B^T,
    grad_b = A^T . grad) in f32."""
    return gemm(grad, B.T, adt=dt, bdt=dt)[0], gemm(A.T, grad, adt=dt, bdt=dt)[0]


# ---- program glue ----------------------------------------------------------
I32, I64, I16 = 3, 4, 5
ADD, SUB, MUL, DIV = 0, 1, 2, 3


def _idx(idx: np.ndarray):
    idx = np.ascontiguousarray(idx.reshape(-1))
    m = {np.dtype(np.int16): I16, np.dtype(np.uint16): I16, np.dtype(np.int32): I32,
         np.dtype(np.int64): I64}
    return idx, m[idx.dtype]


def binary(a: np.ndarray, b: np.ndarray, op: int) -> np.ndarray:
    """nova.add / sub / mul / div with numpy-style broadcasting (f32)."""
    shape = np.broadcast_shapes(a.shape, b.shape)
    A = np.ascontiguousarray(np.broadcast_to(a.astype(np.float32, copy=False), shape))
    B = np.ascontiguousarray(np.broadcast_to(b.astype(np.float32, copy=False), shape))
    C = np.empty(shape, np.float32)
    assert lib().nova_ref_binary_f32(A.ctypes.data, B.ctypes.data, C.ctypes.data, C.size, op) == 0
    return C


def gelu_backward(grad_out: np.ndarray, x: np.ndarray) -> np.ndarray:
    go = np.ascontiguousarray(grad_out, np.float32)
    xx = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(xx)
    lib().nova_ref_gelu_backward_array(go.ctypes.data, xx.ctypes.data, out.ctypes.data, xx.size)
    return out


def gather(table: np.ndarray, idx: np.ndarray) -> np.ndarray:
    """nova.gather along axis 0 (NaN rows for indices outside the table)."""
    t = np.ascontiguousarray(table, np.float32)
    flat, dt = _idx(idx)
    out = np.empty((flat.size, t.shape[1]), np.float32)
    assert lib().nova_ref_gather_f32(t.ctypes.data, t.shape[0], t.shape[1], flat.ctypes.data, dt,
                                     flat.size, out.ctypes.data) == 0
    return out.reshape(tuple(idx.shape) + (t.shape[1],))


def scatter_add(base: np.ndarray, idx: np.ndarray, src: np.ndarray) -> np.ndarray:
    """nova.scatter_add along axis 0: base with src rows added in order."""
    out = np.array(base, np.float32, copy=True, order="C")
    flat, dt = _idx(idx)
    s = np.ascontiguousarray(src.reshape(flat.size, -1), np.float32)
    assert lib().nova_ref_scatter_add_f32(out.ctypes.data, out.shape[0], out.shape[1],
                                          flat.ctypes.data, dt, flat.size, s.ctypes.data) == 0
    return out


def reduce_sum(x: np.ndarray, dim: int) -> np.ndarray:
    """nova.reduce<sum> over one dimension, sequential."""
    x = np.ascontiguousarray(x, np.float32)
    dim = dim % x.ndim
    outer = int(np.prod(x.shape[:dim], dtype=np.int64))
    inner = int(np.prod(x.shape[dim + 1:], dtype=np.int64))
    out = np.empty(x.shape[:dim] + x.shape[dim + 1:], np.float32)
    assert lib().nova_ref_reduce_sum_f32(x.ctypes.data, outer, x.shape[dim], inner,
                                         out.ctypes.data) == 0
    return out


def index_to_i32(idx: np.ndarray) -> np.ndarray:
    flat, dt = _idx(idx)
    out = np.empty(flat.size, np.int32)
    assert lib().nova_ref_index_to_i32(flat.ctypes.data, dt, flat.size, out.ctypes.data) == 0
    return out.reshape(idx.shape)
