"""Seeded synthetic inputs (binding of libnova_seed.so, host/nova_seed.c).

The generator is counter based (splitmix64 of seed and element counter), so
values are identical for any thread count and any machine with IEEE f64 libm;
see host/nova_seed.c for the exact recipe.  Arrays are numpy; bf16 and f16
are returned as uint16 bit patterns.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libnova_seed.so")
F32, BF16, F16 = 0, 1, 2

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} missing: run `make -C nova-compiler_amd`")
        L = ctypes.CDLL(LIB_PATH)
        P, I64, U64, F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float
        L.nova_seed_uniform.argtypes = [P, ctypes.c_int, I64, U64, U64, F, F]
        L.nova_seed_normal.argtypes = [P, ctypes.c_int, I64, U64, U64, F, F]
        L.nova_seed_labels.argtypes = [P, I64, U64, U64, ctypes.c_int32]
        L.nova_seed_round_f32.argtypes = [P, P, ctypes.c_int, I64]
        for f in (L.nova_seed_uniform, L.nova_seed_normal, L.nova_seed_labels,
                  L.nova_seed_round_f32):
            f.restype = ctypes.c_int
        _lib = L
    return _lib


def _alloc(shape, dtype):
    return np.empty(shape, dtype=np.float32 if dtype == F32 else np.uint16)


def uniform(shape, seed: int, lo: float = -1.0, hi: float = 1.0, dtype: int = F32,
            offset: int = 0) -> np.ndarray:
    out = _alloc(shape, dtype)
    rc = lib().nova_seed_uniform(out.ctypes.data, dtype, out.size, seed, offset, lo, hi)
    assert rc == 0
    return out


def normal(shape, seed: int, mean: float = 0.0, std: float = 1.0, dtype: int = F32,
           offset: int = 0) -> np.ndarray:
    out = _alloc(shape, dtype)
    rc = lib().nova_seed_normal(out.ctypes.data, dtype, out.size, seed, offset, mean, std)
    assert rc == 0
    return out


def labels(n: int, n_classes: int, seed: int, offset: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    rc = lib().nova_seed_labels(out.ctypes.data, n, seed, offset, n_classes)
    assert rc == 0
    return out


def round_to(x: np.ndarray, dtype: int) -> np.ndarray:
    """f32 -> bf16/f16 bit patterns, round to nearest even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    rc = lib().nova_seed_round_f32(x.ctypes.data, out.ctypes.data, dtype, x.size)
    assert rc == 0
    return out


def widen(bits: np.ndarray, dtype: int) -> np.ndarray:
    """bf16/f16 bit patterns -> f32 (exact)."""
    if dtype == BF16:
        return (bits.astype(np.uint32) << 16).view(np.float32)
    if dtype == F16:
        return bits.view(np.float16).astype(np.float32)
    return bits.astype(np.float32)


# The configs' inputs.  Tensors drawn from one seed
# form a continued stream: a uniform / label tensor of n elements at counter
# offset u uses counters [u, u+n); a normal tensor at element offset o uses
# counters [2o, 2(o+n)).  Offsets below keep every tensor's counters disjoint.
def config_inputs(name: str):
    """Host arrays for a named config (see the generator recipe above)."""
    if name == "c1":
        n = 256 * 256
        return {"A": uniform((256, 256), 0), "B": uniform((256, 256), 0, offset=n)}
    if name == "c2":
        n = 8 * 4096 * 4096
        return {"A": uniform((8, 4096, 4096), 1, dtype=BF16),
                "B": uniform((8, 4096, 4096), 1, dtype=BF16, offset=n)}
    if name == "c3":
        nx, nw = 4096 * 4096, 11008 * 4096
        return {"x": normal((4096, 4096), 2, 0.0, 1.0, BF16),
                "W": normal((11008, 4096), 2, 0.0, 0.02, BF16, offset=nx),
                "bias": normal((11008,), 2, 0.0, 0.02, BF16, offset=nx + nw)}
    if name == "c4a":
        na = 96 * 197 * 64
        return {"A": uniform((96, 197, 64), 3, dtype=F16),
                "B": uniform((96, 64, 197), 3, dtype=F16, offset=na)}
    if name == "c4b":
        o = 2 * 96 * 197 * 64
        na = 96 * 197 * 197
        return {"A": uniform((96, 197, 197), 3, dtype=F16, offset=o),
                "B": uniform((96, 197, 64), 3, dtype=F16, offset=o + na)}
    if name == "c5_ln":
        nx = 16384 * 4096
        g = normal((4096,), 4, 0.0, 0.1, offset=nx)
        return {"x": normal((16384, 4096), 4),
                "gamma": (np.float32(1.0) + g).astype(np.float32),
                "beta": normal((4096,), 4, 0.0, 0.1, offset=nx + 4096)}
    if name == "c5_sce":
        o = 16384 * 4096 + 2 * 4096
        n = 4096 * 32000
        return {"logits": normal((4096, 32000), 4, 0.0, 2.0, offset=o),
                "labels": labels(4096, 32000, 4, offset=2 * (o + n))}
    raise KeyError(name)
