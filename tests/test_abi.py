"""C-ABI checks that need no GPU: the library loads, exports every symbol
include/nova_hip.h declares, and rejects malformed calls with the right
status code before any HIP call (validation runs on the host first)."""
import ctypes
import os
import re

import pytest

import nova_hip as nh
from conftest import REPO

HEADER = os.path.join(REPO, "include", "nova_hip.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:_mlir_ciface_)?nova_hip_\w+)\s*\(", text)))


def test_header_and_binding_agree():
    declared = header_functions()
    assert len(declared) >= 15
    assert sorted(nh.EXPORTS) == declared


def test_library_exports_every_declared_symbol():
    L = nh.lib()
    for name in header_functions():
        assert hasattr(L, name), name
    assert "gfx950" in nh.version()


def test_descriptor_layout_matches_mlir():
    # {ptr, ptr, i64 offset, i64 sizes[R], i64 strides[R]}
    assert ctypes.sizeof(nh.MemRef1D) == 8 * 5
    assert ctypes.sizeof(nh.MemRef2D) == 8 * 7
    assert ctypes.sizeof(nh.MemRef3D) == 8 * 9
    assert nh.MemRef3D.sizes.offset == 24


FAKE = 1 << 40  # never dereferenced: every call below fails validation


def d3(sizes, strides=None, ptr=FAKE):
    if strides is None:
        strides = (sizes[1] * sizes[2], sizes[2], 1)
    return nh.make_memref(ptr, sizes, strides)


def d2(sizes, strides=None, ptr=FAKE):
    if strides is None:
        strides = (sizes[1], 1)
    return nh.make_memref(ptr, sizes, strides)


def d1(n, stride=1, ptr=FAKE):
    return nh.make_memref(ptr, (n,), (stride,))


def gemm_rc(A, B, C, bias=None, flags=None):
    if flags is None:
        flags = nh.gemm_flags(nh.DT_BF16, nh.DT_F32)
    L = nh.lib()
    return L._mlir_ciface_nova_hip_gemm(nh.ref(A), nh.ref(B), nh.ref(C), nh.ref(bias), flags)


def last_error():
    return nh.lib().nova_hip_last_error().decode()


def test_gemm_null_descriptor():
    L = nh.lib()
    assert L._mlir_ciface_nova_hip_gemm(None, None, None, None, 0) == 1
    assert "null" in last_error()


def test_gemm_shape_mismatch():
    assert gemm_rc(d3((2, 8, 16)), d3((2, 15, 8)), d3((2, 8, 8))) == 2
    assert "disagree" in last_error()
    assert gemm_rc(d3((3, 8, 16)), d3((2, 16, 8)), d3((2, 8, 8))) == 2
    assert "broadcast" in last_error()


def test_gemm_bad_flags():
    A, B, C = d3((1, 8, 16)), d3((1, 16, 8)), d3((1, 8, 8))
    assert gemm_rc(A, B, C, flags=1 << 20) == 1
    assert gemm_rc(A, B, C, flags=nh.gemm_flags(7, 0)) == 4
    assert gemm_rc(A, B, C, flags=nh.gemm_flags(nh.DT_F32, nh.DT_BF16)) == 4
    assert gemm_rc(A, B, C, flags=nh.gemm_flags(nh.DT_BF16, nh.DT_F32, 9)) == 4
    # the narrow accumulator: same 16-bit dtype in and out, no GELU, own-dtype bias
    acc = nh.GEMM_ACC_OUT
    assert gemm_rc(A, B, C, flags=nh.gemm_flags(nh.DT_BF16, nh.DT_F32) | acc) == 4
    assert gemm_rc(A, B, C, flags=nh.gemm_flags(nh.DT_BF16, nh.DT_F16) | acc) == 4
    assert gemm_rc(A, B, C, flags=nh.gemm_flags(nh.DT_F32, nh.DT_F32) | acc) == 4
    assert gemm_rc(A, B, C, flags=nh.gemm_flags(nh.DT_F16, nh.DT_F16, nh.EPI_GELU) | acc) == 4
    assert gemm_rc(A, B, C, d1(8),
                   nh.gemm_flags(nh.DT_F16, nh.DT_F16, nh.EPI_BIAS, nh.DT_F32) | acc) == 4
    assert "bias of its own dtype" in last_error()


def test_gemm_accumulate_into_c_flags():
    """NOVA_HIP_GEMM_ACC_C runs on the exact kernel only: not with the f32
    MFMA form, not for 16-bit operands into an f32 accumulator, and with no
    epilogue (the sum starts from C, not from a bias)."""
    A, B, C = d3((1, 8, 16)), d3((1, 16, 8)), d3((1, 8, 8))
    f32 = nh.gemm_flags(nh.DT_F32, nh.DT_F32)
    accc = nh.GEMM_ACC_C
    assert gemm_rc(A, B, C, flags=f32 | accc | nh.GEMM_F32_MFMA) == 1
    assert "f32 MFMA" in last_error()
    assert gemm_rc(A, B, C, flags=nh.gemm_flags(nh.DT_BF16, nh.DT_F32) | accc) == 4
    assert gemm_rc(A, B, C, d1(8),
                   nh.gemm_flags(nh.DT_F32, nh.DT_F32, nh.EPI_BIAS, nh.DT_F32) | accc) == 1
    assert "no epilogue" in last_error()
    assert gemm_rc(A, B, C, flags=nh.gemm_flags(nh.DT_F32, nh.DT_F32, nh.EPI_GELU) | accc) == 1
    # an empty problem stays a no-op
    assert gemm_rc(d3((1, 0, 16)), B, d3((1, 0, 8)), flags=f32 | accc) == 0
    assert gemm_rc(d3((1, 0, 16)), B, d3((1, 0, 8)),
                   flags=nh.gemm_flags(nh.DT_F16, nh.DT_F16) | nh.GEMM_ACC_OUT | accc) == 0


def test_gemm_bias_required_and_checked():
    A, B, C = d3((1, 8, 16)), d3((1, 16, 8)), d3((1, 8, 8))
    f = nh.gemm_flags(nh.DT_BF16, nh.DT_BF16, nh.EPI_BIAS_GELU, nh.DT_BF16)
    assert gemm_rc(A, B, C, None, f) == 1
    assert gemm_rc(A, B, C, d1(7), f) == 2
    assert gemm_rc(A, B, C, d1(8, stride=2), f) == 3


def test_gemm_strides_without_unit_dim():
    A = d3((1, 8, 16), (128, 32, 2))
    assert gemm_rc(A, d3((1, 16, 8)), d3((1, 8, 8))) == 3
    B = d3((1, 16, 8), (128, 16, 2))
    assert gemm_rc(d3((1, 8, 16)), B, d3((1, 8, 8))) == 3
    C = d3((1, 8, 8), (64, 8, 2))
    assert gemm_rc(d3((1, 8, 16)), d3((1, 16, 8)), C) == 3
    C2 = d3((1, 8, 8), (64, 4, 1))  # rows overlap
    assert gemm_rc(d3((1, 8, 16)), d3((1, 16, 8)), C2) == 3


def test_gemm_null_data_pointer():
    assert gemm_rc(d3((1, 8, 16), ptr=0), d3((1, 16, 8)), d3((1, 8, 8))) == 1


def test_gemm_empty_is_a_no_op():
    # M == 0: nothing to compute, no HIP call is made.
    assert gemm_rc(d3((1, 0, 16)), d3((1, 16, 8)), d3((1, 0, 8))) == 0
    assert gemm_rc(d3((0, 8, 16)), d3((0, 16, 8)), d3((0, 8, 8))) == 0


def test_typed_entry_points_validate():
    L = nh.lib()
    A, B, C = d2((8, 16)), d2((15, 8)), d2((8, 8))
    for n in ("matmul_f32", "matmul_bf16_f32", "matmul_f16_f32"):
        assert getattr(L, "_mlir_ciface_nova_hip_" + n)(nh.ref(A), nh.ref(B), nh.ref(C)) == 2
    A3, B3, C3 = d3((2, 8, 16)), d3((2, 15, 8)), d3((2, 8, 8))
    for n in ("batch_matmul_f32", "batch_matmul_bf16_f32", "batch_matmul_f16_f32"):
        assert getattr(L, "_mlir_ciface_nova_hip_" + n)(nh.ref(A3), nh.ref(B3), nh.ref(C3)) == 2
    assert L._mlir_ciface_nova_hip_linear_bf16_bias_gelu(
        nh.ref(d2((8, 16))), nh.ref(d2((16, 8))), nh.ref(d1(9)), nh.ref(d2((8, 8)))) == 2
    assert L._mlir_ciface_nova_hip_linear(
        nh.ref(d2((8, 16))), nh.ref(d2((16, 8))), nh.ref(d1(8)), nh.ref(d2((8, 8))),
        nh.gemm_flags(nh.DT_F32, nh.DT_F16, nh.EPI_BIAS)) == 4


def ln_rc(x, g, b, y, s=None, r=None, eps=1e-5):
    L = nh.lib()
    return L._mlir_ciface_nova_hip_layer_norm_f32(nh.ref(x), nh.ref(g), nh.ref(b), nh.ref(y),
                                                  nh.ref(s), nh.ref(r), ctypes.c_float(eps))


def test_layer_norm_validation():
    x, y = d2((4, 64)), d2((4, 64))
    assert ln_rc(None, d1(64), d1(64), y) == 1
    assert ln_rc(x, d1(63), d1(64), y) == 2
    assert ln_rc(x, d1(64), d1(64), d2((4, 32))) == 2
    assert ln_rc(x, d1(64), d1(64), y, d1(3)) == 2
    assert ln_rc(d2((4, 64), (64, 2)), d1(64), d1(64), y) == 3
    assert ln_rc(d2((4, 64), (32, 1)), d1(64), d1(64), y) == 3
    assert ln_rc(d2((4, 0)), d1(0), d1(0), d2((4, 0))) == 2
    assert ln_rc(d2((0, 64)), d1(64), d1(64), d2((0, 64))) == 0


def sce_rc(x, t, loss, sm=None):
    L = nh.lib()
    return L._mlir_ciface_nova_hip_sce_f32(nh.ref(x), nh.ref(t), nh.ref(loss), nh.ref(sm))


def test_sce_validation():
    x = d2((4, 10))
    assert sce_rc(None, d1(4), d1(1)) == 1
    assert sce_rc(x, d1(3), d1(1)) == 2
    assert sce_rc(x, d1(4), d1(2)) == 2
    assert sce_rc(x, d1(4), d1(1), d2((4, 9))) == 2
    assert sce_rc(d2((4, 10), (10, 2)), d1(4), d1(1)) == 3
    assert sce_rc(d2((4, 0)), d1(4), d1(1)) == 2


def test_sce_noalloc_validation_and_row_limit():
    """The entry point that allocates nothing validates like sce_f32 and
    refuses more rows than its static array holds, before any HIP call."""
    L = nh.lib()
    f = L._mlir_ciface_nova_hip_sce_f32_noalloc
    assert f(nh.ref(d2((4, 10))), nh.ref(d1(3)), nh.ref(d1(1)), None) == 2
    rows = 262144 + 1   # SCE_NOALLOC_MAX_ROWS + 1
    assert f(nh.ref(d2((rows, 10))), nh.ref(d1(rows)), nh.ref(d1(1)), None) == 5
    assert "scratch maximum of 262144" in last_error()


# One past the row limit of the row kernels and the column sum: their
# in-kernel row arithmetic is 32-bit and runs up to a grid's worth of rows
# past the last row.
ROWS_OVER = 0x7fffffff - (1 << 20) + 1


def test_row_limits_are_checked_before_any_launch():
    assert sce_rc(d2((ROWS_OVER, 1)), d1(ROWS_OVER), d1(1)) == 5
    assert "rows exceed 2^31 - 2^20" in last_error()
    L = nh.lib()
    assert L._mlir_ciface_nova_hip_sce_fwd_bwd_f32(
        nh.ref(d2((ROWS_OVER, 1))), nh.ref(d1(ROWS_OVER)), nh.ref(d1(1)),
        nh.ref(d2((ROWS_OVER, 1)))) == 5
    assert ln_rc(d2((ROWS_OVER, 4)), d1(4), d1(4), d2((ROWS_OVER, 4))) == 5
    assert "rows exceed 2^31 - 2^20" in last_error()


def test_error_text_is_per_call():
    assert gemm_rc(d3((2, 8, 16)), d3((2, 15, 8)), d3((2, 8, 8))) == 2
    assert last_error()
    assert gemm_rc(d3((1, 0, 16)), d3((1, 16, 8)), d3((1, 0, 8))) == 0
    assert last_error() == ""


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(nh, "LIB_PATH", str(tmp_path / "absent.so"))
    monkeypatch.setattr(nh, "_lib", None)
    with pytest.raises(ImportError, match="no fallback"):
        nh.lib()


# ---- backward entry points: host validation only (no call reaches HIP) ----

def test_sce_backward_validation():
    L = nh.lib()
    f = lambda sm, t, g: L._mlir_ciface_nova_hip_sce_backward_f32(nh.ref(sm), nh.ref(t), nh.ref(g))
    assert f(None, d1(4), d2((4, 10))) == 1
    assert f(d2((4, 10)), d1(3), d2((4, 10))) == 2
    assert f(d2((4, 10)), d1(4), d2((4, 9))) == 2
    assert f(d2((4, 10), (10, 2)), d1(4), d2((4, 10))) == 3
    assert f(d2((4, 10), (5, 1)), d1(4), d2((4, 10))) == 3
    assert f(d2((0, 10)), d1(0), d2((0, 10))) == 0


def test_sce_fwd_bwd_validation():
    L = nh.lib()
    f = lambda x, t, loss, g: L._mlir_ciface_nova_hip_sce_fwd_bwd_f32(
        nh.ref(x), nh.ref(t), nh.ref(loss), nh.ref(g))
    assert f(d2((4, 10)), d1(4), d1(1), None) == 1
    assert f(d2((4, 10)), d1(4), d1(1), d2((4, 11))) == 2
    assert f(d2((4, 10)), d1(4), d1(1), d2((4, 10), (10, 2))) == 3
    assert f(d2((4, 10)), d1(4), d1(2), d2((4, 10))) == 2


def ln_bwd_rc(gy, x, g, S, r, dx=None, dg=None, db=None):
    L = nh.lib()
    return L._mlir_ciface_nova_hip_layer_norm_backward_f32(
        nh.ref(gy), nh.ref(x), nh.ref(g), nh.ref(S), nh.ref(r), nh.ref(dx), nh.ref(dg), nh.ref(db))


def test_layer_norm_backward_validation():
    x = d2((4, 64))
    assert ln_bwd_rc(None, x, d1(64), d1(4), d1(4)) == 1
    assert ln_bwd_rc(d2((4, 63)), x, d1(64), d1(4), d1(4)) == 2
    assert ln_bwd_rc(x, x, d1(63), d1(4), d1(4)) == 2
    assert ln_bwd_rc(x, x, d1(64), d1(3), d1(4)) == 2
    assert ln_bwd_rc(x, x, d1(64), d1(4), d1(4), d2((4, 32))) == 2
    assert ln_bwd_rc(x, x, d1(64), d1(4), d1(4), None, d1(32)) == 2
    assert ln_bwd_rc(x, d2((4, 64), (64, 2)), d1(64), d1(4), d1(4)) == 3
    assert ln_bwd_rc(x, x, d1(64), d1(4, 2), d1(4)) == 3
    assert ln_bwd_rc(d2((4, 0)), d2((4, 0)), d1(0), d1(4), d1(4)) == 2
    # rows longer than the LDS column accumulators hold: refused before any launch
    big = d2((4, 8193))
    assert ln_bwd_rc(big, big, d1(8193), d1(4), d1(4)) == 5


def test_linear_backward_validation():
    L = nh.lib()
    fl = nh.gemm_flags(nh.DT_BF16, nh.DT_F32)

    def f(go, x, w, gi=None, gw=None, gb=None, flags=fl):
        return L._mlir_ciface_nova_hip_linear_backward(nh.ref(go), nh.ref(x), nh.ref(w), nh.ref(gi),
                                                       nh.ref(gw), nh.ref(gb), flags)

    go, x, w = d2((8, 16)), d2((8, 32)), d2((32, 16))
    assert f(None, x, w) == 1
    assert f(go, x, w, flags=nh.gemm_flags(nh.DT_BF16, nh.DT_F32, nh.EPI_BIAS)) == 1
    assert f(go, x, w, flags=0x10000) == 1
    assert f(go, x, w, flags=fl | 0x40000) == 1          # no accumulate-into form
    assert f(go, x, d2((31, 16))) == 2
    assert f(d2((8, 15)), x, w) == 2
    assert f(go, x, w, gi=d2((8, 31))) == 2          # grad_input must be [M, K]
    assert f(go, x, w, gw=d2((32, 15))) == 2         # grad_weight must be [K, N]
    assert f(go, x, w, gb=d1(15)) == 2
    assert f(go, x, w, gb=d1(16, 2)) == 3
    assert f(d2((8, 16), (1, 8)), x, w, gb=d1(16)) == 3  # column sums need unit stride on N
    # empty batch: both GEMMs are no-ops, and no bias gradient asked for
    assert f(d2((0, 16)), d2((0, 32)), w, gi=d2((0, 32))) == 0
    # Every output is validated before the first launch: with both GEMM
    # outputs given, a malformed grad_weight or grad_bias still fails
    # validation (a launch, with no GPU here, would give a HIP error).
    gi, gw = d2((8, 32)), d2((32, 16))
    assert f(go, x, w, gi=gi, gw=gw, gb=d1(15)) == 2
    assert f(go, x, w, gi=gi, gw=d2((32, 15))) == 2
    assert f(go, x, w, gi=gi, gw=gw, gb=d1(16, ptr=0)) == 1
    assert f(d2((ROWS_OVER, 16)), d2((ROWS_OVER, 32)), w, gi=d2((ROWS_OVER, 32)),
             gb=d1(16)) == 5
    assert "column sum" in last_error()


def test_matmul_backward_validation():
    L = nh.lib()
    fl = nh.gemm_flags(nh.DT_F32, nh.DT_F32)

    def f(g, A, B, ga=None, gb=None, flags=fl):
        return L._mlir_ciface_nova_hip_matmul_backward(nh.ref(g), nh.ref(A), nh.ref(B), nh.ref(ga),
                                                       nh.ref(gb), flags)

    g, A, B = d2((8, 16)), d2((8, 32)), d2((32, 16))
    assert f(None, A, B) == 1
    assert f(g, A, d2((30, 16))) == 2
    assert f(d2((9, 16)), A, B) == 2
    assert f(g, A, B, flags=nh.gemm_flags(nh.DT_F32, nh.DT_BF16)) == 4
    assert f(g, A, B, flags=nh.gemm_flags(nh.DT_F32, nh.DT_F32, nh.EPI_GELU)) == 1
    assert f(g, A, B, ga=d2((8, 31))) == 2
    # both outputs validated before either GEMM is launched
    assert f(g, A, B, ga=d2((8, 32)), gb=d2((32, 15))) == 2


def d4(sizes, strides=None, ptr=FAKE):
    if strides is None:
        strides = (sizes[1] * sizes[2] * sizes[3], sizes[2] * sizes[3], sizes[3], 1)
    return nh.make_memref(ptr, sizes, strides)


def test_glue_entry_points_validate_before_any_hip_call():
    L = nh.lib()
    r = nh.ref
    # binary: shapes that do not broadcast, unknown op, null data, empty no-op
    assert L._mlir_ciface_nova_hip_binary_f32(r(d4((1, 2, 3, 4))), r(d4((1, 2, 5, 4))),
                                              r(d4((1, 2, 3, 4))), nh.BIN_ADD) == 2
    assert "broadcast" in last_error()
    assert L._mlir_ciface_nova_hip_binary_f32(r(d4((1, 2, 3, 4))), r(d4((1, 1, 1, 4))),
                                              r(d4((1, 2, 3, 4))), 9) == 1
    assert L._mlir_ciface_nova_hip_binary_f32(r(d4((1, 2, 3, 4), ptr=0)), r(d4((1, 1, 1, 4))),
                                              r(d4((1, 2, 3, 4))), nh.BIN_MUL) == 1
    assert L._mlir_ciface_nova_hip_binary_f32(r(d4((1, 0, 3, 4))), r(d4((1, 1, 3, 4))),
                                              r(d4((1, 0, 3, 4))), nh.BIN_MUL) == 0
    # fill / gelu / gelu_backward / index_to_i32
    assert L._mlir_ciface_nova_hip_fill_f32(r(d1(-1)), 1.0) == 2
    assert L._mlir_ciface_nova_hip_gelu_f32(r(d1(8)), r(d1(9))) == 2
    assert L._mlir_ciface_nova_hip_gelu_backward_f32(r(d1(8)), r(d1(8, stride=2)), r(d1(8))) == 3
    assert L._mlir_ciface_nova_hip_index_to_i32(r(d1(8)), r(d1(8)), 7) == 4
    # gather / scatter_add: index dtype, shapes, row strides
    assert L._mlir_ciface_nova_hip_gather_f32(r(d2((10, 4))), r(d1(3)), r(d2((3, 4))), 2) == 4
    assert L._mlir_ciface_nova_hip_gather_f32(r(d2((10, 4))), r(d1(3)), r(d2((3, 5))),
                                              nh.DT_I64) == 2
    assert L._mlir_ciface_nova_hip_gather_f32(r(d2((10, 4), (8, 2))), r(d1(3)),
                                              r(d2((3, 4))), nh.DT_I16) == 3
    assert L._mlir_ciface_nova_hip_scatter_add_f32(r(d2((10, 4))), r(d1(3)), r(d2((2, 4))),
                                                   nh.DT_I32) == 2
    # reduce_sum: out must be [outer, inner]
    assert L._mlir_ciface_nova_hip_reduce_sum_f32(r(d3((2, 5, 7))), r(d2((2, 5)))) == 2
    assert L._mlir_ciface_nova_hip_reduce_sum_f32(r(d3((0, 5, 7))), r(d2((0, 7)))) == 0
