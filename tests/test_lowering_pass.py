"""The MLIR lowering pass (nova-compiler_amd/mlir/NovaHipLowering.cpp) cannot
be compiled in this image (no MLIR).  These checks tie it to what is built
and tested: every callee it can emit is an export of libnova_hip, it lowers
the same Nova ops the planner plans, and the typed aliases it calls check
their flags before any HIP call."""
import ctypes
import itertools
import os
import re

import nova_hip as nh
from conftest import PKG

SRC = os.path.join(PKG, "mlir", "NovaHipLowering.cpp")
DTS = ("f32", "bf16", "f16")


def _source():
    with open(SRC) as f:
        return f.read()


def test_every_emitted_callee_is_exported():
    text = _source()
    fixed = set(re.findall(r'"(nova_hip_[a-z0-9_]+?)"', text))
    prefixes = {n for n in fixed if n.endswith("_")}
    names = fixed - prefixes
    # GEMMs: nova_hip_gemm_<in>_<out>_b<bias>; backward: <prefix><in>_<out>
    names |= {f"nova_hip_gemm_{i}_{o}_b{b}" for i, o, b in itertools.product(DTS, DTS, DTS)}
    for p in ("nova_hip_linear_backward_", "nova_hip_matmul_backward_"):
        assert p in prefixes
        names |= {f"{p}f32_f32"} | {f"{p}{i}_{o}" for i in ("bf16", "f16") for o in DTS}
    assert "nova_hip_gemm_" in prefixes
    L = nh.lib()
    for n in sorted(names):
        assert hasattr(L, "_mlir_ciface_" + n), n
    assert len(names) >= 44


def test_lowers_the_planners_ops():
    text = _source()
    lowered = set(re.findall(r"\b(LinearOp|MatmulOp|LayerNormOp|SceOp|SceBackwardOp|"
                             r"LayerNormBackwardOp|LinearBackwardOp|MatmulBackwardOp)\b", text))
    assert lowered == {"LinearOp", "MatmulOp", "LayerNormOp", "SceOp", "SceBackwardOp",
                       "LayerNormBackwardOp", "LinearBackwardOp", "MatmulBackwardOp"}
    for fold in ("GeluOp", "CastOp", "TransposeOp"):
        assert fold in text
    assert "NOVA_HIP_GEMM_ACC_OUT" in text and "NOVA_HIP_GEMM_F32_MFMA" in text


def test_aliases_check_their_dtypes():
    L = nh.lib()
    A = nh.make_memref(0x1000, (1, 8, 16), (128, 16, 1))
    B = nh.make_memref(0x1000, (1, 16, 8), (128, 8, 1))
    C = nh.make_memref(0x1000, (1, 8, 8), (64, 8, 1))
    bias = nh.make_memref(0x1000, (8,), (1,))
    f = L._mlir_ciface_nova_hip_gemm_bf16_f32_bbf16
    ref = nh.ref
    # f16 operands through the bf16 alias
    assert f(ref(A), ref(B), ref(C), ref(bias), nh.gemm_flags(nh.DT_F16, nh.DT_F32)) == 1
    # bias dtype checked only with a bias epilogue
    assert f(ref(A), ref(B), ref(C), ref(bias),
             nh.gemm_flags(nh.DT_BF16, nh.DT_F32, nh.EPI_BIAS, nh.DT_F32)) == 1
    assert "name other dtypes" in L.nova_hip_last_error().decode()
    g = L._mlir_ciface_nova_hip_linear_backward_bf16_f32
    go = nh.make_memref(0x1000, (8, 8), (8, 1))
    assert g(ref(go), ref(go), ref(go), None, None, None, nh.gemm_flags(nh.DT_F16, nh.DT_F32)) == 1
