"""Nova programs in the op surface, run end to end through libnova_run
(parse -> plan -> device buffers -> libnova_hip launches -> results) on
the GPU, against the CPU oracle on the same seeded inputs.  Bars as in the
other GPU tests: f32 GEMMs bit-exact, bf16 in / f32 accumulate rtol 2e-2
atol 1e-2, reductions f32 rtol 1e-4 with atol 1e-4 * max|c|."""
import os
import subprocess

import numpy as np
import pytest

import nova_cpu_ref as ref
import nova_run
import nova_seed as S
from conftest import GOLDEN, PKG, assert_close_f32, assert_close_lp

pytestmark = pytest.mark.gpu
MLIR = os.path.join(GOLDEN, "mlir")


def prog(name):
    with open(os.path.join(MLIR, name)) as f:
        return nova_run.Program(f.read())


def test_linear_gelu_bf16_program(cuda):
    x = S.normal((96, 160), 71, dtype=S.BF16)
    W = S.normal((200, 160), 71, 0, 0.02, dtype=S.BF16, offset=x.size)
    b = S.normal((200,), 71, 0, 0.02, dtype=S.BF16, offset=x.size + W.size)
    (y,) = prog("linear_gelu_bf16.mlir").run("linear_gelu", x, W, b)
    want = ref.gemm(x, W.T, adt=S.BF16, bdt=S.BF16, bias=b, biasdt=S.BF16,
                    epilogue=ref.EPI_BIAS_GELU, cdt=S.BF16)[0]
    assert_close_lp(S.widen(y, S.BF16), S.widen(want, S.BF16), "linear+gelu program")


@pytest.mark.parametrize("func", ["bmm", "bmm_nova"])
def test_batch_matmul_programs(cuda, func):
    A = S.uniform((4, 128, 96), 72, dtype=S.BF16)
    B = S.uniform((4, 96, 160), 72, dtype=S.BF16, offset=A.size)
    (C,) = prog("batch_matmul_bf16.mlir").run(func, A, B)
    assert_close_lp(C, ref.gemm(A, B, adt=S.BF16, bdt=S.BF16), func)


def test_f32_programs_bit_exact(cuda):
    p = prog("matmul_f32.mlir")
    A = S.uniform((256, 256), 0)
    B = S.uniform((256, 256), 0, offset=A.size)
    (C,) = p.run("mm", A, B)
    assert np.array_equal(C, ref.gemm(A, B)[0])
    x = S.uniform((33, 70), 73)
    w = S.uniform((70, 45), 73, offset=x.size)
    b = S.uniform((45,), 73, offset=x.size + w.size)
    (y,) = p.run("lin", x, w, b)
    assert np.array_equal(y, ref.gemm(x, w, bias=b, epilogue=ref.EPI_BIAS)[0])


def test_layer_norm_programs(cuda):
    p = prog("reductions.mlir")
    x = S.normal((64, 1024), 74)
    g = (1 + S.normal((1024,), 74, 0, 0.1, offset=x.size)).astype(np.float32)
    b = S.normal((1024,), 74, 0, 0.1, offset=x.size + 1024)
    gy = S.normal((64, 1024), 74, offset=x.size + 2048)
    y, s, r = p.run("ln", x, g, b)
    y_ref, s_ref, r_ref = ref.layer_norm(x, g, b)
    assert_close_f32(y, y_ref, "ln y")
    assert_close_f32(s, s_ref, "ln mean_sum")
    assert_close_f32(r, r_ref, "ln rstd")
    y2, dx, dg, db = p.run("ln_train", x, g, b, gy)
    dx_ref, dg_ref, db_ref = ref.layer_norm_backward(gy, x, g, s_ref, r_ref)
    assert_close_f32(y2, y_ref, "ln_train y")
    assert_close_f32(dx, dx_ref, "ln_train dx")
    assert_close_f32(dg, dg_ref, "ln_train dgamma")
    assert_close_f32(db, db_ref, "ln_train dbeta")


def test_sce_train_program(cuda):
    x = S.normal((32, 5000), 75, 0, 2)
    t = S.labels(32, 5000, 75, offset=x.size)
    loss, grad = prog("reductions.mlir").run("sce_train", x, t)
    sm, loss_ref, _ = ref.sce(x, t, softmax=True)
    assert_close_f32(loss, loss_ref, "sce loss")
    assert_close_f32(grad, ref.sce_backward(sm, t), "sce grad")


def test_backward_programs(cuda):
    p = prog("backward.mlir")
    go = S.uniform((40, 24), 76)
    x = S.uniform((40, 36), 76, offset=go.size)
    w = S.uniform((36, 24), 76, offset=go.size + x.size)
    gi, gw, gb = p.run("lin_bwd", go, x, w)
    gi_ref, gw_ref, gb_ref = ref.linear_backward(go, x, w)
    assert np.array_equal(gi, gi_ref) and np.array_equal(gw, gw_ref)
    assert_close_f32(gb, gb_ref, "grad_bias")
    g = S.uniform((64, 96), 77, dtype=S.BF16)
    a = S.uniform((64, 128), 77, dtype=S.BF16, offset=g.size)
    bb = S.uniform((128, 96), 77, dtype=S.BF16, offset=g.size + a.size)
    ga, gbb = p.run("mm_bwd", g, a, bb)
    ga_ref, gb_ref2 = ref.matmul_backward(g, a, bb, dt=S.BF16)
    assert_close_lp(S.widen(ga, S.BF16), ga_ref, "bf16 grad_a")
    assert_close_lp(S.widen(gbb, S.BF16), gb_ref2, "bf16 grad_b")


def test_memref_entry_fills_output_argument(cuda):
    x = S.uniform((64, 96), 78)
    w = S.uniform((96, 80), 78, offset=x.size)
    b = S.uniform((80,), 78, offset=x.size + w.size)
    out = np.zeros((64, 80), np.float32)
    assert prog("memref_main.mlir").run("main", x, w, b, out) == []
    assert np.array_equal(out, ref.gemm(x, w, bias=b, epilogue=ref.EPI_BIAS)[0])


def test_nova_run_cli(cuda):
    exe = os.path.join(PKG, "nova-run")
    r = subprocess.run([exe, os.path.join(MLIR, "batch_matmul_bf16.mlir"), "--func", "bmm",
                        "--reps", "2"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "_mlir_ciface_nova_hip_gemm" in r.stdout and "ms per run" in r.stdout
