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


def test_rank4_matmul_programs_bit_exact(cuda):
    """nova.matmul above rank 3, and with a rank-2 operand broadcast over
    two batch dims: f32 bit-exact against the oracle on the collapsed batch."""
    p = prog("matmul_rank4.mlir")
    A = S.uniform((2, 3, 8, 16), 79)
    B = S.uniform((2, 3, 16, 5), 79, offset=A.size)
    (C,) = p.run("mm4", A, B)
    want = ref.gemm(A.reshape(6, 8, 16), B.reshape(6, 16, 5)).reshape(2, 3, 8, 5)
    assert np.array_equal(C, want)
    W = S.uniform((16, 5), 80)
    (C2,) = p.run("mm4_bcast", A, W)
    want2 = ref.gemm(A.reshape(6, 8, 16), np.broadcast_to(W, (6, 16, 5)).copy()).reshape(2, 3, 8, 5)
    assert np.array_equal(C2, want2)


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
    assert ga.dtype == np.float32 and gbb.dtype == np.float32
    assert_close_lp(ga, ga_ref, "bf16 grad_a")
    assert_close_lp(gbb, gb_ref2, "bf16 grad_b")


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


def gpt_step_oracle(tok, tgt, pos, wte, wpe, g1, be1, w1, c1, w2, c2, g2, be2, wlm):
    """The GPT step composed from the oracle's ops, in the program's order."""
    B, T = tok.shape
    V, D = wte.shape
    N = B * T
    h = ref.binary(ref.gather(wte, tok), ref.gather(wpe, pos), ref.ADD).reshape(N, D)
    y1, S1, r1 = ref.layer_norm(h, g1, be1)
    up = ref.gemm(y1, w1, bias=c1, epilogue=ref.EPI_BIAS)[0]
    act = ref.gelu(up)
    dn = ref.gemm(act, w2, bias=c2, epilogue=ref.EPI_BIAS)[0]
    r = ref.binary(h, dn, ref.ADD)
    y2, S2, r2 = ref.layer_norm(r, g2, be2)
    logits = ref.gemm(y2, wlm)[0]
    t32 = ref.index_to_i32(tgt).reshape(-1)
    sm, loss, _ = ref.sce(logits, t32, softmax=True)
    dl = ref.binary(ref.sce_backward(sm, t32), np.ones(1, np.float32), ref.MUL)
    dflat = ref.gemm(dl, np.ascontiguousarray(wlm.T))[0]
    dwlm = ref.gemm(np.ascontiguousarray(y2.T), dl)[0]
    gr = ref.layer_norm_backward(dflat, r, g2, S2, r2)
    gd = ref.linear_backward(gr[0], act, w2)
    dup = ref.gelu_backward(gd[0], up)
    gu = ref.linear_backward(dup, y1, w1)
    gh = ref.layer_norm_backward(gu[0], h, g1, S1, r1)
    dh = ref.binary(gr[0], gh[0], ref.ADD)
    dwpe = ref.scatter_add(np.zeros((T, D), np.float32), pos.reshape(-1),
                           ref.reduce_sum(dh.reshape(B, T, D), 0))
    dwte = ref.scatter_add(np.zeros((V, D), np.float32), tok.reshape(-1), dh)
    return [loss, dwte, dwpe, gh[1], gh[2], gu[1], gu[2], gd[1], gd[2], gr[1], gr[2], dwlm]


@pytest.mark.parametrize("B,T,V,D,H", [(2, 16, 96, 64, 128), (1, 64, 50304, 64, 128)])
def test_gpt_step_program_end_to_end(cuda, B, T, V, D, H):
    """A whole GPT training step (embeddings, LayerNorm, MLP with GELU,
    residual, LM head, SCE loss and the full backward to the embedding
    gradients) through libnova_run, against the oracle's ops composed in the
    same order.  The second size has the reference's vocab (50304): its SCE
    rows take the streaming path for more than 32768 classes, and the LM
    head's weight gradient is a K = 64 product over 50304 columns."""
    from gpt_program import gpt_step
    r = np.random.default_rng(79)
    f = lambda *s, k=0.1: (r.standard_normal(s) * k).astype(np.float32)  # noqa: E731
    tok = r.integers(0, V, (B, T)).astype(np.int16)
    tgt = r.integers(0, V, (B, T)).astype(np.int16)
    pos = np.arange(T, dtype=np.int64).reshape(1, T)
    args = [tok, tgt, pos, f(V, D, k=0.5), f(T, D, k=0.5), 1 + f(D), f(D), f(D, H), f(H),
            f(H, D), f(D), 1 + f(D), f(D), f(D, V)]
    got = nova_run.Program(gpt_step(B, T, V, D, H)).run("gpt_step", *args)
    want = gpt_step_oracle(*args)
    names = ["loss", "dwte", "dwpe", "dgamma1", "dbeta1", "dw1", "db1", "dw2", "db2",
             "dgamma2", "dbeta2", "dwlm"]
    assert len(got) == len(want)
    for g, w, n in zip(got, want, names):
        assert g.shape == w.shape, n
        assert_close_f32(g, w, "gpt_step " + n)
    # rows of the embedding no token hits get no gradient (i16 tokens are
    # zero-extended, so ids above 32767 are stored as negative int16)
    unused = np.setdiff1d(np.arange(V), tok.reshape(-1).view(np.uint16))
    assert (got[1][unused] == 0).all()


@pytest.mark.parametrize("B,T,V,D,H", [(2, 16, 96, 64, 128), (1, 64, 50304, 64, 128)])
def test_gpt_step_device_resident_f32_mfma(cuda, B, T, V, D, H):
    """The same step through nova_run_execute_device (device-resident
    arguments and results, no host copies) with the f32 GEMMs on the matrix
    cores: every result within the f32 bar of the oracle; a second execution
    into the same result tensors gives the same bits; the exact mode gives
    what the host-array path gives."""
    import torch
    from gpt_program import gpt_step
    r = np.random.default_rng(80)
    f = lambda *s, k=0.1: (r.standard_normal(s) * k).astype(np.float32)  # noqa: E731
    tok = r.integers(0, V, (B, T)).astype(np.int16)
    tgt = r.integers(0, V, (B, T)).astype(np.int16)
    pos = np.arange(T, dtype=np.int64).reshape(1, T)
    args = [tok, tgt, pos, f(V, D, k=0.5), f(T, D, k=0.5), 1 + f(D), f(D), f(D, H), f(H),
            f(H, D), f(D), 1 + f(D), f(D), f(D, V)]
    p = nova_run.Program(gpt_step(B, T, V, D, H))
    dev = [torch.from_numpy(a).to(cuda) for a in args]
    want = gpt_step_oracle(*args)
    names = ["loss", "dwte", "dwpe", "dgamma1", "dbeta1", "dw1", "db1", "dw2", "db2",
             "dgamma2", "dbeta2", "dwlm"]
    p.set_f32_gemm(nova_run.F32_GEMM_MFMA)
    out = p.run_device("gpt_step", *dev)
    torch.cuda.synchronize()
    first = [o.clone() for o in out]
    for g, w, n in zip(out, want, names):
        assert_close_f32(g.cpu().numpy(), w, "device mfma " + n)
    p.run_device("gpt_step", *dev, results=out)
    torch.cuda.synchronize()
    for a, b in zip(first, out):
        assert torch.equal(a, b)
    p.set_f32_gemm(nova_run.F32_GEMM_EXACT)
    out = p.run_device("gpt_step", *dev)
    host = p.run("gpt_step", *args)
    torch.cuda.synchronize()
    for g, h, n in zip(out, host, names):
        if n not in ("dwte", "dwpe"):   # scatter_add's atomics add in no fixed order
            assert np.array_equal(g.cpu().numpy(), h), n


def test_device_execute_writable_argument_and_returned_argument(cuda):
    """A writable memref argument is written in place; an argument returned
    as a result is copied into the result memory."""
    import torch
    p = prog("memref_main.mlir")
    x = S.uniform((64, 96), 84)
    w = S.uniform((96, 80), 84, offset=x.size)
    b = S.uniform((80,), 84, offset=x.size + w.size)
    dx, dw, db = (torch.from_numpy(a).to(cuda) for a in (x, w, b))
    dout = torch.zeros((64, 80), device=cuda)
    assert p.run_device("main", dx, dw, db, dout) == []
    torch.cuda.synchronize()
    assert np.array_equal(dout.cpu().numpy(), ref.gemm(x, w, bias=b, epilogue=ref.EPI_BIAS)[0])
    q = nova_run.Program("""func.func @id(%x: tensor<8x8xf32>) -> (tensor<8x8xf32>, tensor<8x8xf32>) {
      %y = nova.gelu %x : tensor<8x8xf32>
      return %x, %y : tensor<8x8xf32>, tensor<8x8xf32>
    }""")
    xs = S.normal((8, 8), 85)
    rx, ry = q.run_device("id", torch.from_numpy(xs).to(cuda))
    torch.cuda.synchronize()
    assert np.array_equal(rx.cpu().numpy(), xs)
    assert_close_f32(ry.cpu().numpy(), ref.gelu(xs), "gelu")


def test_nova_run_cli_gpt_step_with_i16_arguments(cuda, tmp_path):
    """The CLI fills i16 token / label and i64 position arguments with
    in-range indices and runs a whole GPT step."""
    from gpt_program import gpt_step
    f = tmp_path / "gpt.mlir"
    f.write_text(gpt_step(2, 8, 64, 32, 64))
    exe = os.path.join(PKG, "nova-run")
    r = subprocess.run([exe, str(f), "--reps", "2"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "ms per run" in r.stdout and "nan" not in r.stdout.lower()


def test_cse_fill_and_argument_fill_programs(cuda):
    """Two products over one zero fill, and a fill into an argument that a
    later product reads: every result matches the oracle (f32 bit-exact)."""
    p = nova_run.Program("""func.func @two(%a: tensor<40x24xf32>, %b: tensor<24x16xf32>, %c: tensor<24x16xf32>) -> (tensor<40x16xf32>, tensor<40x16xf32>) {
      %z = arith.constant 0.000000e+00 : f32
      %e = tensor.empty() : tensor<40x16xf32>
      %f = linalg.fill ins(%z : f32) outs(%e : tensor<40x16xf32>) -> tensor<40x16xf32>
      %r1 = linalg.matmul ins(%a, %b : tensor<40x24xf32>, tensor<24x16xf32>) outs(%f : tensor<40x16xf32>) -> tensor<40x16xf32>
      %r2 = linalg.matmul ins(%a, %c : tensor<40x24xf32>, tensor<24x16xf32>) outs(%f : tensor<40x16xf32>) -> tensor<40x16xf32>
      return %r1, %r2 : tensor<40x16xf32>, tensor<40x16xf32>
    }
    func.func @argfill(%a: tensor<32x32xf32>, %x: tensor<32x32xf32>) -> (tensor<32x32xf32>, tensor<32x32xf32>) {
      %z = arith.constant 0.000000e+00 : f32
      %f = linalg.fill ins(%z : f32) outs(%x : tensor<32x32xf32>) -> tensor<32x32xf32>
      %r1 = linalg.matmul ins(%a, %a : tensor<32x32xf32>, tensor<32x32xf32>) outs(%f : tensor<32x32xf32>) -> tensor<32x32xf32>
      %r2 = nova.matmul %x, %a : tensor<32x32xf32>, tensor<32x32xf32>
      return %r1, %r2 : tensor<32x32xf32>, tensor<32x32xf32>
    }""")
    a = S.uniform((40, 24), 81)
    b = S.uniform((24, 16), 81, offset=a.size)
    c = S.uniform((24, 16), 81, offset=a.size + b.size)
    r1, r2 = p.run("two", a, b, c)
    assert np.array_equal(r1, ref.gemm(a, b)[0])
    assert np.array_equal(r2, ref.gemm(a, c)[0])
    a = S.uniform((32, 32), 82)
    x = S.uniform((32, 32), 82, offset=a.size)
    r1, r2 = p.run("argfill", a, x)
    assert np.array_equal(r1, ref.gemm(a, a)[0])
    assert np.array_equal(r2, ref.gemm(x, a)[0])


def test_f16_nova_matmul_accumulates_in_f16(cuda):
    """f16 x f16 nova.matmul gives f16 (NovaOps.cpp:1198) from an f16
    linalg.matmul: the accumulator is f16 (oracle bits)."""
    p = nova_run.Program("""func.func @h(%a: tensor<3x50x300xf16>, %b: tensor<3x300x40xf16>) -> tensor<3x50x40xf16> {
      %r = nova.matmul %a, %b : tensor<3x50x300xf16>, tensor<3x300x40xf16>
      return %r : tensor<3x50x40xf16>
    }""")
    A = S.uniform((3, 50, 300), 83, dtype=S.F16)
    B = S.uniform((3, 300, 40), 83, dtype=S.F16, offset=A.size)
    (C,) = p.run("h", A, B)
    assert np.array_equal(np.asarray(C).view(np.uint16), ref.gemm_acc_out(A, B, dt=S.F16))


CHAIN = """func.func @chain(%x: tensor<1024x1024xf32>, %w1: tensor<1024x1024xf32>, %w2: tensor<1024x1024xf32>) -> tensor<1024x1024xf32> {
  %t = nova.matmul %x, %w1 : tensor<1024x1024xf32>, tensor<1024x1024xf32>
  %r = nova.matmul %t, %w2 : tensor<1024x1024xf32>, tensor<1024x1024xf32>
  return %r : tensor<1024x1024xf32>
}"""


def test_device_executions_on_two_streams_are_ordered(cuda):
    """Device executions of one program share its held intermediates (%t):
    an execution queued on a second stream right after one on the first waits
    for it on the device, so both give the single-stream bits."""
    import torch
    p = nova_run.Program(CHAIN)
    ins = [torch.from_numpy(S.uniform((1024, 1024), 90 + i)).to(cuda) for i in range(4)]
    want1 = p.run_device("chain", ins[0], ins[2], ins[3])[0].clone()
    want2 = p.run_device("chain", ins[1], ins[2], ins[3])[0].clone()
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for _ in range(3):
        with torch.cuda.stream(s1):
            o1 = p.run_device("chain", ins[0], ins[2], ins[3])[0]
        with torch.cuda.stream(s2):
            o2 = p.run_device("chain", ins[1], ins[2], ins[3])[0]
        torch.cuda.synchronize()
        assert torch.equal(o1, want1) and torch.equal(o2, want2)


def test_device_execute_checks_given_results(cuda):
    """Caller-supplied result tensors must be exactly the planned results
    (shape, dtype, contiguity, device): the kernels write their full size."""
    import torch
    p = nova_run.Program(CHAIN)
    x = torch.zeros(1024, 1024, device=cuda)
    for bad in (torch.empty(1024, 1023, device=cuda), torch.empty(1024, 1024, device=cuda,
                dtype=torch.float16), torch.empty(1024, 2048, device=cuda)[:, ::2],
                torch.empty(1024, 1024)):
        with pytest.raises(ValueError, match="result needs"):
            p.run_device("chain", x, x, x, results=[bad])
    with pytest.raises(ValueError, match="has 1 results"):
        p.run_device("chain", x, x, x, results=[])


# The shapes of the reference's own GEMM pipeline tests, as programs in this
# path's op surface, against the oracle (f32: the exact kernel, so bit for
# bit).  test/pipeline-tests/01_matmul_non_aligned.mlir (100x300 . 300x200),
# 03_batch_matmul.mlir (4x64x256 . 4x256x64; 1x128x256 . 1x256x128 in its
# second function), 04_matmul_bias_fusion.mlir (the 100x200 matmul plus a
# [100, 200] bias added elementwise) and 13_matmul_bias_relu.mlir (128x256 .
# 256x512 with a [512] bias, which FuseMatmulBias folds into the accumulator:
# FuseMatmulBias.cpp:184-188).  Those files accumulate into a function
# argument (outs = %C) or go on into linalg.generic / relu, forms outside
# this path; the products and biases are the same.
REF_SHAPES = """func.func @p01(%A: tensor<100x300xf32>, %B: tensor<300x200xf32>) -> tensor<100x200xf32> {
  %r = nova.matmul %A, %B : tensor<100x300xf32>, tensor<300x200xf32>
  return %r : tensor<100x200xf32>
}
func.func @p03(%A: tensor<4x64x256xf32>, %B: tensor<4x256x64xf32>) -> tensor<4x64x64xf32> {
  %z = arith.constant 0.000000e+00 : f32
  %e = tensor.empty() : tensor<4x64x64xf32>
  %c = linalg.fill ins(%z : f32) outs(%e : tensor<4x64x64xf32>) -> tensor<4x64x64xf32>
  %r = linalg.batch_matmul ins(%A, %B : tensor<4x64x256xf32>, tensor<4x256x64xf32>) outs(%c : tensor<4x64x64xf32>) -> tensor<4x64x64xf32>
  return %r : tensor<4x64x64xf32>
}
func.func @p03b(%A: tensor<1x128x256xf32>, %B: tensor<1x256x128xf32>) -> tensor<1x128x128xf32> {
  %r = nova.matmul %A, %B : tensor<1x128x256xf32>, tensor<1x256x128xf32>
  return %r : tensor<1x128x128xf32>
}
func.func @p04(%A: tensor<100x300xf32>, %B: tensor<300x200xf32>, %bias: tensor<100x200xf32>) -> tensor<100x200xf32> {
  %z = arith.constant 0.000000e+00 : f32
  %e = tensor.empty() : tensor<100x200xf32>
  %c = linalg.fill ins(%z : f32) outs(%e : tensor<100x200xf32>) -> tensor<100x200xf32>
  %m = linalg.matmul ins(%A, %B : tensor<100x300xf32>, tensor<300x200xf32>) outs(%c : tensor<100x200xf32>) -> tensor<100x200xf32>
  %r = nova.add %m, %bias : tensor<100x200xf32>, tensor<100x200xf32>
  return %r : tensor<100x200xf32>
}
func.func @p13(%x: tensor<128x256xf32>, %w: tensor<256x512xf32>, %b: tensor<512xf32>) -> tensor<128x512xf32> {
  %r = nova.linear %x, %w, %b : tensor<128x256xf32>, tensor<256x512xf32>, tensor<512xf32>
  return %r : tensor<128x512xf32>
}
func.func @p02(%A: tensor<256x128xf32>, %B: tensor<128x512xf32>, %C: tensor<256x512xf32>) -> tensor<256x512xf32> {
  %r = linalg.matmul ins(%A, %B : tensor<256x128xf32>, tensor<128x512xf32>) outs(%C : tensor<256x512xf32>) -> tensor<256x512xf32>
  return %r : tensor<256x512xf32>
}
func.func @p06(%A: tensor<128x128xf32>, %B: tensor<128x128xf32>, %C: tensor<128x128xf32>) -> tensor<128x128xf32> {
  %r = linalg.matmul ins(%A, %B : tensor<128x128xf32>, tensor<128x128xf32>) outs(%C : tensor<128x128xf32>) -> tensor<128x128xf32>
  return %r : tensor<128x128xf32>
}
func.func @p11(%A: tensor<128x256xf32>, %B: tensor<256x512xf32>, %C: tensor<128x512xf32>) -> tensor<128x512xf32> {
  %r = linalg.matmul ins(%A, %B : tensor<128x256xf32>, tensor<256x512xf32>) outs(%C : tensor<128x512xf32>) -> tensor<128x512xf32>
  return %r : tensor<128x512xf32>
}
"""


def test_reference_pipeline_test_shapes(cuda):
    p = nova_run.Program(REF_SHAPES)
    A = S.uniform((100, 300), 95)
    B = S.uniform((300, 200), 95, offset=A.size)
    (r,) = p.run("p01", A, B)
    assert np.array_equal(r, ref.gemm(A, B)[0])
    A3 = S.uniform((4, 64, 256), 96)
    B3 = S.uniform((4, 256, 64), 96, offset=A3.size)
    (r,) = p.run("p03", A3, B3)
    assert np.array_equal(r, ref.gemm(A3, B3))
    A1 = S.uniform((1, 128, 256), 97)
    B1 = S.uniform((1, 256, 128), 97, offset=A1.size)
    (r,) = p.run("p03b", A1, B1)
    assert np.array_equal(r, ref.gemm(A1, B1))
    bias2 = S.uniform((100, 200), 98)
    (r,) = p.run("p04", A, B, bias2)
    assert np.array_equal(r, ref.binary(ref.gemm(A, B)[0], bias2, ref.ADD))
    x = S.uniform((128, 256), 99)
    w = S.uniform((256, 512), 99, offset=x.size)
    b = S.uniform((512,), 99, offset=x.size + w.size)
    (r,) = p.run("p13", x, w, b)
    assert np.array_equal(r, ref.gemm(x, w, bias=b, epilogue=ref.EPI_BIAS)[0])


@pytest.mark.parametrize("name,m,n,k", [("p02", 256, 512, 128), ("p06", 128, 128, 128),
                                        ("p11", 128, 512, 256)])
def test_reference_pipeline_tests_accumulating_into_outs(cuda, name, m, n, k):
    """02_matmul_aligned.mlir, 06_matmul_exact_tile.mlir and
    11_lowering_config.mlir run linalg.matmul into a function argument C:
    the result is C + A . B with each sum starting from C (bit-exact against
    the oracle), and C itself keeps its data, on host arrays and on device."""
    import torch
    p = nova_run.Program(REF_SHAPES)
    A = S.uniform((m, k), 101)
    B = S.uniform((k, n), 101, offset=A.size)
    C = S.uniform((m, n), 102)
    want = ref.gemm_accumulate(A, B, C)[0]
    (r,) = p.run(name, A, B, C)
    assert np.array_equal(r, want)
    dA, dB, dC = (torch.from_numpy(np.ascontiguousarray(x)).to(cuda) for x in (A, B, C))
    (dr,) = p.run_device(name, dA, dB, dC)
    torch.cuda.synchronize()
    assert np.array_equal(dr.cpu().numpy(), want)
    assert np.array_equal(dC.cpu().numpy(), C)


def test_reference_batch_shape_bf16_into_f32_outs(cuda):
    """03_batch_matmul.mlir's shape with bf16 ins and zero-filled f32 outs
    (the F1 form): f32 accumulate on the matrix cores, at the bf16 bar."""
    text = """func.func @b(%A: tensor<4x64x256xbf16>, %B: tensor<4x256x64xbf16>) -> tensor<4x64x64xf32> {
      %z = arith.constant 0.000000e+00 : f32
      %e = tensor.empty() : tensor<4x64x64xf32>
      %c = linalg.fill ins(%z : f32) outs(%e : tensor<4x64x64xf32>) -> tensor<4x64x64xf32>
      %r = linalg.batch_matmul ins(%A, %B : tensor<4x64x256xbf16>, tensor<4x256x64xbf16>) outs(%c : tensor<4x64x64xf32>) -> tensor<4x64x64xf32>
      return %r : tensor<4x64x64xf32>
    }"""
    A = S.uniform((4, 64, 256), 100, dtype=S.BF16)
    B = S.uniform((4, 256, 64), 100, dtype=S.BF16, offset=A.size)
    (r,) = nova_run.Program(text).run("b", A, B)
    assert_close_lp(r, ref.gemm(A, B, adt=S.BF16, bdt=S.BF16), "03 shape bf16")


def test_materialised_zero_fills(cuda):
    """A zero fill that is read (here: returned) is written on the device: by
    the fill kernel when its byte count is a multiple of four, else by a
    memset (the odd bf16 count), over buffers that held other data before."""
    import torch
    text = """func.func @z(%x: tensor<3x5xf32>, %y: tensor<3x5xbf16>) -> (tensor<3x5xf32>, tensor<3x5xbf16>, tensor<4x6xbf16>) {
      %z = arith.constant 0.000000e+00 : f32
      %zb = arith.constant 0.000000e+00 : bf16
      %f = linalg.fill ins(%z : f32) outs(%x : tensor<3x5xf32>) -> tensor<3x5xf32>
      %g = linalg.fill ins(%zb : bf16) outs(%y : tensor<3x5xbf16>) -> tensor<3x5xbf16>
      %e = tensor.empty() : tensor<4x6xbf16>
      %h = linalg.fill ins(%zb : bf16) outs(%e : tensor<4x6xbf16>) -> tensor<4x6xbf16>
      return %f, %g, %h : tensor<3x5xf32>, tensor<3x5xbf16>, tensor<4x6xbf16>
    }"""
    p = nova_run.Program(text)
    plan = p.plan("z")
    assert plan.count("nova_hip_fill_f32") == 2 and plan.count("hipMemsetAsync") == 1
    x = torch.full((3, 5), 7.0, device=cuda)
    y = torch.full((3, 5), 7.0, device=cuda, dtype=torch.bfloat16)
    res = [torch.full(s, 9.0, device=cuda, dtype=d) for s, d in
           (((3, 5), torch.float32), ((3, 5), torch.bfloat16), ((4, 6), torch.bfloat16))]
    out = p.run_device("z", x, y, results=res)
    torch.cuda.synchronize()
    for t in out:
        assert (t.float() == 0).all()
    assert (x == 7).all() and (y.float() == 7).all()
