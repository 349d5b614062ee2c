"""Pins the CPU oracle (oracle/nova_cpu_ref.c) before anything is compared
against it.  The reference cannot be built here (needs MLIR 21), so each
function is pinned by the reference's own known-answer test, closed forms,
invariants, f64 brute force, and order-sensitive cases chosen so that a
plausible restatement mistake fails (wrong accumulation order or precision,
bias added last instead of first, wrong mean chunking, a dropped GELU term).
"""
import json
import math
import os

import numpy as np
import pytest

import nova_cpu_ref as ref
from conftest import GOLDEN

F32, BF16, F16 = ref.F32, ref.BF16, ref.F16


def rng(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------- GEMM -----

def test_wrapper_kat_golden():
    """test/wrapper.c:94-100: ones(4096x4096) . ones + 0.5 == 4096.5 (+-0.01)."""
    with open(os.path.join(GOLDEN, "wrapper_kat.json")) as f:
        kat = json.load(f)
    n, k = kat["M"], kat["K"]
    A = np.full((n, k), kat["a"], np.float32)
    B = np.full((k, kat["N"]), kat["b"], np.float32)
    bias = np.full(kat["N"], kat["bias"], np.float32)
    idx = np.array([[0, 0, 0], [0, n - 1, kat["N"] - 1], [0, 17, 4000]], np.int64)
    out = ref.gemm_sampled(A, B, idx, bias=bias, epilogue=ref.EPI_BIAS)
    assert np.all(np.abs(out - kat["expected"]) < kat["tol"])
    assert np.all(out == np.float32(4096.5))  # exact: every partial sum is representable


def test_gemm_integer_grid_exact():
    """Small-integer inputs accumulate exactly in f32 (K*max^2 < 2^24), so the
    result must equal the integer matmul bit for bit -- for every layout."""
    g = rng(0)
    A = g.integers(-8, 9, size=(3, 37, 53)).astype(np.float32)
    B = g.integers(-8, 9, size=(3, 53, 29)).astype(np.float32)
    want = np.einsum("bmk,bkn->bmn", A.astype(np.int64), B.astype(np.int64)).astype(np.float32)
    assert np.array_equal(ref.gemm(A, B), want)
    # transposed views of the same data
    At = np.ascontiguousarray(A.transpose(0, 2, 1)).transpose(0, 2, 1)
    Bt = np.ascontiguousarray(B.transpose(0, 2, 1)).transpose(0, 2, 1)
    assert np.array_equal(ref.gemm(At, Bt), want)


def test_gemm_identity_and_unit_vector():
    g = rng(1)
    A = g.standard_normal((40, 40)).astype(np.float32)
    I = np.eye(40, dtype=np.float32)
    assert np.array_equal(ref.gemm(A, I)[0], A)
    e = np.zeros((40, 1), np.float32)
    e[7, 0] = 1.0
    assert np.array_equal(ref.gemm(A, e)[0][:, 0], A[:, 7])


def test_gemm_f64_brute_force_bound():
    """|C - C64| <= gamma_K * sum|a||b| with gamma_K = K u / (1 - K u)."""
    g = rng(2)
    for (m, n, k) in [(1, 1, 1), (5, 7, 3), (33, 17, 129), (64, 64, 256)]:
        A = g.uniform(-1, 1, (m, k)).astype(np.float32)
        B = g.uniform(-1, 1, (k, n)).astype(np.float32)
        c = ref.gemm(A, B)[0].astype(np.float64)
        c64 = A.astype(np.float64) @ B.astype(np.float64)
        u = 2.0 ** -24
        gam = k * u / (1 - k * u)
        bound = gam * (np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64))
        assert np.all(np.abs(c - c64) <= bound + 1e-30)


def test_gemm_sequential_f32_order():
    """Accumulation is f32, k ascending: (1e8 + 1) - 1e8 == 0, where f64
    accumulation or any reordering that pairs the big terms first gives 1."""
    A = np.array([[1e8, 1.0, -1e8]], np.float32)
    B = np.ones((3, 1), np.float32)
    assert ref.gemm(A, B)[0, 0, 0] == 0.0
    A2 = np.array([[1e8, -1e8, 1.0]], np.float32)
    assert ref.gemm(A2, B)[0, 0, 0] == 1.0


def test_gemm_bias_initialises_accumulator():
    """FuseMatmulBias.cpp:184-188: C = bias + sum_k (bias first).  With
    bias 1 and terms [1e8, -1e8]: (1 + 1e8) - 1e8 = 0; bias-last gives 1."""
    A = np.array([[1e8, -1e8]], np.float32)
    B = np.ones((2, 1), np.float32)
    bias = np.array([1.0], np.float32)
    assert ref.gemm(A, B, bias=bias, epilogue=ref.EPI_BIAS)[0, 0, 0] == 0.0


def test_gemm_low_precision_inputs_widen_exactly():
    """bf16/f16 operands are widened exactly (extf) and products are exact in
    f32; integer grids therefore give the exact integer result."""
    g = rng(3)
    Af = g.integers(-16, 17, size=(2, 21, 64)).astype(np.float32)
    Bf = g.integers(-16, 17, size=(2, 64, 19)).astype(np.float32)
    want = np.einsum("bmk,bkn->bmn", Af.astype(np.int64), Bf.astype(np.int64)).astype(np.float32)
    for dt in (BF16, F16):
        a = np.vectorize(lambda v: ref.lib().nova_ref_f32_to_bf16(v) if dt == BF16
                         else ref.lib().nova_ref_f32_to_f16(v), otypes=[np.uint16])(Af)
        b = np.vectorize(lambda v: ref.lib().nova_ref_f32_to_bf16(v) if dt == BF16
                         else ref.lib().nova_ref_f32_to_f16(v), otypes=[np.uint16])(Bf)
        assert np.array_equal(ref.gemm(a, b, adt=dt, bdt=dt), want)


def test_gemm_sampled_matches_dense():
    g = rng(4)
    A = g.uniform(-1, 1, (2, 30, 50)).astype(np.float32)
    B = g.uniform(-1, 1, (2, 50, 20)).astype(np.float32)
    bias = g.uniform(-1, 1, 20).astype(np.float32)
    dense = ref.gemm(A, B, bias=bias, epilogue=ref.EPI_BIAS_GELU)
    idx = np.stack([g.integers(0, 2, 100), g.integers(0, 30, 100), g.integers(0, 20, 100)], 1)
    s = ref.gemm_sampled(A, B, idx, bias=bias, epilogue=ref.EPI_BIAS_GELU)
    assert np.array_equal(s, dense[idx[:, 0], idx[:, 1], idx[:, 2]])


def test_gemm_bf16_output_is_rne_of_f32():
    g = rng(5)
    A = g.uniform(-1, 1, (1, 16, 32)).astype(np.float32)
    B = g.uniform(-1, 1, (1, 32, 24)).astype(np.float32)
    c32 = ref.gemm(A, B)
    cb = ref.gemm(A, B, cdt=BF16)
    want = np.vectorize(ref.lib().nova_ref_f32_to_bf16, otypes=[np.uint16])(c32)
    assert np.array_equal(cb, want)


# ---------------------------------------------------------------- casts ----

def test_bf16_round_to_nearest_even():
    L = ref.lib()
    one = 1.0
    # ties: 1 + 2^-8 is halfway between 1 and 1 + 2^-7 -> even (1.0)
    assert L.nova_ref_bf16_to_f32(L.nova_ref_f32_to_bf16(one + 2 ** -8)) == 1.0
    # 1 + 3*2^-8 halfway between 1+2^-7 and 1+2^-6 -> even (1 + 2^-6)
    assert L.nova_ref_bf16_to_f32(L.nova_ref_f32_to_bf16(one + 3 * 2 ** -8)) == 1 + 2 ** -6
    assert L.nova_ref_bf16_to_f32(L.nova_ref_f32_to_bf16(one + 2 ** -8 + 2 ** -20)) == 1 + 2 ** -7
    # widen is exact: every bf16 pattern round-trips
    bits = np.arange(0, 65536, dtype=np.uint32)
    finite = (bits & 0x7F80) != 0x7F80
    for h in bits[finite][::97]:
        assert L.nova_ref_f32_to_bf16(L.nova_ref_bf16_to_f32(int(h))) == h


def test_f16_matches_numpy_rne():
    L = ref.lib()
    g = rng(6)
    vals = np.concatenate([
        g.standard_normal(4000).astype(np.float32) * 10,
        np.array([0.0, -0.0, 65504.0, 65520.0, 7e4, 6e-8, 5.96e-8, 2.98e-8, 1e-5,
                  6.1035156e-05, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11], np.float32)])
    mine = np.array([L.nova_ref_f32_to_f16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(mine, vals.astype(np.float16).view(np.uint16))
    allh = np.arange(65536, dtype=np.uint16)
    f = allh.view(np.float16).astype(np.float32)
    ok = np.isfinite(f)
    mine_w = np.array([L.nova_ref_f16_to_f32(int(h)) for h in allh[ok][::13]], np.float32)
    assert np.array_equal(mine_w, f[ok][::13])


# ---------------------------------------------------------------- GELU -----

def test_gelu_special_values_and_f64_formula():
    assert ref.lib().nova_ref_gelu_f32(0.0) == 0.0
    x = np.linspace(-8, 8, 4001).astype(np.float32)
    y = ref.gelu(x).astype(np.float64)
    x64 = x.astype(np.float64)
    y64 = 0.5 * x64 * (1 + np.tanh(0.7978845608028654 * (x64 + 0.044715 * x64 ** 3)))
    assert np.all(np.abs(y - y64) <= 1e-6 * np.abs(x64) + 1e-6)
    # odd part: gelu(x) - gelu(-x) == x
    assert np.allclose(y - ref.gelu(-x).astype(np.float64), x64, atol=2e-6)
    # tails: -> x for x >> 0, -> 0 for x << 0
    assert np.all(np.abs(ref.gelu(np.array([10.0, 30.0], np.float32)) - [10.0, 30.0]) < 1e-5)
    assert np.all(np.abs(ref.gelu(np.array([-10.0, -30.0], np.float32))) < 1e-5)
    # the cubic term matters: without it gelu(2) would be 0.5*2*(1+tanh(1.5958))
    assert abs(ref.lib().nova_ref_gelu_f32(2.0) - 1.9545977) < 1e-6


# ---------------------------------------------------------- LayerNorm -----

def test_layer_norm_constant_row():
    x = np.full((3, 64), 2.5, np.float32)
    g = np.linspace(0.5, 1.5, 64).astype(np.float32)
    b = np.linspace(-1, 1, 64).astype(np.float32)
    y, s, r = ref.layer_norm(x, g, b)
    assert np.array_equal(y, np.broadcast_to(b, y.shape))
    assert np.all(s == 160.0)
    assert np.allclose(r, 1.0 / math.sqrt(1e-5), rtol=1e-6)


def test_layer_norm_moments_and_affine_invariance():
    gen = rng(7)
    x = gen.standard_normal((8, 1000)).astype(np.float32)
    one, zero = np.ones(1000, np.float32), np.zeros(1000, np.float32)
    y, s, r = ref.layer_norm(x, one, zero)
    assert np.all(np.abs(y.mean(1)) < 1e-5)
    var = y.astype(np.float64).var(1)
    assert np.all(np.abs(var * (1 + 1e-5 * r.astype(np.float64) ** 2) - 1) < 1e-3)
    y2, _, _ = ref.layer_norm(3.0 * x + 0.25, one, zero)
    assert np.allclose(y2, y, atol=2e-4)
    s64 = x.astype(np.float64).sum(1)
    bound = 1000 * 2.0 ** -24 * np.abs(x).astype(np.float64).sum(1) * 1.01
    assert np.all(np.abs(s - s64) <= bound)


def test_layer_norm_f64_reference():
    gen = rng(8)
    x = gen.standard_normal((16, 257)).astype(np.float32) * 3 + 1
    g = (1 + 0.1 * gen.standard_normal(257)).astype(np.float32)
    b = (0.1 * gen.standard_normal(257)).astype(np.float32)
    y, s, r = ref.layer_norm(x, g, b)
    x64 = x.astype(np.float64)
    mu = x64.mean(1, keepdims=True)
    var = (x64 ** 2).mean(1, keepdims=True) - mu ** 2
    y64 = (x64 - mu) / np.sqrt(var + 1e-5) * g + b
    assert np.allclose(y, y64, rtol=1e-4, atol=1e-4)
    assert np.allclose(r, 1 / np.sqrt(var[:, 0] + 1e-5), rtol=1e-5)


def test_layer_norm_uses_single_pass_variance():
    """var = Q/D - mean^2 (NovaToLinalgGeneric.cpp:2101-2105), not the
    two-pass sum((x-mean)^2)/D: with a large offset the one-pass form loses
    the variance to cancellation, which pins the formula."""
    x = (np.float32(3000.0) + np.array([[0.0, 0.5] * 32], np.float32))
    y, s, r = ref.layer_norm(x, np.ones(64, np.float32), np.zeros(64, np.float32))
    mean = np.float32(s[0] * np.float32(1 / 64))
    q = np.float32(0)
    for v in x[0]:
        q = np.float32(q + np.float32(v * v))
    var = np.float32(np.float32(q * np.float32(1 / 64)) - np.float32(mean * mean))
    want = np.float32(1.0) / np.sqrt(np.float32(var + np.float32(1e-5)))
    assert r[0] == want
    two_pass = 1 / math.sqrt(0.0625 + 1e-5)
    assert abs(float(r[0]) - two_pass) > 0.5  # the forms really differ here


# ---------------------------------------------------------------- SCE -----

def test_mean_64_chunk_order():
    """lowerFullReduceMeanToSCF: 64 chunks of ceil(n/64) summed separately.
    n=128 -> chunks of 2: [1e8,1] -> 1e8; [-1e8,1] -> -1e8; total 0.  A flat
    sequential sum gives 1/128, f64 gives 2/128."""
    v = np.zeros(128, np.float32)
    v[:4] = [1e8, 1.0, -1e8, 1.0]
    assert ref.mean(v) == 0.0
    v2 = np.arange(10, dtype=np.float32)  # n < 64: chunks of 1, rest empty
    assert ref.mean(v2) == np.float32(45.0 / 10.0)
    gen = rng(9)
    v3 = gen.standard_normal(4096).astype(np.float32)
    assert abs(float(ref.mean(v3)) - v3.astype(np.float64).mean()) < 1e-6


def test_sce_closed_forms():
    C = 1000
    x = np.zeros((4, C), np.float32)
    t = np.array([0, 5, 999, 500], np.int32)
    sm, loss, lr = ref.sce(x, t, softmax=True)
    assert np.allclose(lr, math.log(C), rtol=1e-6)
    assert np.allclose(sm.sum(1), 1.0, atol=1e-5)
    x2 = np.zeros((4, C), np.float32)
    x2[np.arange(4), t] = 100.0
    _, loss2, lr2 = ref.sce(x2, t)
    assert np.all(lr2 < 1e-30 + 1e-6) and np.all(lr2 >= 0)
    gen = rng(10)
    x3 = gen.normal(0, 2, (8, 300)).astype(np.float32)
    t3 = gen.integers(0, 300, 8).astype(np.int32)
    _, l3, lr3 = ref.sce(x3, t3)
    _, l4, lr4 = ref.sce(x3 + np.float32(7.0), t3)
    assert np.allclose(lr3, lr4, atol=2e-5)
    assert np.all(lr3 >= 0)
    x64 = x3.astype(np.float64)
    lse = np.log(np.exp(x64 - x64.max(1, keepdims=True)).sum(1)) + x64.max(1)
    want = lse - x64[np.arange(8), t3]
    assert np.allclose(lr3, want, rtol=1e-5, atol=1e-5)
    assert abs(float(l3[0]) - want.mean()) < 1e-5


def test_sce_rejects_out_of_range_label():
    with pytest.raises(ValueError):
        ref.sce(np.zeros((2, 5), np.float32), np.array([0, 5], np.int32))


# ------------------------------------------------- narrow accumulator ------
# linalg.matmul with bf16 / f16 outs accumulates in that type
# (NovaToLinalg.cpp:1027-1049).  Pinned by sums that stall where the narrow
# type runs out of significand bits, by bias-first order, and against
# numpy's float16 / torch's CPU bfloat16 arithmetic (independent rounding
# code) on random data.

def _bits(x, dt):
    x = np.asarray(x, np.float32)
    f = ref.lib().nova_ref_f32_to_bf16 if dt == BF16 else ref.lib().nova_ref_f32_to_f16
    return np.vectorize(lambda v: f(float(v)), otypes=[np.uint16])(x)


def _widen(h, dt):
    f = ref.lib().nova_ref_bf16_to_f32 if dt == BF16 else ref.lib().nova_ref_f16_to_f32
    return np.vectorize(lambda v: f(int(v)), otypes=[np.float32])(h)


@pytest.mark.parametrize("dt,K,stall", [(F16, 4000, 2048.0), (BF16, 300, 256.0)])
def test_narrow_accumulator_stalls(dt, K, stall):
    """sum of K ones: f16 stops at 2048 (2048 + 1 ties to even), bf16 at 256;
    an f32 accumulator stored narrow would give K."""
    A = _bits(np.ones((1, K)), dt)
    B = _bits(np.ones((K, 3)), dt)
    got = _widen(ref.gemm_acc_out(A, B, dt=dt), dt)
    assert np.all(got == stall)
    wide = _widen(ref.gemm(A, B, adt=dt, bdt=dt, cdt=dt), dt)
    assert np.all(wide == K)


def test_narrow_accumulator_bias_first():
    """FuseMatmulBias: the bias initialises the accumulator.  2048 + 1 + 1 + 1
    in f16 stays 2048; bias last (3 + 2048) would give 2052."""
    A = _bits(np.ones((2, 3)), F16)
    B = _bits(np.ones((3, 4)), F16)
    bias = _bits(np.full(4, 2048.0), F16)
    got = _widen(ref.gemm_acc_out(A, B, dt=F16, bias=bias), F16)
    assert np.all(got == 2048.0)


def test_narrow_accumulator_matches_numpy_float16():
    g = rng(11)
    A = g.uniform(-2, 2, (2, 9, 37)).astype(np.float16)
    B = g.uniform(-2, 2, (2, 37, 7)).astype(np.float16)
    want = np.zeros((2, 9, 7), np.float16)
    for b in range(2):
        for i in range(9):
            for j in range(7):
                acc = np.float16(0)
                for k in range(37):
                    acc = np.float16(acc + np.float16(A[b, i, k] * B[b, k, j]))
                want[b, i, j] = acc
    got = ref.gemm_acc_out(A.view(np.uint16), B.view(np.uint16), dt=F16)
    assert np.array_equal(got, want.view(np.uint16))
    # transposed operand views give the same bits
    At = np.ascontiguousarray(A.view(np.uint16).transpose(0, 2, 1)).transpose(0, 2, 1)
    assert np.array_equal(ref.gemm_acc_out(At, B.view(np.uint16), dt=F16), got)


def test_narrow_accumulator_matches_torch_bfloat16():
    import torch
    g = rng(12)
    A = torch.from_numpy(g.uniform(-2, 2, (5, 23)).astype(np.float32)).to(torch.bfloat16)
    B = torch.from_numpy(g.uniform(-2, 2, (23, 6)).astype(np.float32)).to(torch.bfloat16)
    bias = torch.from_numpy(g.uniform(-1, 1, (6,)).astype(np.float32)).to(torch.bfloat16)
    want = torch.empty((5, 6), dtype=torch.bfloat16)
    for i in range(5):
        for j in range(6):
            acc = bias[j].clone()
            for k in range(23):
                acc = acc + A[i, k] * B[k, j]   # each op rounded to bf16 on the CPU
            want[i, j] = acc
    bits = lambda t: t.view(torch.int16).numpy().view(np.uint16)
    got = ref.gemm_acc_out(bits(A), bits(B), dt=BF16, bias=bits(bias))[0]
    assert np.array_equal(got, bits(want))


# ---- linalg.matmul on data-holding outs (C0 + A . B, from C0) ------------

def test_gemm_accumulate_from_zero_and_from_bias_rows():
    """Starting from zeros it is the plain GEMM; from C0 rows equal to a bias
    it is the bias-first GEMM (FuseMatmulBias's accumulator init), bit for
    bit.  C0 is left unmodified."""
    g = rng(21)
    A = g.uniform(-1, 1, (3, 17, 29)).astype(np.float32)
    B = g.uniform(-1, 1, (3, 29, 11)).astype(np.float32)
    zero = np.zeros((3, 17, 11), np.float32)
    assert np.array_equal(ref.gemm_accumulate(A, B, zero), ref.gemm(A, B))
    assert not zero.any()
    bias = g.uniform(-2, 2, 11).astype(np.float32)
    rows = np.broadcast_to(bias, (3, 17, 11)).copy()
    assert np.array_equal(ref.gemm_accumulate(A, B, rows),
                          ref.gemm(A, B, bias=bias, epilogue=ref.EPI_BIAS))


def test_gemm_accumulate_starts_from_c():
    """(1 + 1e8) - 1e8 = 0 in f32 when the sum starts from C0 = 1; adding C0
    after the products ((1e8 - 1e8) + 1) would give 1."""
    A = np.array([[1.0, 1.0]], np.float32)
    B = np.array([[1e8], [-1e8]], np.float32)
    assert ref.gemm_accumulate(A, B, np.ones((1, 1), np.float32))[0, 0, 0] == 0.0


def test_gemm_accumulate_integer_grid_exact():
    g = rng(22)
    A = g.integers(-8, 9, (2, 33, 40)).astype(np.float32)
    B = g.integers(-8, 9, (2, 40, 19)).astype(np.float32)
    C0 = g.integers(-1000, 1001, (2, 33, 19)).astype(np.float32)
    want = C0.astype(np.int64) + np.einsum("bmk,bkn->bmn", A.astype(np.int64), B.astype(np.int64))
    assert np.array_equal(ref.gemm_accumulate(A, B, C0), want.astype(np.float32))
    # a transposed A view, a rank-2 B broadcast over the batch
    At = np.ascontiguousarray(A.transpose(0, 2, 1)).transpose(0, 2, 1)
    want2 = C0.astype(np.int64) + np.einsum("bmk,kn->bmn", A.astype(np.int64),
                                            B[0].astype(np.int64))
    assert np.array_equal(ref.gemm_accumulate(At, B[0], C0), want2.astype(np.float32))


def test_gemm_accumulate_narrow_outs():
    """f16 outs: from zeros it is the narrow-accumulator GEMM; from 2048 a
    sum of ones stays 2048 (each partial sum rounded to f16, C0 first)."""
    g = rng(23)
    A = g.uniform(-2, 2, (9, 31)).astype(np.float16).view(np.uint16)
    B = g.uniform(-2, 2, (31, 5)).astype(np.float16).view(np.uint16)
    zero = np.zeros((1, 9, 5), np.uint16)
    assert np.array_equal(ref.gemm_accumulate(A, B, zero, adt=F16, bdt=F16, cdt=F16),
                          ref.gemm_acc_out(A, B, dt=F16))
    ones_a = _bits(np.ones((2, 3)), F16)
    ones_b = _bits(np.ones((3, 4)), F16)
    c0 = _bits(np.full((1, 2, 4), 2048.0), F16)
    got = _widen(ref.gemm_accumulate(ones_a, ones_b, c0, adt=F16, bdt=F16, cdt=F16), F16)
    assert np.all(got == 2048.0)
