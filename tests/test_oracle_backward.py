"""Pins the backward half of the CPU oracle (nova_ref_sce_backward_f32,
nova_ref_layer_norm_backward_f32, nova_ref_col_sum and the linear / matmul
backward compositions) before any GPU result is compared with it.

The reference holds no known answers for these ops, so each function is
pinned by what the mathematics fixes: finite differences of an f64 forward
(a wrong sign or a dropped term of the LayerNorm gradient fails them), exact
integer column sums, closed forms (rows of the SCE gradient sum to zero,
uniform softmax), f64 brute force, and order-sensitive cases for the
reference's specific choices (multiply by the rounded 1/N, sequential
column sums).
"""
import numpy as np
import pytest

import nova_cpu_ref as ref

F32, BF16 = ref.F32, ref.BF16


def rng(seed):
    return np.random.default_rng(seed)


def softmax64(x):
    x = np.asarray(x, np.float64)
    e = np.exp(x - x.max(axis=1, keepdims=True))
    return e / e.sum(axis=1, keepdims=True)


# ----------------------------------------------------------- SCE backward --

def test_sce_backward_uniform_softmax_closed_form():
    R, C = 6, 10
    sm = np.full((R, C), 0.1, np.float32)
    t = np.array([0, 3, 9, 3, 5, 1], np.int32)
    g = ref.sce_backward(sm, t)
    onehot = np.zeros((R, C))
    onehot[np.arange(R), t] = 1
    want = (0.1 - onehot) / R
    assert np.allclose(g, want, rtol=1e-6, atol=1e-9)
    assert np.all(g[np.arange(R), t] < 0)


def test_sce_backward_f64_and_row_sums():
    g0 = rng(3)
    R, C = 33, 257
    x = g0.normal(0, 2, (R, C)).astype(np.float32)
    t = g0.integers(0, C, R).astype(np.int32)
    sm, _, _ = ref.sce(x, t, softmax=True)
    g = ref.sce_backward(sm, t)
    onehot = np.zeros((R, C))
    onehot[np.arange(R), t] = 1
    want = (softmax64(x) - onehot) / R
    assert np.max(np.abs(g - want)) < 1e-6 / R * 8
    # sum_c (softmax - onehot) = 0 for every row
    assert np.max(np.abs(g.astype(np.float64).sum(axis=1))) < 1e-5 / R


def test_sce_backward_multiplies_by_rounded_reciprocal():
    """The reference scales by getFloatAttr(f32, 1.0/N) with one multiply
    (NovaToLinalgGeneric.cpp:1121-1128), not a division by N.  Find values
    where the two differ and check the oracle takes the multiply."""
    N = 3
    inv = np.float32(1.0 / N)
    cand = np.linspace(0.01, 0.99, 20001, dtype=np.float32)
    diff = cand[(cand * inv) != (cand / np.float32(N))]
    assert diff.size > 0
    p = diff[:4]
    sm = np.tile(np.concatenate([p, [np.float32(0.5)]]).astype(np.float32), (N, 1))
    t = np.full(N, 4, np.int32)  # label on the last column: p stays untouched
    g = ref.sce_backward(sm, t)
    assert np.array_equal(g[:, :4], np.tile(p * inv, (N, 1)))
    assert not np.array_equal(g[:, :4], np.tile(p / np.float32(N), (N, 1)))
    # the label column: (p + (-1)) then the multiply
    assert np.all(g[:, 4] == (np.float32(0.5) - np.float32(1)) * inv)


def test_sce_backward_rejects_out_of_range_label():
    sm = np.full((2, 4), 0.25, np.float32)
    with pytest.raises(ValueError):
        ref.sce_backward(sm, np.array([0, 4], np.int32))
    with pytest.raises(ValueError):
        ref.sce_backward(sm, np.array([-1, 0], np.int32))


# ------------------------------------------------------ LayerNorm backward --

def ln64(x, g, b, eps=1e-5):
    x = np.asarray(x, np.float64)
    m = x.mean(axis=1, keepdims=True)
    v = (x * x).mean(axis=1, keepdims=True) - m * m
    return (x - m) / np.sqrt(v + eps) * g + b


def test_layer_norm_backward_matches_finite_differences():
    """dx of sum(gy * LN(x)) by central differences of an f64 forward.  The
    reference's backward is the exact gradient, so a dropped term or a wrong
    sign in the restatement fails this."""
    g0 = rng(5)
    R, D = 4, 24
    x = g0.normal(0.3, 1.5, (R, D)).astype(np.float32)
    gamma = (1 + g0.normal(0, 0.3, D)).astype(np.float32)
    beta = g0.normal(0, 0.3, D).astype(np.float32)
    gy = g0.normal(0, 1, (R, D)).astype(np.float32)
    _, S, rstd = ref.layer_norm(x, gamma, beta)
    dx, dg, db = ref.layer_norm_backward(gy, x, gamma, S, rstd)
    h = 1e-5
    num = np.zeros((R, D))
    x64 = x.astype(np.float64)
    for r in range(R):
        for d in range(D):
            xp, xm = x64.copy(), x64.copy()
            xp[r, d] += h
            xm[r, d] -= h
            num[r, d] = ((gy * ln64(xp, gamma, beta)).sum() -
                         (gy * ln64(xm, gamma, beta)).sum()) / (2 * h)
    assert np.max(np.abs(dx - num)) < 2e-4 * np.max(np.abs(num))
    # dgamma, dbeta: gradients of sum(gy * LN) w.r.t. gamma and beta
    xhat = (ln64(x, np.ones(D), np.zeros(D)))
    assert np.allclose(dg, (gy * xhat).sum(axis=0), rtol=1e-4, atol=1e-4)
    assert np.allclose(db, gy.astype(np.float64).sum(axis=0), rtol=1e-6, atol=1e-5)


def test_layer_norm_backward_dbeta_integer_exact_and_dx_row_sums():
    g0 = rng(6)
    R, D = 37, 64
    x = g0.normal(0, 1, (R, D)).astype(np.float32)
    gamma = (1 + g0.normal(0, 0.1, D)).astype(np.float32)
    gy = g0.integers(-20, 21, (R, D)).astype(np.float32)
    _, S, rstd = ref.layer_norm(x, gamma, np.zeros(D, np.float32))
    dx, dg, db = ref.layer_norm_backward(gy, x, gamma, S, rstd)
    assert np.array_equal(db, gy.astype(np.int64).sum(axis=0).astype(np.float32))
    # sum_d dx = rstd * (s1 - s1 - (s2/D) * sum_d xhat) ~ 0 since sum xhat ~ 0
    scale = np.abs(gy * gamma).sum(axis=1) * rstd
    assert np.all(np.abs(dx.astype(np.float64).sum(axis=1)) < 1e-4 * scale)


def test_layer_norm_backward_constant_gy_gamma_gives_zero_dx():
    """gy * gamma constant per row: s1 = D c and s2 = c sum xhat ~ 0, so
    dx = rstd (c - c - xhat * ~0) ~ 0."""
    g0 = rng(7)
    R, D = 8, 128
    x = g0.normal(0, 1, (R, D)).astype(np.float32)
    gamma = np.full(D, 2.0, np.float32)
    gy = np.full((R, D), 1.5, np.float32)
    _, S, rstd = ref.layer_norm(x, gamma, np.zeros(D, np.float32))
    dx, _, _ = ref.layer_norm_backward(gy, x, gamma, S, rstd)
    assert np.max(np.abs(dx)) < 1e-5


# --------------------------------------------- column sums, GEMM backward --

def test_col_sum_sequential_order():
    """Sequential f32 over rows: [1, 1e8, -1e8] sums to 0 (the 1 is absorbed
    by 1e8); any reordering or a wider accumulator gives 1."""
    a = np.array([[1.0], [1e8], [-1e8]], np.float32)
    assert ref.col_sum(a)[0] == 0.0
    assert ref.col_sum(a[::-1].copy())[0] == 1.0


def test_col_sum_integer_exact_and_bf16_widening():
    g0 = rng(8)
    a = g0.integers(-100, 101, (300, 77)).astype(np.float32)
    assert np.array_equal(ref.col_sum(a), a.astype(np.int64).sum(axis=0).astype(np.float32))
    bits = (a.view(np.uint32) >> 16).astype(np.uint16)  # small integers are exact in bf16
    assert np.array_equal(ref.col_sum(bits, BF16), ref.col_sum(a))


def test_linear_and_matmul_backward_integer_grid():
    """grad_input = go . W^T, grad_weight = x^T . go, grad_bias = colsum(go),
    grad_a = g . B^T, grad_b = A^T . g: exact on small-integer data."""
    g0 = rng(9)
    M, K, N = 29, 41, 23
    x = g0.integers(-6, 7, (M, K)).astype(np.float32)
    w = g0.integers(-6, 7, (K, N)).astype(np.float32)
    go = g0.integers(-6, 7, (M, N)).astype(np.float32)
    gi, gw, gb = ref.linear_backward(go, x, w)
    i64 = lambda v: v.astype(np.int64)
    assert np.array_equal(gi, (i64(go) @ i64(w).T).astype(np.float32))
    assert np.array_equal(gw, (i64(x).T @ i64(go)).astype(np.float32))
    assert np.array_equal(gb, i64(go).sum(axis=0).astype(np.float32))
    ga, gbb = ref.matmul_backward(go, x, w)
    assert np.array_equal(ga, gi) and np.array_equal(gbb, gw)
