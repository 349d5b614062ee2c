"""Pins the oracle's program-glue restatements (oracle/nova_cpu_ref.c:
nova_ref_binary_f32, nova_ref_gelu_backward_f32, nova_ref_gather_f32,
nova_ref_scatter_add_f32, nova_ref_reduce_sum_f32, nova_ref_index_to_i32)
against independent checks: numpy's own f32 operators, an f64 central
difference of the GELU forward, numpy fancy indexing and np.add.at (which
adds in index order, as the CPU pipeline does), integer-valued sums that are
exact in any order, and the zero-extension of 16-bit indices."""
import math

import numpy as np

import nova_cpu_ref as ref


def rng(seed):
    return np.random.default_rng(seed)


def test_binary_matches_numpy_f32_with_broadcasting():
    r = rng(1)
    a = r.standard_normal((2, 3, 5)).astype(np.float32)
    for b in (r.standard_normal((2, 3, 5)), r.standard_normal((1, 3, 5)),
              r.standard_normal((5,)), r.standard_normal((1,)), r.standard_normal((2, 1, 1))):
        b = b.astype(np.float32) + np.float32(3.0)  # keep the divisor away from 0
        for op, f in ((ref.ADD, np.add), (ref.SUB, np.subtract), (ref.MUL, np.multiply),
                      (ref.DIV, np.divide)):
            got = ref.binary(a, b, op)
            assert got.shape == np.broadcast_shapes(a.shape, b.shape)
            assert np.array_equal(got, f(a, b, dtype=np.float32)), (op, b.shape)


def gelu64(x):
    return 0.5 * x * (1.0 + np.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3)))


def test_gelu_backward_is_the_derivative_of_the_forward():
    x = np.linspace(-6, 6, 2001, dtype=np.float64)
    h = 1e-5
    d = (gelu64(x + h) - gelu64(x - h)) / (2 * h)
    go = np.full(x.shape, 1.0, np.float32)
    got = ref.gelu_backward(go, x.astype(np.float32)).astype(np.float64)
    # f32 evaluation of the analytic derivative against the f64 difference
    assert np.max(np.abs(got - d)) < 2e-6
    # a dropped term (either half of the product rule) would be off by O(0.1)
    half = 0.5 * (1 + np.tanh(0.797884583 * (x + 0.044715 * x ** 3)))
    assert np.max(np.abs(half - d)) > 0.05


def test_gelu_backward_closed_forms_and_linearity_in_grad():
    assert ref.lib().nova_ref_gelu_backward_f32(3.0, 0.0) == 1.5  # gelu'(0) = 1/2
    assert abs(ref.lib().nova_ref_gelu_backward_f32(1.0, 12.0) - 1.0) < 1e-6
    assert abs(ref.lib().nova_ref_gelu_backward_f32(1.0, -12.0)) < 1e-6
    r = rng(2)
    x = r.standard_normal(1000).astype(np.float32)
    g = r.standard_normal(1000).astype(np.float32)
    one = ref.gelu_backward(np.ones_like(x), x)
    assert np.array_equal(ref.gelu_backward(g, x), (g * one).astype(np.float32))


def test_gather_matches_fancy_indexing_and_zero_extends_i16():
    r = rng(3)
    V, D = 40050, 3
    table = r.standard_normal((V, D)).astype(np.float32)
    idx = np.array([0, 5, 40001, 32767, 32768, 7, 7], dtype=np.int64)
    want = table[idx]
    for dt in (np.int64, np.int32):
        assert np.array_equal(ref.gather(table, idx.astype(dt)), want)
    # 40001 and 32768 do not fit i16: as 16-bit patterns they are negative,
    # and zero-extension must read them back as 40001 and 32768
    bits = idx.astype(np.uint16).view(np.int16)
    assert bits[2] < 0 and bits[4] < 0
    assert np.array_equal(ref.gather(table, bits), want)
    out = ref.gather(table, np.array([[1, V], [-1, 2]], np.int64))
    assert out.shape == (2, 2, D)
    assert np.isnan(out[0, 1]).all() and np.isnan(out[1, 0]).all()
    assert np.array_equal(out[0, 0], table[1]) and np.array_equal(out[1, 1], table[2])


def test_scatter_add_matches_add_at_in_order_and_skips_out_of_range():
    r = rng(4)
    V, D, n = 50, 7, 400
    base = r.standard_normal((V, D)).astype(np.float32)
    idx = r.integers(0, V, n).astype(np.int64)
    src = r.standard_normal((n, D)).astype(np.float32)
    want = base.copy()
    np.add.at(want, idx, src)  # unbuffered, in index order
    assert np.array_equal(ref.scatter_add(base, idx, src), want)
    # out-of-range rows are skipped
    bad = idx.copy()
    bad[::5] = V + 3
    keep = bad < V
    want2 = base.copy()
    np.add.at(want2, bad[keep], src[keep])
    assert np.array_equal(ref.scatter_add(base, bad, src), want2)
    # i16 with zero-extension: 16-bit patterns of indices >= 32768
    V2 = 40000
    base2 = np.zeros((V2, 2), np.float32)
    i16 = np.array([33000, 5, 33000], np.int64).astype(np.uint16).view(np.int16)
    out = ref.scatter_add(base2, i16, np.ones((3, 2), np.float32))
    assert out[33000, 0] == 2.0 and out[5, 1] == 1.0 and out.sum() == 6.0


def test_reduce_sum_is_sequential_over_the_dim():
    r = rng(5)
    x = r.standard_normal((3, 9, 4, 5)).astype(np.float32)
    for dim in range(4):
        got = ref.reduce_sum(x, dim)
        xs = np.moveaxis(x, dim, 0)
        acc = np.zeros(xs.shape[1:], np.float32)
        for j in range(xs.shape[0]):
            acc = (acc + xs[j]).astype(np.float32)
        assert np.array_equal(got, acc), dim
    xi = r.integers(-50, 50, (8, 1024, 3)).astype(np.float32)
    assert np.array_equal(ref.reduce_sum(xi, 0), xi.astype(np.int64).sum(0).astype(np.float32))


def test_index_to_i32_zero_extends_narrow_and_truncates_i64():
    i16 = np.array([0, 1, -1, -32768], np.int16)
    assert ref.index_to_i32(i16).tolist() == [0, 1, 65535, 32768]
    i64 = np.array([3, 2 ** 32 + 7, -2], np.int64)
    assert ref.index_to_i32(i64).tolist() == [3, 7, -2]
    assert math.isclose(float(ref.index_to_i32(np.array([9], np.int32))[0]), 9.0)
