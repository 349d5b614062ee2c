"""Program-glue entry points of libnova_hip on the GPU (binary ops with
broadcasting, fill, gelu, gelu_backward, gather, scatter_add, reduce<sum>,
index widening) against the CPU oracle: bit-exact where the GPU performs the
oracle's operations in the oracle's order (one IEEE op per element, copies,
sequential sums), within the f32 tolerance where a device tanhf or the
atomic add order can differ."""
import numpy as np
import pytest

import nova_cpu_ref as ref
import nova_hip as nh
from conftest import assert_close_f32

pytestmark = pytest.mark.gpu


def dev(a, cuda):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def host(t):
    return t.cpu().numpy()


@pytest.mark.parametrize("sa,sb", [((4, 8, 64), (4, 8, 64)), ((8, 16, 24), (1, 16, 24)),
                                   ((3, 5, 7), (7,)), ((64, 33), (1,)), ((1,), (5, 9)),
                                   ((2, 3, 1, 5), (1, 3, 4, 1))])
def test_binary_bit_exact_with_broadcasting(cuda, sa, sb):
    r = np.random.default_rng(11)
    a = r.standard_normal(sa).astype(np.float32)
    b = (r.standard_normal(sb) + 3.0).astype(np.float32)
    for op in (nh.BIN_ADD, nh.BIN_SUB, nh.BIN_MUL, nh.BIN_DIV):
        got = host(nh.binary(dev(a, cuda), dev(b, cuda), op))
        assert np.array_equal(got, ref.binary(a, b, op)), (sa, sb, op)


def test_binary_in_place_and_large_scalar_scale(cuda):
    import torch
    r = np.random.default_rng(12)
    a = r.standard_normal((8, 1024, 515)).astype(np.float32)
    da = dev(a, cuda)
    nh.binary(da, dev(np.array([0.5], np.float32), cuda), nh.BIN_MUL, out=da)
    assert np.array_equal(host(da), (a * np.float32(0.5)).astype(np.float32))
    b = r.standard_normal(a.shape).astype(np.float32)
    db = dev(b, cuda)
    nh.binary(db, da, nh.BIN_ADD, out=db)
    assert np.array_equal(host(db), ref.binary(b, a * np.float32(0.5), nh.BIN_ADD))
    torch.cuda.synchronize()


def test_fill(cuda):
    import torch
    t = torch.empty((1000, 7), dtype=torch.float32, device=cuda)
    nh.fill(t, 1.5)
    assert (host(t) == 1.5).all()
    u = torch.empty(4096 * 4, dtype=torch.float32, device=cuda)
    nh.fill(u, -0.0)
    assert np.array_equal(host(u).view(np.uint32), np.full(u.numel(), 0x80000000, np.uint32))


def test_gelu_and_gelu_backward(cuda):
    r = np.random.default_rng(13)
    x = (r.standard_normal(200_003) * 3).astype(np.float32)
    g = r.standard_normal(x.shape).astype(np.float32)
    assert_close_f32(host(nh.gelu(dev(x, cuda))), ref.gelu(x), "gelu")
    got = host(nh.gelu_backward(dev(g, cuda), dev(x, cuda)))
    assert_close_f32(got, ref.gelu_backward(g, x), "gelu_backward")
    assert host(nh.gelu_backward(dev(np.array([3.0], np.float32), cuda),
                                 dev(np.array([0.0], np.float32), cuda)))[0] == 1.5


@pytest.mark.parametrize("dt", [np.int16, np.int32, np.int64])
def test_gather_exact_and_out_of_range_nan(cuda, dt):
    r = np.random.default_rng(14)
    V, D = 40050, 96
    table = r.standard_normal((V, D)).astype(np.float32)
    idx = r.integers(0, V if dt != np.int16 else 32767, (8, 100)).astype(np.int64)
    idx[0, :3] = [0, V - 1, 5]
    di = dev(idx.astype(dt), cuda)
    got = host(nh.gather(dev(table, cuda), di))
    assert got.shape == (8, 100, D)
    assert np.array_equal(got, ref.gather(table, idx.astype(dt)))
    if dt == np.int16:  # zero-extension of 16-bit patterns >= 32768
        big = np.array([33000, 40001], np.int64).astype(np.uint16).view(np.int16)
        assert np.array_equal(host(nh.gather(dev(table, cuda), dev(big, cuda))),
                              table[[33000, 40001]])
    else:
        bad = np.array([V, -1, 3], dt)
        out = host(nh.gather(dev(table, cuda), dev(bad, cuda)))
        assert np.isnan(out[:2]).all() and np.array_equal(out[2], table[3])


def test_scatter_add_integer_exact_and_random_close(cuda):
    r = np.random.default_rng(15)
    V, D, n = 1000, 384, 8192
    idx = r.integers(0, V, n).astype(np.int64)
    idx[:50] = 7  # a heavily repeated row
    idx[60] = V + 5  # skipped
    src_i = r.integers(-8, 8, (n, D)).astype(np.float32)  # exact in any order
    base = r.integers(-4, 4, (V, D)).astype(np.float32)
    got = host(nh.scatter_add(dev(base, cuda), dev(idx, cuda), dev(src_i, cuda)))
    assert np.array_equal(got, ref.scatter_add(base, idx, src_i))
    src = r.standard_normal((n, D)).astype(np.float32)
    i16 = idx.astype(np.int16)
    got = host(nh.scatter_add(dev(np.zeros((V, D), np.float32), cuda), dev(i16, cuda),
                              dev(src, cuda)))
    assert_close_f32(got, ref.scatter_add(np.zeros((V, D), np.float32), i16, src), "scatter_add")


@pytest.mark.parametrize("shape,dim", [((8, 1024, 384), 0), ((3, 100, 7), 1), ((5, 9), 1),
                                       ((1000, 3), 0), ((2, 3, 4, 5), 2)])
def test_reduce_sum_bit_exact(cuda, shape, dim):
    x = np.random.default_rng(16).standard_normal(shape).astype(np.float32)
    assert np.array_equal(host(nh.reduce_sum(dev(x, cuda), dim)), ref.reduce_sum(x, dim))


def test_index_to_i32(cuda):
    i16 = np.array([0, 1, -1, -32768, 12345], np.int16)
    assert host(nh.index_to_i32(dev(i16, cuda))).tolist() == ref.index_to_i32(i16).tolist()
    i64 = np.array([3, 2 ** 32 + 7, -2], np.int64)
    assert host(nh.index_to_i32(dev(i64, cuda))).tolist() == [3, 7, -2]
