"""GPU parity for nova.layer_norm and nova.sce (libnova_hip through its C
ABI) against the CPU oracle on identical seeded inputs, full size for
config 5, plus the edge cases: ragged / unaligned widths, strided rows,
single rows, empty batches, out-of-range labels.  Bar: f32, rtol 1e-4 with
a normwise atol of 1e-4 * max|c|."""
import math

import numpy as np
import pytest

import nova_cpu_ref as ref
import nova_hip as nh
import nova_seed as S
from conftest import assert_close_f32

pytestmark = pytest.mark.gpu


def dev(a, cuda):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def check_ln(x, g, b, cuda, what):
    y_ref, s_ref, r_ref = ref.layer_norm(x, g, b)
    y, s, r = nh.layer_norm(dev(x, cuda), dev(g, cuda), dev(b, cuda))
    assert_close_f32(y.cpu().numpy(), y_ref, what + " y")
    assert_close_f32(s.cpu().numpy(), s_ref, what + " mean_sum")
    assert_close_f32(r.cpu().numpy(), r_ref, what + " rstd")


@pytest.mark.parametrize("rows,D", [(1, 1), (3, 3), (5, 64), (7, 1000), (33, 1024),
                                    (9, 4096), (4, 5000), (2, 9000), (130, 257)])
def test_layer_norm_shapes(cuda, rows, D):
    x = S.normal((rows, D), 31)
    g = (1 + S.normal((D,), 31, 0, 0.1, offset=rows * D)).astype(np.float32)
    b = S.normal((D,), 31, 0, 0.1, offset=rows * D + D)
    check_ln(x, g, b, cuda, f"ln {rows}x{D}")


def test_layer_norm_strided_rows(cuda):
    import torch
    wide = S.normal((16, 1200), 32)
    x = dev(wide, cuda)[:, 100:1124]  # row stride 1200, offset 100
    g = dev(np.ones(1024, np.float32), cuda)
    b = dev(np.zeros(1024, np.float32), cuda)
    y, s, r = nh.layer_norm(x, g, b)
    y_ref, s_ref, r_ref = ref.layer_norm(wide[:, 100:1124], np.ones(1024, np.float32),
                                         np.zeros(1024, np.float32))
    assert_close_f32(y.cpu().numpy(), y_ref, "strided y")
    assert_close_f32(r.cpu().numpy(), r_ref, "strided rstd")


def test_layer_norm_constant_rows_give_beta(cuda):
    x = np.full((8, 4096), 3.0, np.float32)
    g = S.normal((4096,), 33)
    b = S.normal((4096,), 33, offset=4096)
    y, s, r = nh.layer_norm(dev(x, cuda), dev(g, cuda), dev(b, cuda))
    assert np.array_equal(y.cpu().numpy(), np.broadcast_to(b, (8, 4096)))
    assert np.allclose(r.cpu().numpy(), 1 / math.sqrt(1e-5), rtol=1e-6)


def test_c5_layer_norm_full_size(cuda):
    inp = S.config_inputs("c5_ln")
    check_ln(inp["x"], inp["gamma"], inp["beta"], cuda, "c5 ln")


def check_sce(x, t, cuda, what, softmax=False):
    sm_ref, loss_ref, _ = ref.sce(x, t, softmax=softmax)
    sm, loss = nh.sce(dev(x, cuda), dev(t, cuda), softmax=softmax)
    assert_close_f32(loss.cpu().numpy(), loss_ref, what + " loss")
    if softmax:
        assert_close_f32(sm.cpu().numpy(), sm_ref, what + " softmax")


@pytest.mark.parametrize("rows,C", [(1, 1), (1, 3), (5, 10), (64, 1000), (65, 2049),
                                    (130, 4096), (7, 32000), (200, 333)])
def test_sce_shapes(cuda, rows, C):
    x = S.normal((rows, C), 41, 0, 2)
    t = S.labels(rows, C, 41, offset=2 * rows * C)
    check_sce(x, t, cuda, f"sce {rows}x{C}", softmax=(rows * C <= 1 << 20))


def test_sce_closed_forms_on_gpu(cuda):
    x = np.zeros((100, 5000), np.float32)
    t = (np.arange(100) * 37 % 5000).astype(np.int32)
    _, loss = nh.sce(dev(x, cuda), dev(t, cuda))
    assert abs(float(loss.cpu()[0]) - math.log(5000)) < 1e-4 * math.log(5000)
    x[np.arange(100), t] = 80.0
    _, loss = nh.sce(dev(x, cuda), dev(t, cuda))
    assert 0 <= float(loss.cpu()[0]) < 1e-5


def test_sce_repeat_calls_identical(cuda):
    """Back-to-back calls (and a smaller second call) give identical,
    correct results."""
    x = S.normal((300, 777), 42, 0, 2)
    t = S.labels(300, 777, 42, offset=2 * 300 * 777)
    X, T = dev(x, cuda), dev(t, cuda)
    _, l1 = nh.sce(X, T)
    _, l2 = nh.sce(X, T)
    _, l3 = nh.sce(X[:17], T[:17])
    _, ref17, _ = ref.sce(x[:17], t[:17])
    assert float(l1.cpu()[0]) == float(l2.cpu()[0])
    assert_close_f32(l3.cpu().numpy(), ref17, "second, smaller call")


def _chunk_mean_f32(v):
    """The mean in the order of lowerFullReduceMeanToSCF
    (NovaToLinalg.cpp:1974-2126): 64 contiguous chunks of ceil(R/64) rows,
    each summed sequentially in f32, the chunk sums sequentially, then / R."""
    R = len(v)
    per = (R + 63) // 64
    total = np.float32(0)
    for c in range(64):
        p = np.float32(0)
        for r in range(c * per, min(c * per + per, R)):
            p = np.float32(p + v[r])
        total = np.float32(total + p)
    return np.float32(total / np.float32(R))


@pytest.mark.parametrize("rows,C", [(5, 2052), (1000, 2052), (4173, 2052), (4288, 2052),
                                    (64, 32000)])
def test_sce_mean_is_the_chunked_order_of_its_row_losses(cuda, rows, C):
    """Each row's loss, taken from a one-row call (whose mean is the row loss
    itself), summed on the host in the reference's 64-chunk order, gives the
    batched call's loss bit for bit: the device mean keeps that order
    exactly, for chunks of one row, 16, 66 and 67 rows (more than one
    float4 batch; chunk starts 0-3 rows off a 16-byte boundary, so every
    length of the single-row head and tail) and 64 chunks of one row each.
    The fused forward+backward gives the same loss bits."""
    import torch
    x = S.normal((rows, C), 47, 0, 2)
    t = S.labels(rows, C, 47, offset=rows * C)
    X, T = dev(x, cuda), dev(t, cuda)
    single = np.empty(rows, np.float32)
    for r in range(rows):
        _, lr = nh.sce(X[r:r + 1], T[r:r + 1])
        single[r] = lr.cpu().numpy()[0]
    _, loss = nh.sce(X, T)
    want = _chunk_mean_f32(single)
    got = loss.cpu().numpy()[0]
    assert got.view(np.uint32) == want.view(np.uint32), (got, want)
    lf, _ = nh.sce_fwd_bwd(X, T)
    assert torch.equal(lf, loss)
    _, loss_ref, _ = ref.sce(x, t)
    assert_close_f32(loss.cpu().numpy(), loss_ref, f"sce {rows}x{C}")


@pytest.mark.parametrize("C,pitch", [(32003, 32004), (50303, 50304), (4099, 4100)])
def test_sce_row_kernel_labels_in_every_part(cuda, C, pitch):
    """The on-chip row kernel takes x[label] from where the row sits: a
    thread's registers, the LDS part past 32768 classes, or thread 0's C % 4
    tail (rows padded to a 16-byte pitch, so the row kernel runs with
    C % 4 != 0).  Labels in each part, at their edges, and out of range:
    loss and fused gradient against the oracle, NaN for the bad label."""
    import torch
    labels = [0, 1, 4097, 8191 * 4 + 3, C - 1, C - 3, 4 * (C // 4) - 1, 32768, 40001]
    labels = [l for l in labels if l < C]
    rows = len(labels)
    x = S.normal((rows, C), 49, 0, 2)
    t = np.array(labels, np.int32)
    wide = np.zeros((rows, pitch), np.float32)
    wide[:, :C] = x
    X = dev(wide, cuda)[:, :C]
    T = dev(t, cuda)
    _, loss = nh.sce(X, T)
    sm_ref, loss_ref, _ = ref.sce(x, t, softmax=True)
    assert_close_f32(loss.cpu().numpy(), loss_ref, f"sce labels {C}")
    single = np.array([nh.sce(X[r:r + 1], T[r:r + 1])[1].cpu().numpy()[0] for r in range(rows)])
    for r in range(rows):
        _, lr, _ = ref.sce(x[r:r + 1], t[r:r + 1])
        assert_close_f32(single[r:r + 1], lr, f"row {r} label {labels[r]}")
    gpad = torch.zeros(rows, pitch, device=cuda)
    lf, _ = nh.sce_fwd_bwd(X, T, grad=gpad[:, :C])
    assert torch.equal(lf, loss)
    assert_close_f32(gpad[:, :C].cpu().numpy(), ref.sce_backward(sm_ref, t), "fused grad")
    bad = T.clone()
    bad[1] = C
    _, lb = nh.sce(X, bad)
    assert math.isnan(float(lb.cpu()[0]))


def test_sce_strided_rows(cuda):
    wide = S.normal((40, 600), 43, 0, 2)
    t = S.labels(40, 500, 43, offset=2 * 40 * 600)
    X = dev(wide, cuda)[:, 3:503]
    _, loss = nh.sce(X, dev(t, cuda))
    _, loss_ref, _ = ref.sce(wide[:, 3:503], t)
    assert_close_f32(loss.cpu().numpy(), loss_ref, "strided sce")


def test_sce_empty_batch_and_bad_label_give_nan(cuda):
    import torch
    x = torch.zeros(0, 10, device=cuda)
    t = torch.zeros(0, dtype=torch.int32, device=cuda)
    _, loss = nh.sce(x, t)
    assert math.isnan(float(loss.cpu()[0]))
    x = dev(S.normal((4, 10), 44), cuda)
    t = dev(np.array([1, 2, 10, 3], np.int32), cuda)
    _, loss = nh.sce(x, t)
    assert math.isnan(float(loss.cpu()[0]))


def test_c5_sce_full_size(cuda):
    inp = S.config_inputs("c5_sce")
    check_sce(inp["logits"], inp["labels"], cuda, "c5 sce")


@pytest.mark.parametrize("C", [40000, 50304, 32772, 51200, 51204, 65540])
def test_sce_streaming_rows_above_32k(cuda, C):
    """Rows of more than 32768 classes with 16-byte aligned rows (C % 4 == 0):
    up to 51200 classes the row kernel keeps the part of the row past its
    registers in LDS (the GPT step's vocab is 50304; 51200 fills both
    exactly), above that the chunked streaming path reads the row twice.
    Loss and softmax against the oracle, plus the fused gradient and
    sce_backward bit-identical to each other."""
    import torch
    rows = 24
    assert C % 4 == 0 and C > 32768
    x = S.normal((rows, C), 45, 0, 2)
    t = S.labels(rows, C, 45, offset=rows * C)
    t[0], t[1] = 0, C - 1                # the row ends
    check_sce(x, t, cuda, f"sce {rows}x{C}", softmax=True)
    sm_ref, loss_ref, _ = ref.sce(x, t, softmax=True)
    X, T = dev(x, cuda), dev(t, cuda)
    loss, grad = nh.sce_fwd_bwd(X, T)
    assert_close_f32(loss.cpu().numpy(), loss_ref, "fused loss")
    assert_close_f32(grad.cpu().numpy(), ref.sce_backward(sm_ref, t), "fused grad")
    sm, _ = nh.sce(X, T, softmax=True)
    g2 = nh.sce_backward(sm, T)
    assert torch.equal(grad, g2)
    # sce_backward from the oracle's softmax: the same two f32 operations
    g3 = nh.sce_backward(dev(sm_ref, cuda), T)
    assert np.array_equal(g3.cpu().numpy(), ref.sce_backward(sm_ref, t))


@pytest.mark.parametrize("mean", [1.0, 3.0])
def test_layer_norm_offset_data(cuda, mean):
    """x ~ N(mean, 1).  The reference's one-pass variance var = Q/D - mean^2
    (NovaToLinalgGeneric.cpp:2064-2113) cancels: Q/D ~ mean^2 + 1, so the
    rounding error of Q is amplified by (mean^2 + 1) in var.  The GPU sums Q
    in a different order from the oracle's sequential loop; at D = 4096 the
    two stay within the 1e-4 bar up to |mean| / sigma = 3 (error ~ 2e-5 at
    3, growing as mean^2)."""
    rows, D = 64, 4096
    x = (S.normal((rows, D), 34) + np.float32(mean)).astype(np.float32)
    g = (1 + S.normal((D,), 34, 0, 0.1, offset=rows * D)).astype(np.float32)
    b = S.normal((D,), 34, 0, 0.1, offset=rows * D + D)
    check_ln(x, g, b, cuda, f"ln N({mean}, 1)")


def test_sce_loss_only_entry_point(cuda):
    """_mlir_ciface_nova_hip_sce_loss_f32 (what a lowered module calls for a
    nova.sce with a dead softmax) gives sce_f32's loss."""
    import ctypes
    import torch
    x = S.normal((50, 3000), 46, 0, 2)
    t = S.labels(50, 3000, 46, offset=50 * 3000)
    X, T = dev(x, cuda), dev(t, cuda)
    _, want = nh.sce(X, T)
    loss = torch.empty(1, device=cuda)
    nh._bind_stream()
    nh.check(nh.lib()._mlir_ciface_nova_hip_sce_loss_f32(
        nh.ref(nh.memref_of(X)), nh.ref(nh.memref_of(T)), nh.ref(nh.memref_of(loss))))
    assert torch.equal(loss, want)
