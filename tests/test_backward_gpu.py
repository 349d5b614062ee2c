"""GPU parity for the backward ops (nova.sce_backward, the fused SCE forward +
backward, nova.layer_norm_backward, nova.linear_backward, nova.matmul_backward)
through libnova_hip's C ABI against the CPU oracle on identical seeded
inputs.  Full size for the config-5 reductions, sampled outputs for the
config-3 scale GEMMs, plus the edge cases the kernels branch on: ragged and
unaligned widths, strided rows, transposed output views, empty batches,
out-of-range labels.

Bars: sce_backward bit-exact (the same two f32 operations per element);
the fused SCE gradient bit-exact against this library's own softmax fed to
sce_backward and f32 rtol 1e-4 against the oracle; LayerNorm backward f32
rtol 1e-4 with atol 1e-4 * max|c| (the row and column sums are reordered);
f32 GEMMs bit-exact; bf16 in / f32 accumulate rtol 2e-2, atol 1e-2; column
sums bit-exact on integer-valued data, f32 tolerance otherwise."""
import numpy as np
import pytest

import nova_cpu_ref as ref
import nova_hip as nh
import nova_seed as S
from conftest import assert_close_f32, assert_close_lp

pytestmark = pytest.mark.gpu


def dev(a, cuda):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def to_dev(a, dt, cuda):
    import torch
    if dt == S.F32:
        return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    t = torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(cuda)
    return t.view(torch.bfloat16 if dt == S.BF16 else torch.float16)


def sce_inputs(R, C, seed):
    x = S.normal((R, C), seed, 0, 2)
    t = S.labels(R, C, seed, offset=x.size)
    return x, t


# ----------------------------------------------------------- SCE backward --

@pytest.mark.parametrize("R,C", [(1, 1), (3, 5), (37, 1001), (64, 32000), (5, 2049), (130, 4096)])
def test_sce_backward_bit_exact(cuda, R, C):
    x, t = sce_inputs(R, C, 41)
    sm, _, _ = ref.sce(x, t, softmax=True)
    want = ref.sce_backward(sm, t)
    got = nh.sce_backward(dev(sm, cuda), dev(t, cuda)).cpu().numpy()
    assert np.array_equal(got, want)


def test_sce_backward_strided_and_misaligned(cuda):
    x, t = sce_inputs(9, 1203, 42)
    sm, _, _ = ref.sce(x, t, softmax=True)
    wide = np.zeros((9, 1210), np.float32)
    wide[:, 3:1206] = sm
    d = dev(wide, cuda)[:, 3:1206]  # offset 3 floats: not 16-byte aligned
    got = nh.sce_backward(d, dev(t, cuda)).cpu().numpy()
    assert np.array_equal(got, ref.sce_backward(sm, t))


def test_sce_backward_out_of_range_label_gives_nan_row(cuda):
    sm = np.full((4, 10), 0.1, np.float32)
    t = np.array([0, 10, 3, -1], np.int32)
    got = nh.sce_backward(dev(sm, cuda), dev(t, cuda)).cpu().numpy()
    assert np.isnan(got[1]).all() and np.isnan(got[3]).all()
    ok = ref.sce_backward(sm[[0, 2]], t[[0, 2]])
    # rows 0 and 2 of a 4-row batch scale by 1/4, not 1/2
    assert np.allclose(got[[0, 2]], ok * 0.5, rtol=1e-6)


def test_sce_backward_c5_full_size(cuda):
    inp = S.config_inputs("c5_sce")
    x, t = inp["logits"], inp["labels"]
    sm, _, _ = ref.sce(x, t, softmax=True)
    got = nh.sce_backward(dev(sm, cuda), dev(t, cuda)).cpu().numpy()
    assert np.array_equal(got, ref.sce_backward(sm, t))


# ----------------------------------------------- fused SCE forward+backward --

@pytest.mark.parametrize("R,C", [(2, 3), (37, 1001), (64, 32000), (17, 5000), (3, 65537)])
def test_sce_fwd_bwd_matches_two_step_and_oracle(cuda, R, C):
    x, t = sce_inputs(R, C, 43)
    xd, td = dev(x, cuda), dev(t, cuda)
    loss, grad = nh.sce_fwd_bwd(xd, td)
    sm_gpu, loss2 = nh.sce(xd, td, softmax=True)
    two_step = nh.sce_backward(sm_gpu, td)
    assert np.array_equal(grad.cpu().numpy(), two_step.cpu().numpy())
    assert np.array_equal(loss.cpu().numpy(), loss2.cpu().numpy())
    sm, loss_ref, _ = ref.sce(x, t, softmax=True)
    assert_close_f32(grad.cpu().numpy(), ref.sce_backward(sm, t), f"fused grad {R}x{C}")
    assert_close_f32(loss.cpu().numpy(), loss_ref, "fused loss")


def test_sce_fwd_bwd_c5_full_size(cuda):
    inp = S.config_inputs("c5_sce")
    x, t = inp["logits"], inp["labels"]
    loss, grad = nh.sce_fwd_bwd(dev(x, cuda), dev(t, cuda))
    sm, loss_ref, _ = ref.sce(x, t, softmax=True)
    assert_close_f32(grad.cpu().numpy(), ref.sce_backward(sm, t), "c5 fused grad")
    assert_close_f32(loss.cpu().numpy(), loss_ref, "c5 fused loss")


# ------------------------------------------------------ LayerNorm backward --

def ln_bwd_inputs(R, D, seed):
    x = S.normal((R, D), seed)
    g = (1 + S.normal((D,), seed, 0, 0.1, offset=R * D)).astype(np.float32)
    gy = S.normal((R, D), seed, offset=R * D + D)
    _, Sm, rs = ref.layer_norm(x, g, np.zeros(D, np.float32))
    return gy, x, g, Sm, rs


def check_ln_bwd(gy, x, g, Sm, rs, cuda, what):
    dx_ref, dg_ref, db_ref = ref.layer_norm_backward(gy, x, g, Sm, rs)
    dx, dg, db = nh.layer_norm_backward(dev(gy, cuda), dev(x, cuda), dev(g, cuda), dev(Sm, cuda),
                                        dev(rs, cuda))
    assert_close_f32(dx.cpu().numpy(), dx_ref, what + " dx")
    assert_close_f32(dg.cpu().numpy(), dg_ref, what + " dgamma")
    assert_close_f32(db.cpu().numpy(), db_ref, what + " dbeta")
    return dx, dg, db


@pytest.mark.parametrize("R,D", [(1, 4), (3, 3), (5, 64), (7, 1000), (33, 1024), (9, 4096),
                                 (4, 5000), (2, 8192), (130, 257), (1001, 1024),
                                 (301, 4096), (600, 2048)])
def test_layer_norm_backward_shapes(cuda, R, D):
    check_ln_bwd(*ln_bwd_inputs(R, D, 51), cuda, f"ln_bwd {R}x{D}")


def test_layer_norm_backward_deterministic_and_optional_outputs(cuda):
    gy, x, g, Sm, rs = ln_bwd_inputs(300, 4096, 52)
    args = [dev(a, cuda) for a in (gy, x, g, Sm, rs)]
    a1 = nh.layer_norm_backward(*args)
    a2 = nh.layer_norm_backward(*args)
    for u, v in zip(a1, a2):
        assert np.array_equal(u.cpu().numpy(), v.cpu().numpy())
    dx, dg, db = nh.layer_norm_backward(*args, want=(False, True, False))
    assert dx is None and db is None
    assert np.array_equal(dg.cpu().numpy(), a1[1].cpu().numpy())
    dx, dg, db = nh.layer_norm_backward(*args, want=(True, False, False))
    assert np.array_equal(dx.cpu().numpy(), a1[0].cpu().numpy())


def test_layer_norm_backward_integer_dbeta_exact(cuda):
    gy, x, g, Sm, rs = ln_bwd_inputs(2000, 1024, 53)
    gy = np.round(gy * 4).astype(np.float32)  # small integers: every partial sum exact
    _, _, db = nh.layer_norm_backward(dev(gy, cuda), dev(x, cuda), dev(g, cuda), dev(Sm, cuda),
                                      dev(rs, cuda))
    assert np.array_equal(db.cpu().numpy(), gy.astype(np.int64).sum(0).astype(np.float32))


def test_layer_norm_backward_strided_rows(cuda):
    gy, x, g, Sm, rs = ln_bwd_inputs(16, 1024, 54)
    wide = np.zeros((16, 1100), np.float32)
    wide[:, 40:1064] = x
    xd = dev(wide, cuda)[:, 40:1064]
    dx, dg, db = nh.layer_norm_backward(dev(gy, cuda), xd, dev(g, cuda), dev(Sm, cuda),
                                        dev(rs, cuda))
    dx_ref, dg_ref, db_ref = ref.layer_norm_backward(gy, x, g, Sm, rs)
    assert_close_f32(dx.cpu().numpy(), dx_ref, "strided dx")
    assert_close_f32(dg.cpu().numpy(), dg_ref, "strided dgamma")


def test_layer_norm_backward_empty_batch(cuda):
    import torch
    z = torch.zeros((0, 64), dtype=torch.float32, device=cuda)
    g = torch.ones(64, dtype=torch.float32, device=cuda)
    s = torch.zeros(0, dtype=torch.float32, device=cuda)
    dx, dg, db = nh.layer_norm_backward(z, z, g, s, s)
    assert dx.shape == (0, 64)
    assert np.array_equal(dg.cpu().numpy(), np.zeros(64, np.float32))
    assert np.array_equal(db.cpu().numpy(), np.zeros(64, np.float32))


def test_layer_norm_backward_c5_full_size(cuda):
    inp = S.config_inputs("c5_ln")
    x, g = inp["x"], inp["gamma"]
    gy = S.normal(x.shape, 4, offset=7 * x.size)
    _, Sm, rs = ref.layer_norm(x, g, inp["beta"])
    check_ln_bwd(gy, x, g, Sm, rs, cuda, "c5 ln_bwd")


# --------------------------------------------------- linear / matmul backward --

@pytest.mark.parametrize("M,K,N", [(1, 1, 1), (7, 5, 3), (33, 31, 17), (64, 64, 64),
                                   (197, 64, 197), (96, 160, 200)])
def test_linear_backward_f32_bit_exact(cuda, M, K, N):
    x = S.uniform((M, K), 61)
    w = S.uniform((K, N), 61, offset=x.size)
    go = S.uniform((M, N), 61, offset=x.size + w.size)
    gi, gw, gb = nh.linear_backward(dev(go, cuda), dev(x, cuda), dev(w, cuda))
    gi_ref, gw_ref, gb_ref = ref.linear_backward(go, x, w)
    assert np.array_equal(gi.cpu().numpy(), gi_ref)
    assert np.array_equal(gw.cpu().numpy(), gw_ref)
    assert_close_f32(gb.cpu().numpy(), gb_ref, "f32 grad_bias")


@pytest.mark.parametrize("M,K,N", [(7, 5, 3), (96, 160, 200), (256, 512, 256), (300, 200, 520),
                                   (6400, 64, 96)])
def test_linear_backward_bf16(cuda, M, K, N):
    dt = S.BF16
    x = S.normal((M, K), 62, dtype=dt)
    w = S.normal((K, N), 62, 0, 0.02, dtype=dt, offset=x.size)
    go = S.normal((M, N), 62, dtype=dt, offset=x.size + w.size)
    gi, gw, gb = nh.linear_backward(to_dev(go, dt, cuda), to_dev(x, dt, cuda), to_dev(w, dt, cuda))
    gi_ref, gw_ref, gb_ref = ref.linear_backward(go, x, w, dt=dt)
    assert_close_lp(gi.cpu().numpy(), gi_ref, "bf16 grad_input")
    assert_close_lp(gw.cpu().numpy(), gw_ref, "bf16 grad_weight")
    assert_close_f32(gb.cpu().numpy(), gb_ref, "bf16 grad_bias")


def test_linear_backward_integer_bias_exact_and_transposed_outputs(cuda):
    """Weight as a transposed view of a row-major [N, K] tensor (the C3
    layout) and grad_weight written into a transposed view of a row-major
    [N, K] buffer; grad_bias on integer-valued data is exact."""
    import torch
    M, K, N = 300, 256, 520
    x = S.uniform((M, K), 63)
    W = S.uniform((N, K), 63, offset=x.size)                  # row-major [N, K]
    go = np.round(S.uniform((M, N), 63, offset=x.size + W.size) * 8).astype(np.float32)
    Wd = dev(W, cuda)
    gw_buf = torch.empty((N, K), dtype=torch.float32, device=cuda)
    gi, gw, gb = nh.linear_backward(dev(go, cuda), dev(x, cuda), Wd.t(), grad_weight=gw_buf.t())
    gi_ref, gw_ref, _ = ref.linear_backward(go, x, W.T)
    assert np.array_equal(gi.cpu().numpy(), gi_ref)
    assert np.array_equal(gw_buf.cpu().numpy(), gw_ref.T)
    assert np.array_equal(gb.cpu().numpy(), go.astype(np.int64).sum(0).astype(np.float32))


def test_matmul_backward_f32_and_bf16(cuda):
    M, K, N = 65, 130, 96
    A = S.uniform((M, K), 64)
    B = S.uniform((K, N), 64, offset=A.size)
    g = S.uniform((M, N), 64, offset=A.size + B.size)
    ga, gb = nh.matmul_backward(dev(g, cuda), dev(A, cuda), dev(B, cuda))
    ga_ref, gb_ref = ref.matmul_backward(g, A, B)
    assert np.array_equal(ga.cpu().numpy(), ga_ref)
    assert np.array_equal(gb.cpu().numpy(), gb_ref)
    dt = S.BF16
    Ab, Bb, gbits = (S.round_to(v, dt) for v in (A, B, g))
    ga, gb = nh.matmul_backward(to_dev(gbits, dt, cuda), to_dev(Ab, dt, cuda), to_dev(Bb, dt, cuda))
    ga_ref, gb_ref = ref.matmul_backward(gbits, Ab, Bb, dt=dt)
    assert_close_lp(ga.cpu().numpy(), ga_ref, "bf16 grad_a")
    assert_close_lp(gb.cpu().numpy(), gb_ref, "bf16 grad_b")


def sample_idx(M, N, count, seed):
    g = np.random.default_rng(seed)
    idx = np.stack([np.zeros(count, np.int64), g.integers(0, M, count), g.integers(0, N, count)], 1)
    corners = np.array([[0, i, j] for i in (0, M - 1) for j in (0, N - 1)], np.int64)
    return np.concatenate([corners, idx]).astype(np.int64)


def test_linear_backward_c3_scale(cuda):
    """Backward of config 3 (x bf16 [4096,4096], W bf16 [11008,4096] used
    transposed): grad_input [4096,4096] = go . W, grad_weight written as a
    transposed view of [11008,4096], grad_bias [11008]; sampled outputs."""
    import torch
    dt = S.BF16
    inp = S.config_inputs("c3")
    x, W = inp["x"], inp["W"]
    M, K, N = x.shape[0], x.shape[1], W.shape[0]
    go = S.normal((M, N), 2, 0, 1, dtype=dt, offset=99_000_000)
    Wd = to_dev(W, dt, cuda)
    gw_buf = torch.empty((N, K), dtype=torch.float32, device=cuda)
    gi, gw, gb = nh.linear_backward(to_dev(go, dt, cuda), to_dev(x, dt, cuda), Wd.t(),
                                    grad_weight=gw_buf.t())
    idx = sample_idx(M, K, 4096, 65)
    want = ref.gemm_sampled(go, W, idx, adt=dt, bdt=dt)
    got = gi.cpu().numpy()[idx[:, 1], idx[:, 2]]
    assert_close_lp(got, want, "c3 grad_input")
    idx = sample_idx(K, N, 4096, 66)
    want = ref.gemm_sampled(x.T, go, idx, adt=dt, bdt=dt)
    got = gw_buf.cpu().numpy()[idx[:, 2], idx[:, 1]]
    assert_close_lp(got, want, "c3 grad_weight")
    assert_close_f32(gb.cpu().numpy(), ref.col_sum(go, dt), "c3 grad_bias")
