"""GPU parity for the GEMM family (libnova_hip through its C ABI) against the
CPU oracle on identical seeded inputs.  Small shapes are compared in full,
the BASELINE configs at full size on a deterministic sample of outputs.
Bars: f32 bit-exact (same arithmetic as the reference CPU pipeline);
bf16/f16 with f32 accumulate: |g-c| <= 2e-2|c| + 1e-2."""
import numpy as np
import pytest

import nova_cpu_ref as ref
import nova_hip as nh
import nova_seed as S
from conftest import assert_close_f32, assert_close_lp

pytestmark = pytest.mark.gpu


def to_dev(a, dt, dev):
    import torch
    if dt == S.F32:
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    t = torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)
    return t.view(torch.bfloat16 if dt == S.BF16 else torch.float16)


def lp_inputs(shape_a, shape_b, dt, seed):
    na = int(np.prod(shape_a))
    return (S.uniform(shape_a, seed, dtype=dt), S.uniform(shape_b, seed, dtype=dt, offset=na))


def sample_idx(batch, M, N, count, seed):
    g = np.random.default_rng(seed)
    idx = np.stack([g.integers(0, batch, count), g.integers(0, M, count),
                    g.integers(0, N, count)], 1).astype(np.int64)
    # always include the corners, where edge-tile bugs live
    corners = np.array([[b, i, j] for b in (0, batch - 1) for i in (0, M - 1) for j in (0, N - 1)],
                       np.int64)
    return np.concatenate([corners, idx])


def view_as(a_host, layout, dev, dt):
    """Device tensor with logical shape of a_host ([..., R, C]); layout 'T'
    stores it transposed (unit stride on the second-to-last dim)."""
    if layout == "N":
        return to_dev(a_host, dt, dev)
    t = to_dev(np.ascontiguousarray(np.swapaxes(a_host, -1, -2)), dt, dev)
    return t.transpose(-1, -2)


SMALL = [(1, 1, 1, 1), (1, 7, 5, 3), (2, 33, 31, 17), (1, 64, 64, 64), (3, 65, 63, 72),
         (2, 128, 96, 8), (1, 197, 197, 64), (2, 197, 64, 197), (1, 255, 257, 129),
         (4, 16, 16, 0)]


@pytest.mark.parametrize("dt", [S.BF16, S.F16])
@pytest.mark.parametrize("layout", ["NN", "NT", "TN", "TT"])
@pytest.mark.parametrize("shape", SMALL)
def test_gemm_small_shapes(cuda, dt, layout, shape):
    batch, M, N, K = shape
    a, b = lp_inputs((batch, M, K), (batch, K, N), dt, seed=11)
    want = ref.gemm(a, b, adt=dt, bdt=dt)
    A = view_as(a, layout[0], cuda, dt)
    B = view_as(b, layout[1], cuda, dt)
    got = nh.gemm(A, B).cpu().numpy()
    assert_close_lp(got, want, f"gemm {shape} {layout} dt={dt}")


def test_gemm_mfma_lane_layout_exact(cuda):
    """Integer-grid inputs make bf16 MFMA exact, so any misplaced lane,
    row or k-chunk shows up as a wrong integer."""
    g = np.random.default_rng(12)
    for (batch, M, N, K) in [(1, 64, 64, 64), (2, 100, 72, 136), (64, 256, 256, 64)]:
        af = g.integers(-4, 5, (batch, M, K)).astype(np.float32)
        bf = g.integers(-4, 5, (batch, K, N)).astype(np.float32)
        a, b = S.round_to(af, S.BF16), S.round_to(bf, S.BF16)
        want = np.einsum("bmk,bkn->bmn", af.astype(np.int64), bf.astype(np.int64))
        got = nh.gemm(to_dev(a, S.BF16, cuda), to_dev(b, S.BF16, cuda)).cpu().numpy()
        assert np.array_equal(got, want.astype(np.float32)), (batch, M, N, K)


@pytest.mark.parametrize("dt", [S.BF16, S.F16])
@pytest.mark.parametrize("layout", ["NN", "NT", "TN", "TT"])
def test_gemm_dma_path_exact(cuda, dt, layout):
    """Whole 256x256 tiles, K % 64 == 0 and 128..255 tiles select the
    one-tile-per-workgroup LDS-DMA kernel (transposing LDS reads for
    M/N-contiguous operands).  Integer grids make the result exact, so any
    lane / swizzle slip is caught."""
    g = np.random.default_rng(19)
    batch, M, N, K = 32, 512, 512, 384
    af = g.integers(-4, 5, (batch, M, K)).astype(np.float32)
    bf = g.integers(-4, 5, (batch, K, N)).astype(np.float32)
    a, b = S.round_to(af, dt), S.round_to(bf, dt)
    want = np.matmul(af.astype(np.float64), bf.astype(np.float64)).astype(np.float32)
    A = view_as(a, layout[0], cuda, dt)
    B = view_as(b, layout[1], cuda, dt)
    got = nh.gemm(A, B).cpu().numpy()
    assert np.array_equal(got, want), (layout, float(np.abs(got - want).max()))


@pytest.mark.parametrize("dt,layout,shape", [
    (S.BF16, "NN", (17, 1024, 1024, 128)),   # 272 tiles: 16 workgroups take two
    (S.BF16, "NT", (9, 1536, 1280, 192)),    # 270 tiles, three K steps
    (S.BF16, "TN", (17, 1024, 1024, 128)),
    (S.BF16, "TT", (9, 1536, 1280, 192)),
    (S.F16, "NN", (3, 2816, 2304, 320)),     # 297 tiles, five K steps
    (S.F16, "TT", (17, 1024, 1024, 128)),
])
def test_gemm_persistent_path_exact(cuda, dt, layout, shape):
    """A full round of 256x256 tiles or more (one workgroup per CU), K % 64
    == 0, K >= 128 and no epilogue op select the persistent LDS-DMA kernel:
    each workgroup computes several tiles and prefetches the next tile's
    first K steps during an epilogue.  A last, partial round leaves some
    workgroups one tile fewer.  Integer grids make the result exact."""
    g = np.random.default_rng(23)
    batch, M, N, K = shape
    af = g.integers(-4, 5, (batch, M, K)).astype(np.float32)
    bf = g.integers(-4, 5, (batch, K, N)).astype(np.float32)
    a, b = S.round_to(af, dt), S.round_to(bf, dt)
    want = np.matmul(af.astype(np.float64), bf.astype(np.float64)).astype(np.float32)
    A = view_as(a, layout[0], cuda, dt)
    B = view_as(b, layout[1], cuda, dt)
    got = nh.gemm(A, B).cpu().numpy()
    assert np.array_equal(got, want), (layout, shape, float(np.abs(got - want).max()))


@pytest.mark.parametrize("out", ["bf16", "f16"])
def test_gemm_persistent_path_16bit_out(cuda, out):
    """The persistent kernel's 16-bit epilogue: integer sums up to 2048 are
    exact in bf16 only up to 256, so compare against the RNE rounding of the
    exact f32 result."""
    import torch
    g = np.random.default_rng(29)
    batch, M, N, K = 17, 1024, 1024, 128
    af = g.integers(-4, 5, (batch, M, K)).astype(np.float32)
    bf = g.integers(-4, 5, (batch, K, N)).astype(np.float32)
    a, b = S.round_to(af, S.BF16), S.round_to(bf, S.BF16)
    exact = np.matmul(af.astype(np.float64), bf.astype(np.float64)).astype(np.float32)
    odt = torch.bfloat16 if out == "bf16" else torch.float16
    got = nh.gemm(to_dev(a, S.BF16, cuda), to_dev(b, S.BF16, cuda), out_dtype=odt)
    want = torch.from_numpy(exact).to(odt)
    assert torch.equal(got.cpu(), want), out


@pytest.mark.parametrize("layout", ["NN", "NT", "TN"])
def test_gemm_big_tile_path(cuda, layout):
    """>= 256 macro-tiles of 256x256 selects the big-tile kernel; M and N
    are not multiples of 256, exercising its masked edges."""
    batch, M, N, K = 64, 500, 504, 136
    a, b = lp_inputs((batch, M, K), (batch, K, N), S.BF16, seed=13)
    A = view_as(a, layout[0], cuda, S.BF16)
    B = view_as(b, layout[1], cuda, S.BF16)
    got = nh.gemm(A, B).cpu().numpy()
    idx = sample_idx(batch, M, N, 20000, 14)
    want = ref.gemm_sampled(a, b, idx, adt=S.BF16, bdt=S.BF16)
    assert_close_lp(got[idx[:, 0], idx[:, 1], idx[:, 2]], want, f"big tile {layout}")


def test_gemm_broadcast_rank2_operand(cuda):
    """NovaToLinalg.cpp:992-1025: a rank-2 operand broadcasts over the batch."""
    a, b = lp_inputs((3, 40, 48), (48, 24), S.F16, seed=15)
    want = ref.gemm(a, b, adt=S.F16, bdt=S.F16)
    A = to_dev(a, S.F16, cuda)
    B = to_dev(b, S.F16, cuda).unsqueeze(0).expand(3, 48, 24)
    got = nh.gemm(A, B).cpu().numpy()
    assert_close_lp(got, want, "broadcast")


@pytest.mark.parametrize("out_dt", [S.F32, S.BF16, S.F16])
@pytest.mark.parametrize("epi", [nh.EPI_BIAS, nh.EPI_BIAS_GELU, nh.EPI_GELU])
def test_gemm_epilogues(cuda, out_dt, epi):
    import torch
    M, N, K = 70, 90, 200
    x = S.normal((M, K), 21, dtype=S.BF16)
    w = S.normal((N, K), 21, 0.0, 0.05, dtype=S.BF16, offset=M * K)
    bias = S.normal((N,), 21, 0.0, 0.5, dtype=S.BF16, offset=M * K + N * K)
    want = ref.gemm(x, w.T, adt=S.BF16, bdt=S.BF16, bias=bias, biasdt=S.BF16, epilogue=epi,
                    cdt=out_dt)
    want = S.widen(want, out_dt) if out_dt != S.F32 else want
    od = {S.F32: torch.float32, S.BF16: torch.bfloat16, S.F16: torch.float16}[out_dt]
    X = to_dev(x, S.BF16, cuda)
    W = to_dev(w, S.BF16, cuda)
    Bb = to_dev(bias, S.BF16, cuda)
    has_bias = epi in (nh.EPI_BIAS, nh.EPI_BIAS_GELU)
    got = nh.gemm(X, W.t(), bias=Bb if has_bias else None, epilogue=epi, out_dtype=od)
    assert_close_lp(got.float().cpu().numpy(), want[0], f"epilogue {epi} out {out_dt}")


def test_c1_matmul_f32_bit_exact(cuda):
    """Config 1: nova.matmul f32 A[256,256] @ B[256,256], U[-1,1] seed 0.
    Same arithmetic as the CPU pipeline -> identical bits."""
    inp = S.config_inputs("c1")
    want = ref.gemm(inp["A"], inp["B"])[0]
    import ctypes
    import torch
    A = to_dev(inp["A"], S.F32, cuda)
    B = to_dev(inp["B"], S.F32, cuda)
    C = torch.empty(256, 256, device=cuda)
    dA, dB, dC = nh.memref_of(A), nh.memref_of(B), nh.memref_of(C)
    nh._bind_stream()
    nh.check(nh.lib()._mlir_ciface_nova_hip_matmul_f32(nh.ref(dA), nh.ref(dB), nh.ref(dC)))
    got = C.cpu().numpy()
    assert np.array_equal(got, want), float(np.abs(got - want).max())


def test_f32_gemm_layouts_bias_gelu_bit_exact(cuda):
    g = np.random.default_rng(16)
    a = g.uniform(-1, 1, (2, 37, 70)).astype(np.float32)
    b = g.uniform(-1, 1, (2, 70, 45)).astype(np.float32)
    bias = g.uniform(-1, 1, 45).astype(np.float32)
    want = ref.gemm(a, b, bias=bias, epilogue=ref.EPI_BIAS)
    for layout in ("NN", "TN", "NT", "TT"):
        A = view_as(a, layout[0], cuda, S.F32)
        B = view_as(b, layout[1], cuda, S.F32)
        got = nh.gemm(A, B, bias=to_dev(bias, S.F32, cuda), epilogue=nh.EPI_BIAS).cpu().numpy()
        assert np.array_equal(got, want), layout
    # GELU goes through tanhf on both sides: within the f32 bar, not bitwise.
    want_g = ref.gemm(a, b, bias=bias, epilogue=ref.EPI_BIAS_GELU)
    got_g = nh.gemm(to_dev(a, S.F32, cuda), to_dev(b, S.F32, cuda), bias=to_dev(bias, S.F32, cuda),
                    epilogue=nh.EPI_BIAS_GELU).cpu().numpy()
    assert_close_f32(got_g, want_g, "f32 bias+gelu")


# The exact f32 GEMM's vector forms (16-byte aligned rows): rows x columns
# per thread and the relative rate the library's choice weighs them by.
VEC_FORMS = [(8, 8, 1.0), (4, 8, 0.95), (4, 6, 0.93), (4, 4, 0.8), (4, 2, 0.6)]


def vec_form(batch, M, N, cus):
    """The form the library picks: least (waves of two tiles per CU) x tile
    area / rate; the 16x16 tiny form (index 5, rate 0.5) only when the 64x32
    form's tiles are fewer than the CUs."""
    best, best_cost = None, None
    for f, (rm, cn, rate) in enumerate(VEC_FORMS):
        tm, tn = 16 * rm, 16 * cn
        tiles = batch * -(-M // tm) * -(-N // tn)
        cost = -(-tiles // (2 * cus)) * tm * tn / rate
        if best is None or cost < best_cost:
            best, best_cost = f, cost
    if batch * -(-M // 64) * -(-N // 32) < cus:
        tiny = batch * -(-M // 16) * -(-N // 16)
        if -(-tiny // (2 * cus)) * 256 / 0.5 < best_cost:
            return 5
    return best


# One problem per form (on a 256-CU part), M and N off the tile edges, K
# ending in a partial stage (stages of 16, 16, 32, 64, 64 and 128 k).
VEC_CASES = [(0, (1, 2044, 4092, 37)), (1, (1, 2044, 2044, 70)), (2, (1, 1020, 3070, 101)),
             (3, (1, 1000, 1100, 130)), (4, (2, 500, 777, 130)), (5, (3, 100, 200, 200))]
VEC_IDS = ["128x128", "64x128", "64x96", "64x64", "64x32", "16x16"]


def _vec_case(cuda, form, shape):
    import torch
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count
    if vec_form(*shape[:3], cus) != form:
        pytest.skip(f"a {cus}-CU device picks another form for {shape}")
    return shape


@pytest.mark.parametrize("layout", ["NN", "NT", "TN", "TT"])
@pytest.mark.parametrize("bias_dt", [None, S.F32, S.BF16])
@pytest.mark.parametrize("form,shape", VEC_CASES, ids=VEC_IDS)
def test_f32_gemm_vector_forms_bit_exact(cuda, layout, bias_dt, form, shape):
    """The exact f32 GEMM's vector forms (aligned rows; 128x128, 64x128, 64x96,
    64x64, 64x32 and 16x16 tiles) against the oracle's sequential arithmetic, bit for bit,
    on 65,536 sampled outputs and the corners, in all four layouts, with no
    bias, an f32 bias and a bf16 bias."""
    import torch
    batch, M, N, K = _vec_case(cuda, form, shape)
    g = np.random.default_rng(57 + form)
    a = g.uniform(-1, 1, (batch, M, K)).astype(np.float32)
    b = g.uniform(-1, 1, (batch, K, N)).astype(np.float32)
    bias = g.uniform(-1, 1, N).astype(np.float32) if bias_dt is not None else None
    if bias_dt == S.BF16:
        bias = S.round_to(bias, S.BF16)
    A = view_as(a, layout[0], cuda, S.F32)
    B = view_as(b, layout[1], cuda, S.F32)
    epi = nh.EPI_BIAS if bias is not None else nh.EPI_NONE
    Bs = to_dev(bias, bias_dt, cuda) if bias is not None else None
    got = nh.gemm(A, B, bias=Bs, epilogue=epi)
    if batch == 1:
        got = got.reshape(1, M, N)
    idx = sample_idx(batch, M, N, 65536, 58)
    it = torch.from_numpy(idx).to(cuda)
    gs = got[it[:, 0], it[:, 1], it[:, 2]].cpu().numpy()
    want = ref.gemm_sampled(a, b, idx, bias=bias, biasdt=bias_dt, epilogue=ref.EPI_BIAS if bias is not None else ref.EPI_NONE)
    assert np.array_equal(gs, want), (layout, float(np.abs(gs - want).max()))


@pytest.mark.parametrize("form,shape", VEC_CASES, ids=VEC_IDS)
def test_f32_gemm_vector_forms_padded_rows_and_gelu(cuda, form, shape):
    """The vector forms with K = 101 and A's rows padded to 104 floats (the
    last 16-byte load of a row reaches past K), with a bias and GELU
    epilogue: bias-only outputs bit-exact, GELU within the f32 bar (tanhf on
    both sides)."""
    import torch
    batch, M, N, _ = _vec_case(cuda, form, shape)
    K = 101
    g = np.random.default_rng(59 + form)
    a = g.uniform(-1, 1, (batch, M, K)).astype(np.float32)
    b = g.uniform(-1, 1, (batch, K, N)).astype(np.float32)
    bias = g.uniform(-1, 1, N).astype(np.float32)
    store = torch.zeros(batch, M, 104, device=cuda)
    store[:, :, :K] = torch.from_numpy(a).to(cuda)
    A = store[:, :, :K]
    B = to_dev(b, S.F32, cuda)
    idx = sample_idx(batch, M, N, 65536, 60)
    it = torch.from_numpy(idx).to(cuda)
    got = nh.gemm(A, B, bias=to_dev(bias, S.F32, cuda), epilogue=nh.EPI_BIAS)
    want = ref.gemm_sampled(a, b, idx, bias=bias, biasdt=S.F32, epilogue=ref.EPI_BIAS)
    gs = got[it[:, 0], it[:, 1], it[:, 2]].cpu().numpy()
    assert np.array_equal(gs, want), float(np.abs(gs - want).max())
    got = nh.gemm(A, B, bias=to_dev(bias, S.F32, cuda), epilogue=nh.EPI_BIAS_GELU)
    want = ref.gemm_sampled(a, b, idx, bias=bias, biasdt=S.F32, epilogue=ref.EPI_BIAS_GELU)
    assert_close_f32(got[it[:, 0], it[:, 1], it[:, 2]].cpu().numpy(), want, "vector-form gelu")


def test_f32_gemm_gpt_step_input_gradient_shape(cuda):
    """The LM-head input-gradient shape of the GPT step at reduced K:
    [8192, K] x [K, 384] with B a transposed view (the 64x96 form, two tiles
    per CU), bit-exact against the oracle on sampled outputs."""
    import torch
    M, N, K = 8192, 384, 200
    g = np.random.default_rng(61)
    a = g.uniform(-1, 1, (1, M, K)).astype(np.float32)
    b = g.uniform(-1, 1, (1, K, N)).astype(np.float32)
    A = to_dev(a[0], S.F32, cuda)
    B = view_as(b[0], "T", cuda, S.F32)
    got = nh.gemm(A, B).reshape(1, M, N)
    idx = sample_idx(1, M, N, 65536, 62)
    it = torch.from_numpy(idx).to(cuda)
    want = ref.gemm_sampled(a, b, idx)
    assert np.array_equal(got[it[:, 0], it[:, 1], it[:, 2]].cpu().numpy(), want)


@pytest.mark.parametrize("shape,layout", [((8192, 384, 50304), "NT"), ((384, 1536, 8192), "TN"),
                                          ((1536, 384, 8192), "TN")],
                         ids=["lm_head_grad_input", "mlp_grad_weight_384x1536", "mlp_grad_weight_1536x384"])
def test_f32_gemm_gpt_step_shapes_full_k(cuda, shape, layout):
    """The GPT step's long-K exact f32 GEMMs at their full shapes (the
    LM-head input gradient, K = 50304, on the 64x96 form; the MLP weight
    gradients, K = 8192, on the deep-stage 64x32 form), in the step's
    operand layouts, bit-exact against the oracle's sequential sum on
    16,384 sampled outputs and the corners."""
    import torch
    M, N, K = shape
    g = np.random.default_rng(63)
    a = g.uniform(-1, 1, (1, M, K)).astype(np.float32)
    b = g.uniform(-1, 1, (1, K, N)).astype(np.float32)
    A = view_as(a[0], layout[0], cuda, S.F32)
    B = view_as(b[0], layout[1], cuda, S.F32)
    got = nh.gemm(A, B).reshape(1, M, N)
    idx = sample_idx(1, M, N, 16384, 64)
    it = torch.from_numpy(idx).to(cuda)
    want = ref.gemm_sampled(a, b, idx)
    assert np.array_equal(got[it[:, 0], it[:, 1], it[:, 2]].cpu().numpy(), want)


def test_wrapper_kat_on_gpu(cuda):
    """test/wrapper.c:94-100 through the linear entry point, at full size."""
    import torch
    n = 4096
    x = torch.ones(n, n, device=cuda, dtype=torch.bfloat16)
    w = torch.ones(n, n, device=cuda, dtype=torch.bfloat16)
    bias = torch.full((n,), 0.5, device=cuda, dtype=torch.float32)
    y = nh.linear(x, w, bias, out_dtype=torch.float32)
    assert float((y - 4096.5).abs().max()) < 0.01


def test_c2_batch_matmul_bf16_full_size(cuda):
    """Config 2: linalg.batch_matmul bf16 -> f32, B=8, M=N=K=4096, seed 1."""
    inp = S.config_inputs("c2")
    A = to_dev(inp["A"], S.BF16, cuda)
    B = to_dev(inp["B"], S.BF16, cuda)
    import ctypes
    import torch
    C = torch.empty(8, 4096, 4096, device=cuda)
    dA, dB, dC = nh.memref_of(A), nh.memref_of(B), nh.memref_of(C)
    nh._bind_stream()
    nh.check(nh.lib()._mlir_ciface_nova_hip_batch_matmul_bf16_f32(nh.ref(dA), nh.ref(dB), nh.ref(dC)))
    idx = sample_idx(8, 4096, 4096, 65536, 17)
    it = torch.from_numpy(idx).to(cuda)
    got = C[it[:, 0], it[:, 1], it[:, 2]].cpu().numpy()
    want = ref.gemm_sampled(inp["A"], inp["B"], idx, adt=S.BF16, bdt=S.BF16)
    assert_close_lp(got, want, "c2")
    assert bool(torch.isfinite(C).all())


def test_c3_linear_bias_gelu_full_size(cuda):
    """Config 3: x[4096,4096] . W^T (W [11008,4096]) + b -> GELU(tanh) -> bf16."""
    import torch
    inp = S.config_inputs("c3")
    x = to_dev(inp["x"], S.BF16, cuda)
    W = to_dev(inp["W"], S.BF16, cuda)
    b = to_dev(inp["bias"], S.BF16, cuda)
    y = torch.empty(4096, 11008, device=cuda, dtype=torch.bfloat16)
    wt = W.t()  # nova.transpose view: [K,N] with strides (1, K)
    d = [nh.memref_of(t) for t in (x, wt)] + [nh.memref_of(b), nh.memref_of(y)]
    nh._bind_stream()
    nh.check(nh.lib()._mlir_ciface_nova_hip_linear_bf16_bias_gelu(*[nh.ref(v) for v in d]))
    idx = sample_idx(1, 4096, 11008, 65536, 18)
    it = torch.from_numpy(idx).to(cuda)
    got = y[it[:, 1], it[:, 2]].float().cpu().numpy()
    want = ref.gemm_sampled(inp["x"], inp["W"].T, idx, adt=S.BF16, bdt=S.BF16, bias=inp["bias"],
                            biasdt=S.BF16, epilogue=ref.EPI_BIAS_GELU, cdt=S.BF16)
    assert_close_lp(got, want, "c3")


@pytest.mark.parametrize("N", [2048, 4352])
@pytest.mark.parametrize("epi", [nh.EPI_GELU, nh.EPI_BIAS_GELU, nh.EPI_BIAS])
def test_dma_epilogue_f32_out(cuda, epi, N):
    """The LDS-DMA kernels' epilogue (bias staged in LDS as f32, GELU in its
    sigmoid form on the hardware exp2 / reciprocal) with f32 output, held to
    the f32 bar against the oracle's libm tanh evaluation.  N = 2048 gives 128
    whole 256x256 tiles (the one-tile-per-workgroup kernel), N = 4352 gives
    272 (the persistent kernel: 16 workgroups take two tiles, and each tile's
    bias goes to the LDS buffer of its parity)."""
    import torch
    M, K = 4096, 192
    x = S.normal((M, K), 31, dtype=S.BF16)
    w = S.normal((N, K), 31, 0.0, 0.08, dtype=S.BF16, offset=M * K)
    bias = S.normal((N,), 31, 0.0, 0.5, dtype=S.F32, offset=M * K + N * K)
    X = to_dev(x, S.BF16, cuda)
    Wt = to_dev(w, S.BF16, cuda).t()
    has_bias = epi in (nh.EPI_BIAS, nh.EPI_BIAS_GELU)
    Bs = torch.from_numpy(bias).to(cuda) if has_bias else None
    got = nh.gemm(X, Wt, bias=Bs, epilogue=epi).cpu().numpy()
    idx = sample_idx(1, M, N, 65536, 32)
    want = ref.gemm_sampled(x, w.T, idx, adt=S.BF16, bdt=S.BF16,
                            bias=bias if has_bias else None, biasdt=S.F32 if has_bias else None,
                            epilogue=epi)
    assert_close_f32(got[idx[:, 1], idx[:, 2]], want, f"dma epilogue {epi} N={N}")


@pytest.mark.parametrize("epi,odt", [(nh.EPI_BIAS_GELU, "bf16"), (nh.EPI_NONE, "bf16"),
                                     (nh.EPI_BIAS_GELU, "f16"), (nh.EPI_GELU, "f16")])
def test_persistent_epilogue_bf16_out(cuda, epi, odt):
    """The persistent kernel with 16-bit output (config 3's epilogue form for
    bf16): 272 tiles, bias in bf16, against the oracle rounded to the output
    dtype."""
    import torch
    cdt, tdt = (S.BF16, torch.bfloat16) if odt == "bf16" else (S.F16, torch.float16)
    M, N, K = 4096, 4352, 256
    x = S.normal((M, K), 33, dtype=S.BF16)
    w = S.normal((N, K), 33, 0.0, 0.06, dtype=S.BF16, offset=M * K)
    bias = S.normal((N,), 33, 0.0, 0.5, dtype=S.BF16, offset=M * K + N * K)
    has_bias = epi in (nh.EPI_BIAS, nh.EPI_BIAS_GELU)
    X = to_dev(x, S.BF16, cuda)
    Wt = to_dev(w, S.BF16, cuda).t()
    Bs = to_dev(bias, S.BF16, cuda) if has_bias else None
    got = nh.gemm(X, Wt, bias=Bs, epilogue=epi, out_dtype=tdt)
    idx = sample_idx(1, M, N, 65536, 34)
    it = torch.from_numpy(idx).to(cuda)
    g = got[it[:, 1], it[:, 2]].float().cpu().numpy()
    want = ref.gemm_sampled(x, w.T, idx, adt=S.BF16, bdt=S.BF16,
                            bias=bias if has_bias else None, biasdt=S.BF16 if has_bias else None,
                            epilogue=epi, cdt=cdt)
    assert_close_lp(g, want, f"persistent {odt} epilogue {epi}")


@pytest.mark.parametrize("epi,odt", [(nh.EPI_BIAS_GELU, "bf16"), (nh.EPI_BIAS, "f32"),
                                     (nh.EPI_GELU, "f16")])
def test_persistent_nn_epilogue(cuda, epi, odt):
    """The persistent kernel's NN form (row-major [K,N] weight, B staged in
    half-stages of 32 k) with bias / GELU epilogues: 272 tiles (16 workgroups
    take two, so the next tile's bias goes to the other LDS buffer) and five
    K steps, against the oracle at the output dtype's bar."""
    import torch
    cdt, tdt = {"bf16": (S.BF16, torch.bfloat16), "f16": (S.F16, torch.float16),
                "f32": (S.F32, torch.float32)}[odt]
    M, N, K = 4096, 4352, 320
    x = S.normal((M, K), 35, dtype=S.BF16)
    w = S.normal((K, N), 35, 0.0, 0.06, dtype=S.BF16, offset=M * K)
    bias = S.normal((N,), 35, 0.0, 0.5, dtype=S.BF16, offset=M * K + N * K)
    has_bias = epi in (nh.EPI_BIAS, nh.EPI_BIAS_GELU)
    Bs = to_dev(bias, S.BF16, cuda) if has_bias else None
    got = nh.gemm(to_dev(x, S.BF16, cuda), to_dev(w, S.BF16, cuda), bias=Bs, epilogue=epi,
                  out_dtype=tdt)
    idx = sample_idx(1, M, N, 65536, 36)
    it = torch.from_numpy(idx).to(cuda)
    g = got[it[:, 1], it[:, 2]].float().cpu().numpy()
    want = ref.gemm_sampled(x, w, idx, adt=S.BF16, bdt=S.BF16,
                            bias=bias if has_bias else None, biasdt=S.BF16 if has_bias else None,
                            epilogue=epi, cdt=cdt)
    if odt == "f32":
        assert_close_f32(g, want, f"persistent NN epilogue {epi}")
    else:
        assert_close_lp(g, want, f"persistent NN {odt} epilogue {epi}")


@pytest.mark.parametrize("epi,odt", [(nh.EPI_BIAS_GELU, "bf16"), (nh.EPI_BIAS, "f16"),
                                     (nh.EPI_GELU, "f32"), (nh.EPI_BIAS_GELU, "f32")])
@pytest.mark.parametrize("shape", [(3, 197, 197, 64), (2, 70, 61, 197), (1, 33, 257, 40),
                                   (2, 70, 64, 197), (96, 197, 64, 197), (96, 197, 197, 64)])
def test_gemm_small_epilogues(cuda, epi, odt, shape):
    """The small-K staged kernel (rows not 16-byte aligned) with bias / GELU
    epilogues and every output dtype: odd N puts a partial quad of four
    columns at the row end (element stores), and 16-bit rows of odd length
    leave some quads without 4-byte alignment.  N = 64 with f32 output
    writes whole 128-byte lines (the nontemporal-store form).  96 batches of
    197 rows make more 64-row tiles than CUs, so the last two shapes run in
    128-row windows, one workgroup per CU staging on sixteen waves: A staged
    (config 4b's form) and A read directly (config 4a's form)."""
    import torch
    cdt, tdt = {"bf16": (S.BF16, torch.bfloat16), "f16": (S.F16, torch.float16),
                "f32": (S.F32, torch.float32)}[odt]
    batch, M, N, K = shape
    a, b = lp_inputs((batch, M, K), (batch, K, N), S.F16, seed=41)
    bias = S.normal((N,), 41, 0.0, 0.5, dtype=S.F16, offset=7)
    has_bias = epi in (nh.EPI_BIAS, nh.EPI_BIAS_GELU)
    Bs = to_dev(bias, S.F16, cuda) if has_bias else None
    got = nh.gemm(to_dev(a, S.F16, cuda), to_dev(b, S.F16, cuda), bias=Bs, epilogue=epi,
                  out_dtype=tdt).float().cpu().numpy()
    want = ref.gemm(a, b, adt=S.F16, bdt=S.F16, bias=bias if has_bias else None,
                    biasdt=S.F16 if has_bias else None, epilogue=epi, cdt=cdt)
    want = S.widen(want, cdt) if cdt != S.F32 else want
    if odt == "f32":
        assert_close_f32(got, want, f"small {shape} epilogue {epi}")
    else:
        assert_close_lp(got, want, f"small {shape} {odt} epilogue {epi}")


@pytest.mark.parametrize("dt", [S.F16, S.BF16])
@pytest.mark.parametrize("shape", [(2, 197, 197, 64), (5, 100, 131, 32), (1, 37, 301, 16),
                                   (3, 260, 77, 48), (2, 129, 255, 64), (96, 197, 197, 64),
                                   (100, 150, 50, 32)])
def test_gemm_small_direct_a_exact(cuda, dt, shape):
    """The small-K kernel with A read straight into MFMA fragments (K-
    contiguous A with 16-byte aligned rows, K a multiple of 16 up to 64; B
    with unaligned N-contiguous rows is staged): 64- and 128-row windows,
    M off the 32-row blocks, N past one 256-column tile.  The last two
    shapes make more 64-row tiles than CUs but no more 128-row ones, so each
    workgroup is alone on its CU and stages on sixteen waves (config 4a's
    form), eight of which only stage.  Integer-valued
    inputs make every product and sum exact, so the output must equal the
    oracle's exactly."""
    import torch
    batch, M, N, K = shape
    g = np.random.default_rng(71)
    a = g.integers(-4, 5, (batch, M, K)).astype(np.float32)
    b = g.integers(-4, 5, (batch, K, N)).astype(np.float32)
    A = to_dev(S.round_to(a, dt), dt, cuda)
    B = to_dev(S.round_to(b, dt), dt, cuda)
    got = nh.gemm(A, B).cpu().numpy()
    want = ref.gemm(S.round_to(a, dt), S.round_to(b, dt), adt=dt, bdt=dt)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dt", [S.F16, S.BF16])
@pytest.mark.parametrize("layout", ["NN", "NT", "TN", "TT"])
@pytest.mark.parametrize("shape", [(100, 150, 50, 40), (96, 197, 64, 197)])
def test_gemm_small_128_row_windows_exact(cuda, dt, layout, shape):
    """The small-K kernel in 128-row windows with A staged: more 64-row tiles
    than CUs, so the 128-row form (eight computing waves) is chosen, and at
    K = 197 its staging (up to ~106 KB with A transposed) only fits because
    each workgroup has a CU to itself; such a workgroup stages on sixteen
    waves.  Integer-valued inputs make every
    product and sum exact, so every layout must equal the oracle exactly."""
    batch, M, N, K = shape
    g = np.random.default_rng(73)
    a = S.round_to(g.integers(-4, 5, (batch, M, K)).astype(np.float32), dt)
    b = S.round_to(g.integers(-4, 5, (batch, K, N)).astype(np.float32), dt)
    got = nh.gemm(view_as(a, layout[0], cuda, dt), view_as(b, layout[1], cuda, dt)).cpu().numpy()
    want = ref.gemm(a, b, adt=dt, bdt=dt)
    assert np.array_equal(got, want), f"{shape} {layout} dt={dt}"


@pytest.mark.parametrize("cfg", ["c4a", "c4b"])
def test_c4_fp16_unaligned_full(cuda, cfg):
    """Config 4: fp16 batch GEMM with non-tile-aligned shapes (edge tiles)."""
    inp = S.config_inputs(cfg)
    want = ref.gemm(inp["A"], inp["B"], adt=S.F16, bdt=S.F16)
    A = to_dev(inp["A"], S.F16, cuda)
    B = to_dev(inp["B"], S.F16, cuda)
    got = nh.batch_matmul(A, B).cpu().numpy()
    assert_close_lp(got, want, cfg)


def _strided_view(host, layout, dev, dt, offset, batch_pad):
    """Device view of host [batch, R, C] at element `offset` of a flat buffer,
    batch stride R*C + batch_pad; layout 'T' stores each slice transposed."""
    import torch
    batch, R, C = host.shape
    sl = host if layout == "N" else np.swapaxes(host, -1, -2)
    inner = sl.shape[1] * sl.shape[2]
    sb = inner + batch_pad
    flat = np.zeros(offset + batch * sb + 8, host.dtype)
    for b in range(batch):
        flat[offset + b * sb: offset + b * sb + inner] = np.ascontiguousarray(sl[b]).ravel()
    t = to_dev(flat, dt, dev)
    if layout == "N":
        return torch.as_strided(t, (batch, R, C), (sb, C, 1), offset)
    return torch.as_strided(t, (batch, R, C), (sb, 1, R), offset)


@pytest.mark.parametrize("layout", ["NN", "NT", "TN", "TT"])
@pytest.mark.parametrize("shape", [(3, 37, 45, 23), (2, 197, 197, 64), (2, 197, 64, 197),
                                   (2, 70, 300, 40)])
@pytest.mark.parametrize("offsets", [(1, 5), (3, 0), (0, 7)])
def test_gemm_staged_misaligned_exact(cuda, layout, shape, offsets):
    """Small-K kernel: slice bases at every 16-byte misalignment (odd storage
    offsets and odd batch strides).  Integer inputs make the f32 sums exact,
    so any misplaced element shows as an exact mismatch."""
    batch, M, N, K = shape
    g = np.random.default_rng(batch * 1000 + M + N + K)
    a = g.integers(-4, 5, size=(batch, M, K)).astype(np.float32)
    b = g.integers(-4, 5, size=(batch, K, N)).astype(np.float32)
    a16 = a.astype(np.float16).view(np.uint16)
    b16 = b.astype(np.float16).view(np.uint16)
    A = _strided_view(a16, layout[0], cuda, S.F16, offsets[0], 3)
    B = _strided_view(b16, layout[1], cuda, S.F16, offsets[1], 5)
    got = nh.gemm(A, B).cpu().numpy()
    want = np.einsum("bmk,bkn->bmn", a.astype(np.float64), b.astype(np.float64))
    np.testing.assert_array_equal(got, want.astype(np.float32))


@pytest.mark.parametrize("dt", [S.BF16, S.F16])
@pytest.mark.parametrize("layout", ["NN", "NT", "TN"])
@pytest.mark.parametrize("shape", [(1, 1, 1, 1), (2, 37, 45, 23), (1, 64, 64, 300), (3, 65, 70, 129)])
@pytest.mark.parametrize("bias", [False, True])
def test_gemm_narrow_accumulator_bit_exact(cuda, dt, layout, shape, bias):
    """NOVA_HIP_GEMM_ACC_OUT: linalg.matmul with bf16 / f16 outs accumulates in
    that type (NovaToLinalg.cpp:1027-1049); same bits as the oracle."""
    import torch
    batch, M, N, K = shape
    A, B = lp_inputs((batch, M, K), (batch, K, N), dt, 91 + K)
    bvec = S.uniform((N,), 92, dtype=dt) if bias else None
    dA = view_as(A, layout[0], cuda, dt)
    dB = view_as(B, layout[1], cuda, dt)
    tdt = torch.bfloat16 if dt == S.BF16 else torch.float16
    C = nh.gemm(dA, dB, bias=to_dev(bvec, dt, cuda) if bias else None,
                epilogue=nh.EPI_BIAS if bias else nh.EPI_NONE, out_dtype=tdt, acc_out=True)
    got = C.view(torch.int16).cpu().numpy().view(np.uint16)
    want = ref.gemm_acc_out(A, B, dt=dt, bias=bvec)
    assert np.array_equal(got, want)


def test_gemm_narrow_accumulator_stall_on_gpu(cuda):
    """4000 ones summed in f16 stop at 2048 (an f32 accumulator gives 4000)."""
    import torch
    A = torch.ones((1, 4000), dtype=torch.float16, device=cuda)
    B = torch.ones((4000, 8), dtype=torch.float16, device=cuda)
    C = nh.gemm(A, B, out_dtype=torch.float16, acc_out=True)
    assert (C.float() == 2048).all()
    assert (nh.gemm(A, B, out_dtype=torch.float16).float() == 4000).all()


def test_gemm_narrow_accumulator_refuses_other_forms(cuda):
    import torch
    A = torch.ones((4, 8), dtype=torch.bfloat16, device=cuda)
    with pytest.raises(nh.NovaHipError):
        nh.gemm(A, A.t().contiguous(), out_dtype=torch.float16, acc_out=True)   # bf16 -> f16
    with pytest.raises(nh.NovaHipError):
        nh.gemm(A, A.t().contiguous(), out_dtype=torch.float32, acc_out=True)   # f32 out
    with pytest.raises(nh.NovaHipError):
        nh.gemm(A, A.t().contiguous(), out_dtype=torch.bfloat16, acc_out=True,
                epilogue=nh.EPI_GELU)


# ------------------------------------------------ f32 on the matrix cores --
# NOVA_HIP_GEMM_F32_MFMA: f32 products, f32 sums in the MFMA's order.  Bar:
# the f32 one (rtol 1e-4, atol 1e-4 * max|c|), not bit-exactness.

@pytest.mark.parametrize("layout", ["NN", "NT", "TN", "TT"])
@pytest.mark.parametrize("shape", [(1, 1, 1, 1), (2, 37, 45, 23), (1, 130, 129, 70),
                                   (3, 128, 256, 96), (1, 200, 96, 4100), (1, 64, 384, 8192)])
def test_f32_mfma_gemm_layouts(cuda, layout, shape):
    batch, M, N, K = shape
    A = S.uniform((batch, M, K), 95)
    B = S.uniform((batch, K, N), 95, offset=A.size)
    C = nh.gemm(view_as(A, layout[0], cuda, S.F32), view_as(B, layout[1], cuda, S.F32),
                f32_mfma=True)
    assert_close_f32(C.cpu().numpy(), ref.gemm(A, B), f"f32 mfma {layout} {shape}")


@pytest.mark.parametrize("epi", [nh.EPI_BIAS, nh.EPI_BIAS_GELU, nh.EPI_GELU])
@pytest.mark.parametrize("K", [96, 6144])
def test_f32_mfma_gemm_epilogues(cuda, epi, K):
    """Bias first (split 0 starts from it) and GELU after the split sum."""
    M, N = 100, 200
    A = S.normal((M, K), 96, 0, 0.05)
    B = S.normal((K, N), 96, 0, 0.05, offset=A.size)
    bias = S.normal((N,), 96, offset=A.size + B.size)
    has_bias = epi != nh.EPI_GELU
    C = nh.gemm(to_dev(A, S.F32, cuda), to_dev(B, S.F32, cuda),
                bias=to_dev(bias, S.F32, cuda) if has_bias else None, epilogue=epi,
                f32_mfma=True)
    want = ref.gemm(A, B, bias=bias if has_bias else None, epilogue=epi)[0]
    assert_close_f32(C.cpu().numpy(), want, f"f32 mfma epilogue {epi} K={K}")


def test_f32_mfma_same_bits_every_run_and_unaligned_rows(cuda):
    import torch
    A = S.uniform((65, 3001), 97)
    B = S.uniform((3001, 77), 97, offset=A.size)
    dA, dB = to_dev(A, S.F32, cuda), to_dev(B, S.F32, cuda)
    c1 = nh.gemm(dA, dB, f32_mfma=True)
    c2 = nh.gemm(dA, dB, f32_mfma=True)
    assert torch.equal(c1, c2)
    assert_close_f32(c1.cpu().numpy(), ref.gemm(A, B)[0], "unaligned f32 mfma")
    # an offset view: rows no longer 16-byte aligned
    wide = S.uniform((40, 130), 98)
    dW = to_dev(wide, S.F32, cuda)[:, 1:129]
    Bs = S.uniform((128, 50), 98, offset=wide.size)
    c = nh.gemm(dW, to_dev(Bs, S.F32, cuda), f32_mfma=True)
    assert_close_f32(c.cpu().numpy(), ref.gemm(np.ascontiguousarray(wide[:, 1:129]), Bs)[0],
                     "offset rows")


def test_f32_mfma_split_k_with_many_tiles(cuda):
    """K split over workgroups also when the tiles alone fill more than a
    round (600 tiles of K = 4096: the time model picks 4 splits on a
    256-CU part), checked on 65,536 sampled outputs against the oracle's
    sequential sum at the f32 bar, with a bias that only split 0 adds."""
    import torch
    M, N, K = 384, 25600, 4096
    A = S.uniform((1, M, K), 101)
    B = S.uniform((1, K, N), 101, offset=A.size)
    bias = S.uniform((N,), 102)
    C = nh.gemm(to_dev(A[0], S.F32, cuda), view_as(B[0], "T", cuda, S.F32),
                bias=to_dev(bias, S.F32, cuda), epilogue=nh.EPI_BIAS, f32_mfma=True).reshape(1, M, N)
    idx = sample_idx(1, M, N, 65536, 103)
    it = torch.from_numpy(idx).to(cuda)
    want = ref.gemm_sampled(A, B, idx, bias=bias, biasdt=S.F32, epilogue=ref.EPI_BIAS)
    assert_close_f32(C[it[:, 0], it[:, 1], it[:, 2]].cpu().numpy(), want, "split-K, many tiles")


def test_f32_mfma_backward_entry_points(cuda):
    M, K, N = 300, 96, 200
    x = S.normal((M, K), 99)
    w = S.normal((K, N), 99, 0, 0.1, offset=x.size)
    go = S.normal((M, N), 99, offset=x.size + w.size)
    gi, gw, gb = nh.linear_backward(to_dev(go, S.F32, cuda), to_dev(x, S.F32, cuda),
                                    to_dev(w, S.F32, cuda), f32_mfma=True)
    gi_r, gw_r, gb_r = ref.linear_backward(go, x, w)
    assert_close_f32(gi.cpu().numpy(), gi_r, "grad_input")
    assert_close_f32(gw.cpu().numpy(), gw_r, "grad_weight")
    assert_close_f32(gb.cpu().numpy(), gb_r, "grad_bias")


def test_typed_gemm_alias_matches_generic_entry_point(cuda):
    """The typed alias a lowered module calls gives the generic entry point's
    bits (bf16 in, bf16 bias + GELU epilogue, bf16 out)."""
    import torch
    A, B = lp_inputs((1, 96, 160), (1, 160, 200), S.BF16, 93)
    bias = S.uniform((200,), 94, dtype=S.BF16)
    dA, dB, db = to_dev(A, S.BF16, cuda), to_dev(B, S.BF16, cuda), to_dev(bias, S.BF16, cuda)
    want = nh.gemm(dA, dB, bias=db, epilogue=nh.EPI_BIAS_GELU, out_dtype=torch.bfloat16)
    got = torch.empty_like(want)
    flags = nh.gemm_flags(nh.DT_BF16, nh.DT_BF16, nh.EPI_BIAS_GELU, nh.DT_BF16)
    d = [nh.memref_of(t) for t in (dA, dB, got, db)]
    nh._bind_stream()
    nh.check(nh.lib()._mlir_ciface_nova_hip_gemm_bf16_bf16_bbf16(*[nh.ref(v) for v in d], flags))
    assert torch.equal(got, want)


def _random_cases(n, seed):
    """Seeded GEMM problems spread over every kernel path: small and odd
    shapes (register-staged and small-K kernels), multiples of 256 with
    enough tiles for the LDS-DMA and persistent kernels, the f32 exact and
    matrix-core forms; random layout, batch, bias dtype, epilogue and output
    dtype."""
    g = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        dt = [S.BF16, S.F16, S.F32][i % 3]
        kind = g.integers(0, 4)
        if kind == 0:      # small / odd
            batch, M, N, K = int(g.integers(1, 4)), int(g.integers(1, 300)), int(g.integers(1, 300)), int(g.integers(1, 300))
        elif kind == 1:    # unaligned rows, small K
            batch, M, N, K = int(g.integers(1, 9)), int(g.integers(100, 260)) | 1, int(g.integers(60, 260)) | 1, int(g.integers(8, 200))
        elif kind == 2:    # tile-aligned, many tiles
            batch, M, N, K = int(g.integers(2, 5)), 256 * int(g.integers(4, 9)), 256 * int(g.integers(4, 9)), 64 * int(g.integers(2, 6))
        else:              # medium, ragged
            batch, M, N, K = 1, int(g.integers(500, 1400)), int(g.integers(500, 1400)), int(g.integers(30, 400))
        layout = "NT"[g.integers(0, 2)] + "NT"[g.integers(0, 2)]
        epi = [nh.EPI_NONE, nh.EPI_BIAS, nh.EPI_BIAS_GELU, nh.EPI_GELU][g.integers(0, 4)]
        odt = dt if dt == S.F32 else [S.F32, dt][g.integers(0, 2)]
        mfma = dt == S.F32 and bool(g.integers(0, 2))
        cases.append((i, dt, layout, (batch, M, N, K), epi, odt, mfma))
    return cases


@pytest.mark.parametrize("case", _random_cases(48, 61), ids=lambda c: f"r{c[0]}")
def test_gemm_random_sweep(cuda, case):
    """Random problems across the GEMM family against the oracle on sampled
    outputs: bf16/f16 at the low-precision bar, f32 bit-exact (the exact
    kernels; GELU through tanhf within the f32 bar) or at the f32 bar (the
    matrix-core form)."""
    import torch
    i, dt, layout, (batch, M, N, K), epi, odt, mfma = case
    g = np.random.default_rng(1000 + i)
    if dt == S.F32:
        a = g.uniform(-1, 1, (batch, M, K)).astype(np.float32)
        b = g.uniform(-1, 1, (batch, K, N)).astype(np.float32)
    else:
        a, b = lp_inputs((batch, M, K), (batch, K, N), dt, seed=1000 + i)
    has_bias = epi in (nh.EPI_BIAS, nh.EPI_BIAS_GELU)
    bias = (S.normal((N,), 1000 + i, 0.0, 0.5, dtype=dt, offset=3) if dt != S.F32
            else g.uniform(-1, 1, N).astype(np.float32)) if has_bias else None
    tdt = {S.F32: torch.float32, S.BF16: torch.bfloat16, S.F16: torch.float16}[odt]
    A = view_as(a, layout[0], cuda, dt)
    B = view_as(b, layout[1], cuda, dt)
    got = nh.gemm(A, B, bias=to_dev(bias, dt, cuda) if has_bias else None, epilogue=epi,
                  out_dtype=tdt, f32_mfma=mfma)
    idx = sample_idx(batch, M, N, 4096, 2000 + i)
    it = torch.from_numpy(idx).to(cuda)
    gs = got[it[:, 0], it[:, 1], it[:, 2]].float().cpu().numpy()
    want = ref.gemm_sampled(a, b, idx, adt=None if dt == S.F32 else dt, bdt=None if dt == S.F32 else dt,
                            bias=bias, biasdt=dt if has_bias else None, epilogue=epi, cdt=odt)
    what = f"case {i}: {dt} {layout} {(batch, M, N, K)} epi {epi} out {odt} mfma {mfma}"
    if dt != S.F32:
        assert_close_lp(gs, want, what)
    elif mfma or epi in (nh.EPI_GELU, nh.EPI_BIAS_GELU):
        assert_close_f32(gs, want, what)
    else:
        assert np.array_equal(gs, want), (what, float(np.abs(gs - want).max()))


def test_small_k_output_rows_far_apart(cuda):
    """Small-K kernel, f32 output rows 2^26 elements apart (a strided view
    of a 512 MB buffer) and M = 2: a store instruction of the last row window
    addresses rows up to 31, whose 32-bit byte offsets (row * 2^28) would
    wrap around 2^32 onto row 0 if the buffer-store path took them.  Every
    written row matches the oracle and the rows between stay untouched."""
    import torch
    M, N, K, stride = 2, 64, 9, 1 << 26
    a, b = lp_inputs((1, M, K), (1, K, N), S.F16, seed=17)
    want = ref.gemm(a, b, adt=S.F16, bdt=S.F16)[0]
    big = torch.full((M, stride), 7.0, device=cuda)
    C = big[:, :N]
    nh.gemm(to_dev(a[0], S.F16, cuda), to_dev(b[0], S.F16, cuda), out=C)
    assert_close_lp(C.cpu().numpy(), want, "rows 2^26 apart")
    assert bool((big[:, N:N + 4096] == 7.0).all())


def _wide_small_cases(n=12, seed=2026):
    """Seeded shapes for the small-K kernel's sixteen-wave form: 197 rows,
    odd K or N (16-bit rows not 16-byte aligned), and a batch that makes
    more 64-row tiles than a 256-CU part has CUs but no more 128-row ones."""
    g = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        i = len(cases)
        dt = [S.F16, S.BF16][(i // 3) % 2]
        if i % 3 == 0:
            # K-contiguous A with 16-byte aligned rows, K a multiple of 16
            # up to 64: A read directly; B's N-contiguous rows of odd N keep
            # the small-K kernel.
            K = 16 * int(g.integers(1, 5))
            N = int(g.integers(1, 129)) | 1
            layout = "NN"
        else:
            K = int(g.integers(1, 161)) | 1
            N = int(g.integers(1, 257))
            layout = ["NN", "NT", "TN", "TT"][i % 4]
        batch = int(g.integers(65, 129))
        cases.append((batch, 197, N, K, layout, dt))
    return cases


@pytest.mark.parametrize("case", _wide_small_cases())
def test_gemm_small_sixteen_wave_random_exact(cuda, case):
    """The small-K kernel when each workgroup has a CU to itself (128-row
    windows, sixteen staging waves; A staged or, for K-contiguous aligned A,
    read directly): random shapes and layouts from a fixed seed.  Integer-
    valued inputs make every product and sum exact, so the output must equal
    the oracle's exactly."""
    batch, M, N, K, layout, dt = case
    g = np.random.default_rng(batch * 100003 + N * 311 + K)
    a = S.round_to(g.integers(-4, 5, (batch, M, K)).astype(np.float32), dt)
    b = S.round_to(g.integers(-4, 5, (batch, K, N)).astype(np.float32), dt)
    got = nh.gemm(view_as(a, layout[0], cuda, dt), view_as(b, layout[1], cuda, dt)).cpu().numpy()
    want = ref.gemm(a, b, adt=dt, bdt=dt)
    assert np.array_equal(got, want), case


@pytest.mark.parametrize("layout", ["NN", "NT", "TN", "TT"])
@pytest.mark.parametrize("shape", [(1, 100, 200, 300), (1, 256, 512, 128), (1, 128, 128, 128),
                                   (2, 37, 45, 23), (3, 65, 70, 129), (4, 64, 64, 256)])
def test_gemm_accumulate_into_c_bit_exact(cuda, layout, shape):
    """NOVA_HIP_GEMM_ACC_C (linalg.matmul on data-holding outs): C + A . B with
    each sum starting from C's value, k ascending; the exact kernel's scalar
    form (unaligned rows) and vector forms (aligned), bit for bit."""
    import torch
    batch, M, N, K = shape
    g = np.random.default_rng(131 + K)
    a = g.uniform(-1, 1, (batch, M, K)).astype(np.float32)
    b = g.uniform(-1, 1, (batch, K, N)).astype(np.float32)
    c0 = g.uniform(-4, 4, (batch, M, N)).astype(np.float32)
    A = view_as(a, layout[0], cuda, S.F32)
    B = view_as(b, layout[1], cuda, S.F32)
    C = torch.from_numpy(c0).to(cuda)
    nh.gemm(A, B, C, acc_c=True)
    assert np.array_equal(C.cpu().numpy(), ref.gemm_accumulate(a, b, c0)), (shape, layout)


@pytest.mark.parametrize("dt", [S.BF16, S.F16])
def test_gemm_accumulate_into_narrow_c_bit_exact(cuda, dt):
    """The same into bf16 / f16 outs: every product and partial sum rounded
    to that type, starting from C's value."""
    import torch
    batch, M, N, K = 2, 37, 45, 23
    A, B = lp_inputs((batch, M, K), (batch, K, N), dt, 133)
    c0 = S.uniform((batch, M, N), 134, dtype=dt)
    C = to_dev(c0, dt, cuda).clone()
    nh.gemm(to_dev(A, dt, cuda), to_dev(B, dt, cuda), C, acc_out=True, acc_c=True)
    got = C.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got, ref.gemm_accumulate(A, B, c0, adt=dt, bdt=dt, cdt=dt))


def test_gemm_accumulate_with_k0_leaves_c(cuda):
    import torch
    A = torch.zeros((1, 5, 0), device=cuda)
    B = torch.zeros((1, 0, 7), device=cuda)
    C = torch.arange(35, dtype=torch.float32, device=cuda).reshape(1, 5, 7)
    before = C.clone()
    nh.gemm(A, B, C, acc_c=True)
    assert torch.equal(C, before)
