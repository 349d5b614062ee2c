"""libnova_hip under HIP graph capture.  Once each entry point has run on a
stream (which allocates that stream's workspace), its launches on that
stream can be captured into a graph: they make no allocation, no
synchronisation and no memset.  A sequence of the library's entry points is
captured once and replayed three times, with new inputs written eagerly
between the replays, and every replay's outputs equal, bit for bit, the same
calls made eagerly on the new inputs."""
import numpy as np
import pytest

import nova_hip as nh
import nova_seed as S

pytestmark = pytest.mark.gpu


def test_library_calls_replay_from_a_hip_graph(cuda):
    import torch

    def dev(a, dt=None):
        t = torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
        return t if dt is None else t.to(dt)

    bf = torch.bfloat16
    g = torch.Generator(device="cpu").manual_seed(5)

    def fresh(*shape, dt=torch.float32, scale=1.0):
        return (torch.randn(*shape, generator=g) * scale).to(dt).to(cuda)

    # inputs (rewritten in place between replays)
    A, B = fresh(2, 512, 384, dt=bf), fresh(2, 384, 640, dt=bf)
    x, W, b = fresh(256, 512, dt=bf), fresh(768, 512, dt=bf, scale=0.05), fresh(768, dt=bf)
    xl = fresh(300, 1024)
    gam, bet = fresh(1024, scale=0.1) + 1.0, fresh(1024, scale=0.1)
    logits = fresh(200, 5000, scale=2.0)
    labels = dev(S.labels(200, 5000, 7))
    gy = fresh(300, 1024)
    go = fresh(256, 768, dt=bf)
    f32a, f32b = fresh(64, 96), fresh(96, 80)
    inputs = [A, B, x, W, b, xl, logits, gy, go, f32a, f32b]

    # outputs (preallocated: the capture allocates nothing)
    C = torch.empty(2, 512, 640, device=cuda)
    Y = torch.empty(256, 768, device=cuda, dtype=bf)
    yl, sl, rl = torch.empty(300, 1024, device=cuda), torch.empty(300, device=cuda), torch.empty(300, device=cuda)
    loss = torch.empty(1, device=cuda)
    dx, dg, db = torch.empty(300, 1024, device=cuda), torch.empty(1024, device=cuda), torch.empty(1024, device=cuda)
    gi, gw, gb = torch.empty(256, 512, device=cuda), torch.empty(512, 768, device=cuda), torch.empty(768, device=cuda)
    Cf = torch.empty(64, 80, device=cuda)
    Cacc = torch.empty(64, 80, device=cuda)
    outs = [C, Y, yl, sl, rl, loss, dx, dg, db, gi, gw, gb, Cf, Cacc]

    def run():
        nh.gemm(A, B, C)                                           # batch GEMM bf16 -> f32
        nh.gemm(x, W.t(), Y, bias=b, epilogue=nh.EPI_BIAS_GELU)    # linear + bias + GELU -> bf16
        nh.layer_norm(xl, gam, bet, y=yl, mean_sum=sl, rstd=rl)
        nh.sce(logits, labels, loss=loss)                          # row kernel + mean, workspace
        nh.layer_norm_backward(gy, xl, gam, sl, rl, dx=dx, dgamma=dg, dbeta=db)
        nh.linear_backward(go, x, W.t(), grad_input=gi, grad_weight=gw, grad_bias=gb)
        nh.gemm(f32a, f32b, Cf)                                    # exact f32
        Cacc.copy_(Cf)
        nh.gemm(f32a, f32b, Cacc, acc_c=True)                      # accumulate into C

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()                      # set-up: the stream's workspace is allocated here
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            run()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for i in range(3):
        for t in inputs:
            t.copy_((torch.randn(t.shape, generator=g) * 0.5).to(t.dtype))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [o.clone() for o in outs]
        run()                      # eager, on the current stream
        torch.cuda.synchronize()
        for k, (a, e) in enumerate(zip(got, outs)):
            assert torch.equal(a, e), (i, k)
