"""Concurrent calls from several host threads, each on a stream of its own
or all on one: the calling thread's stream (nova_hip_set_stream is
thread-local) and the per-stream workspace (SCE row losses,
LayerNorm-backward partials, split-K partials of the f32 matrix-core GEMM),
held per call under the stream's lease, keep the calls apart, and every
result equals the same call made alone on one stream, bit for bit."""
import threading

import numpy as np
import pytest

import nova_hip as nh
import nova_seed as S

pytestmark = pytest.mark.gpu


def _inputs(torch, dev, seed, rows):
    """One thread's inputs: sizes differ per thread, so the workspaces do."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn(rows, 1024, generator=g).to(dev)
    lab = torch.randint(0, 1024, (rows,), generator=g, dtype=torch.int32).to(dev)
    gy = torch.randn(rows, 1024, generator=g).to(dev)
    gamma = (1 + 0.1 * torch.randn(1024, generator=g)).to(dev)
    A = torch.randn(64 + seed, 8192, generator=g).to(dev)
    B = torch.randn(8192, 320, generator=g).to(dev)
    return x, lab, gy, gamma, A, B


def _run(torch, inp):
    x, lab, gy, gamma, A, B = inp
    loss, grad = nh.sce_fwd_bwd(x, lab)
    beta = torch.zeros_like(gamma)
    y, S_, r = nh.layer_norm(x, gamma, beta)
    dx, dg, db = nh.layer_norm_backward(gy, x, gamma, S_, r)
    C = nh.gemm(A, B, f32_mfma=True)  # K = 8192 over few tiles: split K
    return [loss, grad, y, dx, dg, db, C]


def test_threads_on_own_streams_match_single_stream(cuda):
    import torch
    inputs = [_inputs(torch, cuda, s, 512 + 96 * s) for s in range(4)]
    want = [[t.clone() for t in _run(torch, inp)] for inp in inputs]
    torch.cuda.synchronize()
    got = [None] * len(inputs)
    errors = []

    def worker(i):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                out = None
                for _ in range(5):
                    out = _run(torch, inputs[i])
                s.synchronize()
                got[i] = [t.clone() for t in out]
                s.synchronize()
        except Exception as e:  # reported below
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(inputs))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    names = ["loss", "grad", "y", "dx", "dgamma", "dbeta", "gemm"]
    for i in range(len(inputs)):
        for n, a, b in zip(names, got[i], want[i]):
            assert torch.equal(a, b), (i, n)


def test_threads_sharing_one_stream_match_single_stream(cuda):
    """Threads on one stream (as every thread that sets no stream shares the
    null stream): each call enqueues its kernels under the stream's
    workspace lease, so no call's mean, column sums or split-K reduction
    reads another call's partials.  Equal sizes on every thread: the shared
    buffer is never regrown, only contended."""
    import torch
    inputs = [_inputs(torch, cuda, s, 640) for s in range(4)]
    inputs = [(x, lab, gy, gamma, A[:64].contiguous(), B) for x, lab, gy, gamma, A, B in inputs]
    want = [[t.clone() for t in _run(torch, inp)] for inp in inputs]
    torch.cuda.synchronize()
    shared = torch.cuda.Stream()
    got = [None] * len(inputs)
    errors = []

    def worker(i):
        try:
            with torch.cuda.stream(shared):
                outs = [_run(torch, inputs[i]) for _ in range(8)]
                shared.synchronize()
                got[i] = [[t.clone() for t in out] for out in outs]
                shared.synchronize()
        except Exception as e:  # reported below
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(inputs))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    names = ["loss", "grad", "y", "dx", "dgamma", "dbeta", "gemm"]
    for i in range(len(inputs)):
        for k, out in enumerate(got[i]):
            for n, a, b in zip(names, out, want[i]):
                assert torch.equal(a, b), (i, k, n)
