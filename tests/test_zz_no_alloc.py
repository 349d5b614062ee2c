"""_mlir_ciface_nova_hip_sce_f32_noalloc, the SCE entry point that allocates
nothing (row losses in the library's static per-GPU array), against
_mlir_ciface_nova_hip_sce_f32 through the C ABI: the same loss and softmax
bits on consecutive calls, the later ones smaller, and the oracle's loss."""
import numpy as np
import pytest

import nova_cpu_ref as ref
import nova_hip as nh
import nova_seed as S
from conftest import assert_close_f32

pytestmark = pytest.mark.gpu

MAX_ROWS = 262144  # SCE_NOALLOC_MAX_ROWS of include/nova_hip.h


def _pair(x, t, cuda):
    import torch
    X, T = torch.from_numpy(x).to(cuda), torch.from_numpy(t).to(cuda)
    sm1, l1 = nh.sce(X, T, softmax=True)
    sm2, l2 = nh.sce(X, T, softmax=True, noalloc=True)
    torch.cuda.synchronize()
    return sm1, l1, sm2, l2


def test_sce_noalloc_matches_the_allocating_entry_point(cuda):
    import torch
    # large then smaller: the second call's rows are a prefix of the array
    # the first filled, so stale row losses would show in its mean
    for rows, C, seed in ((300, 5000, 61), (37, 40000, 62), (5, 777, 63)):
        x = S.normal((rows, C), seed, 0, 2)
        t = S.labels(rows, C, seed, offset=rows * C)
        sm1, l1, sm2, l2 = _pair(x, t, cuda)
        assert torch.equal(l1, l2), (rows, C)
        assert torch.equal(sm1, sm2), (rows, C)
        _, lref, _ = ref.sce(x, t)
        assert_close_f32(l2.cpu().numpy(), lref, f"noalloc {rows}x{C}")


def test_sce_noalloc_at_the_row_limit(cuda):
    import torch
    rows, C = MAX_ROWS, 3
    x = S.normal((rows, C), 64, 0, 2)
    t = S.labels(rows, C, 64, offset=rows * C)
    sm1, l1, sm2, l2 = _pair(x, t, cuda)
    assert torch.equal(l1, l2) and torch.equal(sm1, sm2)
    X = torch.zeros((rows + 1, C), device=cuda)
    T = torch.zeros(rows + 1, dtype=torch.int32, device=cuda)
    with pytest.raises(nh.NovaHipError) as e:
        nh.sce(X, T, noalloc=True)
    assert e.value.code == 5 and "scratch maximum" in str(e.value)
    # a smaller call after the refusal still matches
    x = S.normal((9, 100), 65, 0, 2)
    t = S.labels(9, 100, 65, offset=900)
    sm1, l1, sm2, l2 = _pair(x, t, cuda)
    assert torch.equal(l1, l2) and torch.equal(sm1, sm2)


def test_sce_noalloc_under_hip_graph_capture(cuda):
    """The callers this entry point is for: captured in a HIP graph (which
    the allocating entry point's first call could not be) and replayed
    three times, with new logits written eagerly between the replays; every
    replay's loss equals the allocating entry point's on the same logits."""
    import torch
    rows, C = 256, 3000
    X = torch.empty((rows, C), device=cuda)
    T = torch.from_numpy(S.labels(rows, C, 66)).to(cuda)
    loss = torch.empty(1, device=cuda)
    X.copy_(torch.from_numpy(S.normal((rows, C), 66, 0, 2)))
    nh.sce(X, T, loss=loss, noalloc=True)  # set-up call outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            nh.sce(X, T, loss=loss, noalloc=True)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for i in range(3):
        X.copy_(torch.from_numpy(S.normal((rows, C), 67 + i, 0, 2)))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = loss.clone()
        _, want = nh.sce(X, T)
        torch.cuda.synchronize()
        assert torch.equal(got, want), i
