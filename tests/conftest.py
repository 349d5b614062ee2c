"""Shared test setup: paths to the package, the oracle and the golden data;
the `gpu` marker; tolerance helpers stating the parity bar."""
import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "nova-compiler_amd")
ORACLE = os.path.join(REPO, "oracle")
GOLDEN = os.path.join(REPO, "tests", "golden")
for p in (PKG, ORACLE):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu)")


# Parity bar: element-wise |g - c| <= rtol*|c| + atol.
#   f32:            rtol 1e-4, atol 1e-4 * max|c| (normwise floor)
#   bf16/f16 in, f32 accumulate: rtol 2e-2, atol 1e-2
F32_RTOL = 1e-4
LP_RTOL, LP_ATOL = 2e-2, 1e-2


def assert_close_f32(got, want, what=""):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    if want.size == 0:
        return
    atol = F32_RTOL * float(np.max(np.abs(want)))
    err = np.abs(got - want)
    bad = err > F32_RTOL * np.abs(want) + atol
    assert not bad.any(), (
        f"{what}: {int(bad.sum())} of {want.size} outside rtol 1e-4 / atol {atol:.3g}; "
        f"worst |d|={err.max():.3g} at {np.unravel_index(np.argmax(err), err.shape)}")


def assert_close_lp(got, want, what=""):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    err = np.abs(got - want)
    bad = err > LP_RTOL * np.abs(want) + LP_ATOL
    assert not bad.any(), (
        f"{what}: {int(bad.sum())} of {want.size} outside rtol 2e-2 / atol 1e-2; "
        f"worst |d|={err.max():.3g}")


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    return torch.device("cuda:0")
