"""bench.py's command-line contract on the CPU: more than one GPU is refused
with a message and exit status 2 (this build measures one GPU; sharding is
design-only), a host with no GPU gets exit status 1 and a message rather
than a traceback or a fallback measurement, and --help lists the flags the
driver passes."""
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run_bench(*args, timeout=300):
    return subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), *args], cwd=REPO,
                          capture_output=True, text=True, timeout=timeout)


@pytest.mark.parametrize("n", ["2", "8"])
def test_more_than_one_gpu_is_refused(n):
    r = run_bench("--gpus", n, "--steps", "1", "--warmup", "0")
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""


def test_help_lists_the_driver_flags():
    r = run_bench("--help")
    assert r.returncode == 0
    for flag in ("--gpus", "--steps", "--warmup", "--only", "--no-cpu-baseline"):
        assert flag in r.stdout


def test_no_gpu_is_an_error_not_a_measurement():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible here")
    r = run_bench("--steps", "1", "--warmup", "0", "--no-cpu-baseline")
    assert r.returncode == 1
    assert "no GPU visible" in r.stderr
    assert r.stdout == ""
