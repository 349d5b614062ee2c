"""bench.py's output on the GPU: one JSON line on stdout that carries
BASELINE.json's metric, config 2's time and throughput consistent with each
other and with the roofline object, and a finite result.  A short run:
config 2 only, two timed steps, no CPU baseline."""
import json
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
C2_FLOP = 2 * 8 * 4096 ** 3


def test_bench_line_contract(cuda):
    r = subprocess.run([sys.executable, "-u", os.path.join(REPO, "bench.py"), "--only", "c2",
                        "--steps", "2", "--warmup", "1", "--no-cpu-baseline"],
                       cwd=REPO, capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = r.stdout.strip().splitlines()
    assert len(lines) == 1, lines
    d = json.loads(lines[0])
    with open(os.path.join(REPO, "BASELINE.json")) as f:
        assert d["metric"] == json.load(f)["metric"]
    assert (d["unit"], d["n_gpus"], d["steps"], d["warmup"]) == ("TFLOP/s", 1, 2, 1)
    assert d["higher_is_better"] is True and d["vs_baseline"] is None
    assert d["config"]["workload"].startswith("c2:")
    ms, v = d["ms_per_step"], d["value"]
    assert 0.3 < ms < 5.0, ms
    assert v == pytest.approx(C2_FLOP / (ms * 1e-3) / 1e12, rel=1e-9)
    rl = d["roofline"]
    assert (rl["bound"], rl["unit"], rl["peak"]) == ("mfma", "TFLOP/s", 2516.6)
    assert rl["achieved"] == v and rl["frac"] == pytest.approx(v / rl["peak"], rel=1e-9)
    assert "[bench] c2:" in r.stderr and '"finite": true' in r.stderr
