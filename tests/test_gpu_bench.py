"""bench.py's workloads run end to end on the GPU (short versions): every workload's timing path
is exercised by the test suite, not only by the benchmark run itself."""

from __future__ import annotations

import json
import math
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402

pytestmark = pytest.mark.gpu


def test_bptt30_training_iteration_runs():
    """The 30x30 BPTT training iteration (pool sample, 32-step chunk, AdamW, write-back)."""
    res = bench.run_bptt(bench.WORKLOADS["bptt30"], "bf16", 1, 0)
    assert res["ms_per_step"] > 0 and all(math.isfinite(v) for v in res["loss"])
    assert res["workspace_bytes"] > 0


@pytest.mark.parametrize("workload", ["sudoku9", "maze13", "hardmaze30", "maze201"])
def test_bench_workload_line(workload):
    """`bench.py --workload W` at a few steps prints one JSON line with the contract's keys."""
    cmd = [sys.executable, str(ROOT / "bench.py"), "--workload", workload, "--steps", "1", "--warmup", "0",
           "--no-cpu", "--no-fp32", "--no-regimes", "--depth", "4"]
    out = subprocess.run(cmd, capture_output=True, text=True, timeout=600, cwd=ROOT)
    assert out.returncode == 0, out.stderr[-2000:]
    line = json.loads(out.stdout.strip().splitlines()[-1])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "ms_per_step", "dtype", "config", "roofline"):
        assert key in line, key
    assert line["value"] > 0 and line["n_gpus"] == 1
