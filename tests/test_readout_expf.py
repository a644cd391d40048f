"""The readout's exponential is non-decreasing on [-87, 0], checked for every float of that range.

The C = 32 streamed kernel makes the gated-firing decision of a 2-output mlp head
(conf > tau, engine/rollout.py's adaptive firing through the readout of model.py) by comparing the
gap between the two logits with a limit found on the host, instead of evaluating
1 + readout_expf(gap) < conf_s. The two agree for every gap exactly when readout_expf never
decreases as its argument grows (below -87 it is clamped, so constant). `expf_monotone.hip`
includes the kernel's own definition and walks all 1.1e9 floats of the range on the CPU.
"""
from __future__ import annotations

import os
import subprocess

import pytest

from ncas_amd import build as B

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(not os.path.exists(B.HIPCC), reason="hipcc is not installed")
def test_readout_expf_is_non_decreasing_on_its_whole_range(tmp_path):
    exe = str(tmp_path / "expf_monotone")
    cmd = [B.HIPCC, *B.FLAGS, "-o", exe, os.path.join(HERE, "expf_monotone.hip"), "-lpthread"]
    subprocess.run(cmd, check=True, capture_output=True, timeout=300)
    res = subprocess.run([exe], capture_output=True, text=True, timeout=600)
    assert res.stdout.strip() == "decreasing steps: 0", res.stdout + res.stderr
    assert res.returncode == 0
