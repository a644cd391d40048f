"""The training recipe around the HIP engine (ncas_amd.trainer.train_fast) on the GPU: it writes
the reference's run files, its final weights load back, and a run interrupted at a checkpoint
resumes bit for bit (reference tests/test_engine_train.py:228-249), also when stopped with
stop_at_step under a warm-up + cosine schedule (test_engine_train.py:185-210)."""

from __future__ import annotations

import json

import pytest
import torch

from ncas_amd.trainer import load_model, train_fast

pytestmark = pytest.mark.gpu


def _cfg(steps, **train):
    tr = dict(steps=steps, batch_size=4, pool_mult=4, rollout=6, chunk=4, loss="ce", lr=5e-4,
              log_every=2, eval_every=steps, checkpoint_every=3, damage={"p": 0.5},
              swap={"p": 0.25}, noise={"sigma": 0.0}, eval={"n": 8, "depth": 6, "k": 1})
    tr.update(train)
    return {
        "task": {"name": "maze", "train": {"n": 64, "size": 9, "seed": 0},
                 "val": {"n": 8, "size": 9, "seed": 1}},
        "model": {"preset": "maze_hard_c32", "overrides": {"fire_rate": 0.8}},
        "train": tr,
        "engine": {"backend": "fused"},
    }


# the C=32 cell: kernels 4x9, fc1 256x128 + 256, fc2 32x256 + 32, a 2-class head on 4 channels
N_PARAMS = 36 + 256 * 128 + 256 + 32 * 256 + 32 + 2 * 4 + 2


def _same_final(a, b):
    fa = torch.load(a / "final.pt", weights_only=True)["model"]
    fb = torch.load(b / "final.pt", weights_only=True)["model"]
    assert fa.keys() == fb.keys()
    for k in fa:
        assert torch.equal(fa[k], fb[k]), k


def test_train_fast_writes_the_run_files_and_resumes_exactly(tmp_path):
    out_a = tmp_path / "a"
    res = train_fast(_cfg(6), out_a, seed=0, quiet=True)
    assert "val_exact" in res
    for f in ("final.pt", "run.json", "log.jsonl", "summary.json", "checkpoint.pt"):
        assert (out_a / f).exists(), f
    recs = [json.loads(line) for line in open(out_a / "log.jsonl")]
    assert "iter_seconds" in recs[0] and "loss" in recs[0]
    run = json.loads((out_a / "run.json").read_text())
    assert run["engine"]["fused_chunk"] and run["params"] == N_PARAMS
    model, _ = load_model(out_a / "final.pt")
    assert sum(p.numel() for p in model.parameters()) == N_PARAMS
    # interrupted after 3 steps, then resumed: identical weights
    out_b = tmp_path / "b"
    train_fast(_cfg(3), out_b, seed=0, quiet=True)
    train_fast(_cfg(6), out_b, seed=0, quiet=True)
    _same_final(out_a, out_b)


def test_stop_at_step_keeps_the_schedule_and_resumes_exactly(tmp_path):
    cfg = _cfg(6, schedule="cosine", warmup_ratio=0.25)
    full, split = tmp_path / "full", tmp_path / "split"
    train_fast(cfg, full, quiet=True, resume=False)
    train_fast(cfg, split, quiet=True, resume=False, stop_at_step=2)
    partial = torch.load(split / "checkpoint.pt", weights_only=True)
    summary = json.loads((split / "summary.json").read_text())
    assert partial["step"] == summary["steps"] == 2
    assert summary["target_steps"] == 6 and not summary["training_complete"]
    with pytest.raises(ValueError, match="after the resumed"):
        train_fast(cfg, split, quiet=True, stop_at_step=2)
    train_fast(cfg, split, quiet=True, stop_at_step=6)
    _same_final(full, split)


def test_train_fast_with_step_noise_and_pool_swaps(tmp_path):
    """Step noise sends the chunk through the differentiable step; swaps from the pool, batch
    noise and the official damage geometry run too."""
    cfg = _cfg(4, noise={"p_t": 0.5, "p_s": 0.3, "sigma": 0.1}, swap_source="pool",
               batch_noise={"p": 0.5}, damage={"p": 0.5, "geometry": "official"})
    res = train_fast(cfg, tmp_path / "n", seed=1, quiet=True)
    run = json.loads((tmp_path / "n" / "run.json").read_text())
    assert not run["engine"]["fused_chunk"]
    recs = [json.loads(line) for line in open(tmp_path / "n" / "log.jsonl")]
    assert all(torch.isfinite(torch.tensor(r["loss"])) for r in recs if "loss" in r)
    assert 0.0 <= res["val_exact"] <= 1.0
