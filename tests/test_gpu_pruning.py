"""Niche-capped pruning on the GPU through the C ABI (nca_prune_select) and the pruned rollout.

* The selection equals the oracle's (oracle/pruning.py, the reference's rule with the same
  Philox niche order) bit for bit on boards with few distinct decoded boards (large niches),
  tied confidences, dead trials, several n_cap and events, and K up to 256; the reference's
  known answers (tests/test_model.py:165-177).
* rollout() with pruning (reference tests/test_rollout.py:74-95, 202-225): the ensemble halves at
  every pruning step and the batch shrinks (16 -> 8 -> 4 -> 2 rows), pruned trajectories keep
  their last decode and stop counting updates; the whole pruned rollout equals the oracle's
  composition (fp32 steps, C readout, numpy pruning with the same renumbered Philox rows).
"""

from __future__ import annotations

import copy
import sys

import numpy as np
import pytest
import torch

sys.path.insert(0, __file__.rsplit("/", 1)[0])
from cells import DYN, oracle_cell, perturbed_model  # noqa: E402

import ncas_amd.rollout as R  # noqa: E402
from ncas_amd.pruning import prune_select  # noqa: E402
from ncas_amd.tasks import MazeTask, maze_boards  # noqa: E402
from oracle import clib  # noqa: E402
from oracle import nca_oracle as O  # noqa: E402
from oracle.pruning import niche_capped_pruning  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    clib.build()


def test_known_answers():
    dec = torch.zeros(1, 8, 2, 2, dtype=torch.long)
    dec[0, 4:] = 1
    conf = torch.tensor([[0.9, 0.8, 0.7, 0.6, 0.5, 0.4, 0.3, 0.2]])
    new = prune_select(dec.to(DEV), conf.to(DEV), torch.ones(1, 8, dtype=torch.bool, device=DEV), 3, 0, 0)
    new = new.cpu()
    assert new.sum() == 4 and new[0, :4].sum() == 2 and new[0, 4:].sum() == 2
    assert new[0, 0] and new[0, 4]


@pytest.mark.parametrize("N,K,cells,patterns", [(40, 8, 4, 3), (30, 64, 81, 5), (6, 256, 9, 12), (3, 128, 900, 2)])
def test_selection_matches_oracle(N, K, cells, patterns):
    rng = np.random.default_rng(N * K)
    pat = rng.integers(0, 5, size=(patterns, cells))
    which = rng.integers(0, patterns, size=(N, K))
    dec = pat[which].astype(np.int32)
    dec[rng.random((N, K)) < 0.1, 0] = 7  # a few singletons
    conf = (rng.integers(0, 8, size=(N, K)) / 8).astype(np.float32)
    alive = rng.random((N, K)) < 0.85
    alive[0] = False
    alive[1] = False
    alive[1, 3] = True  # one alive trial: unchanged
    for n_cap, seed, event in ((1, 0, 0), (3, 2**40 + 7, 5), (4, 11, 2**31)):
        got = prune_select(torch.from_numpy(dec).to(DEV), torch.from_numpy(conf).to(DEV),
                           torch.from_numpy(alive).to(DEV), n_cap, seed, event).cpu().numpy()
        ref = niche_capped_pruning(dec, conf, alive, n_cap, seed, event)
        assert np.array_equal(got, ref), (n_cap, seed, event)


def _model():
    m = perturbed_model("maze_c16", 0, *DYN["maze_c16"])
    return m, copy.deepcopy(m).to(DEV)


def test_pruned_rollout_halves_and_compacts(monkeypatch):
    m, md = _model()
    b = maze_boards(2, 9, 0)
    seen = []
    orig = R.rollout_steps

    def spy(model, x, *a, **kw):
        seen.append((x.shape[0], a[2] if len(a) > 2 else kw.get("n_steps")))
        return orig(model, x, *a, **kw)

    monkeypatch.setattr(R, "rollout_steps", spy)
    rc = R.RolloutConfig(depth=8, k=8, pruning={"m": 4, "n_cap": 3}, record_every=2)
    res = R.rollout(md, MazeTask(), b, rc, seed=0)
    assert [s[0] for s in seen] == [16, 8, 4, 2]  # rows of the launches after each halving
    assert res.alive.sum(axis=1).tolist() == [1, 1]
    assert res.pred.shape == (2, 8, 9, 9) and np.isfinite(res.conf).all()
    dead = ~res.alive
    assert (res.cell_updates[dead] < res.cell_updates[res.alive].min()).all()
    assert res.trace_exact.shape == (2, 8, 4) and (res.trace_updates[..., -1] > 0).all()
    monkeypatch.setattr(R, "rollout_steps", orig)
    rc = R.RolloutConfig(depth=8, k=4, pruning={"m": 4, "n_cap": 3}, record_every=2)
    res = R.rollout(md, MazeTask(), maze_boards(3, 9, 1), rc, seed=0)
    assert res.alive.sum(axis=1).tolist() == [1, 1, 1]  # 4 -> 2 -> 1 -> 1


def test_pruned_rollout_matches_the_oracle_composition():
    """fp32, 3 boards x 8 trials, depth 12, pruning at steps 4 and 8: the alive sets, the decoded
    boards and the confidences (within 1e-5) of every (board, trial) equal the oracle's
    composition of the same segments."""
    m, md = _model()
    cell = oracle_cell(m)
    b = maze_boards(3, 9, 2)
    N, K, (H, W) = 3, 8, b.shape
    rc = R.RolloutConfig(depth=12, k=K, pruning={"m": 3, "n_cap": 2}, fire_rate=0.5)
    res = R.rollout(md, MazeTask(), b, rc, seed=4)
    # oracle: the same flow on the CPU
    inputs = torch.from_numpy(np.repeat(b.inputs, K, 0))
    given = torch.from_numpy(np.repeat(b.given, K, 0))
    clamp = md.clamp_values(inputs.to(DEV)).cpu()
    x = md.apply_clamp(torch.zeros(N * K, 16, H, W, device=DEV), given[:, None].to(DEV),
                       clamp.to(DEV)).cpu()
    tokens = np.array(m.cfg.output_tokens)
    idx = np.arange(N * K)
    alive = np.ones(N * K, bool)
    pred = np.zeros((N * K, H, W), np.int64)
    conf_o = np.zeros(N * K, np.float32)
    t, event = 0, 0
    g4 = given[:, None]

    def decode(xs, rows):
        cc, cb, am = O.readout(cell, xs)
        d = np.where(given[rows].numpy(), inputs[rows].numpy(), tokens[am])
        return d, cb

    for stop in (4, 8, 12):
        x, _ = O.rollout(cell, x, g4[idx], clamp[idx], stop - t, "fp32", seed=4, row0=0, step0=t,
                         p_fire=0.5)
        t = stop
        d, cb = decode(x, idx)
        if stop < 12:
            dfull = np.zeros((N * K, H, W), np.int64)
            cfull = np.full(N * K, -np.inf, np.float32)
            afull = np.zeros(N * K, bool)
            dfull[idx], cfull[idx], afull[idx] = d, cb, True
            keep = niche_capped_pruning(dfull.reshape(N, K, -1), cfull.reshape(N, K),
                                        afull.reshape(N, K), 2, 4, event).reshape(-1)[idx]
            event += 1
            pred[idx[~keep]], conf_o[idx[~keep]] = d[~keep], cb[~keep]
            alive[idx[~keep]] = False
            x, idx = x[torch.from_numpy(keep)], idx[keep]
    pred[idx], conf_o[idx] = d, cb
    assert np.array_equal(res.alive.reshape(-1), alive)
    assert np.array_equal(res.pred.reshape(N * K, H, W), pred)
    assert np.abs(res.conf.reshape(-1) - conf_o).max() <= 1e-5
