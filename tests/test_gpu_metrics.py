"""Task metrics, compact pruning and the rollout's result fields on the GPU, through the C ABI.

* `nca_maze_metrics` ("valid" / "optimal") and `nca_sudoku_valid` equal the oracle
  (oracle/metrics.py, pinned on hand-built boards) on every row: generated targets, targets
  with random cell flips, random paths, hand-built breaks, k_per_board > 1, ragged and 201x201
  grids, and the reference's Maze-OOD vocabulary.
* `nca_prune_select_rows` on a compacted batch equals `nca_prune_select` on the full layout.
* `rollout()` reports the task metrics of every (board, trial) (`RolloutResult.metrics`,
  `score_candidates`) equal to the oracle's on its decoded boards; `record_boards` keeps trial
  0's decoded board of the first boards at every record step (reference rollout.py:284-287);
  a depth shorter than the number of pruning rounds prunes nothing (reference rollout.py:249).
"""

from __future__ import annotations

import copy
import sys

import numpy as np
import pytest
import torch

sys.path.insert(0, __file__.rsplit("/", 1)[0])
from cells import DYN, perturbed_model  # noqa: E402

import ncas_amd.rollout as R  # noqa: E402
from ncas_amd.model import MAZE_GOAL, MAZE_OPEN, MAZE_PATH, MAZE_START  # noqa: E402
from ncas_amd.pruning import prune_select, prune_select_rows  # noqa: E402
from ncas_amd.tasks import Boards, MazeTask, SudokuTask, maze_boards, sudoku_boards  # noqa: E402
from oracle import metrics as OM  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
ENDS = (MAZE_START, MAZE_GOAL)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"


def _maze_preds(b: Boards, k: int, rng) -> np.ndarray:
    """k decodes per board: the target, flips of a few cells between OPEN and PATH, and a path
    of random walks."""
    N, H, W = b.inputs.shape
    out = np.repeat(b.targets, k, 0).copy()
    for r in range(N * k):
        kind = r % 4
        n = r // k
        if kind == 1:  # flip a few free cells
            for _ in range(int(rng.integers(1, 4))):
                i, j = rng.integers(0, H), rng.integers(0, W)
                if not b.given[n, i, j]:
                    out[r, i, j] = MAZE_PATH if out[r, i, j] != MAZE_PATH else MAZE_OPEN
        elif kind == 2:  # drop one path cell
            cells = np.argwhere(out[r] == MAZE_PATH)
            if len(cells):
                out[r][tuple(cells[rng.integers(len(cells))])] = MAZE_OPEN
        elif kind == 3:  # random PATH noise on free cells
            free = ~b.given[n]
            out[r][free & (rng.random((H, W)) < 0.3)] = MAZE_PATH
    return out


def _check_maze(b: Boards, preds: np.ndarray, k: int, task=None, path=MAZE_PATH, ends=ENDS):
    task = task or MazeTask()
    got = task.metrics(preds, b, k=k)
    rep = lambda a: np.repeat(a, k, 0)  # noqa: E731
    v, o = OM.maze_metrics(preds, rep(b.inputs), rep(b.targets), rep(b.given), path, ends)
    assert np.array_equal(got["valid"], v)
    assert np.array_equal(got["optimal"], o)
    exact = ((preds == rep(b.targets)) | rep(b.given)).all(axis=(1, 2))
    assert np.array_equal(got["exact"], exact)
    return v, o


@pytest.mark.parametrize("n,size,extra,k", [(64, 13, 0.0, 4), (40, 30, 0.1, 8), (6, 37, 0.1, 3),
                                            (4, 201, 0.0, 2)])
def test_maze_metrics_match_oracle(n, size, extra, k):
    rng = np.random.default_rng(size)
    b = maze_boards(n, size, seed=size, extra_openings=extra)
    preds = _maze_preds(b, k, rng)
    v, o = _check_maze(b, preds, k)
    assert v[::4].all() and o[::4].all()  # the targets
    assert (~v).any()  # some broken ones


def test_maze_metrics_hand_built_and_ragged():
    # the oracle's hand-built cases, on a ragged 5 x 7 grid: straight, detour, detached cycle,
    # gap, spur, wide path
    H, W = 5, 7
    inp = np.full((H, W), MAZE_OPEN, np.int64)
    inp[0, 0], inp[0, 6] = MAZE_START, MAZE_GOAL
    tgt = inp.copy()
    tgt[0, 1:6] = MAZE_PATH
    straight = [(0, j) for j in range(1, 6)]
    cases = [straight, [(1, j) for j in range(7)], straight + [(3, 1), (3, 2), (4, 1), (4, 2)],
             straight[:2] + straight[3:], straight + [(1, 3)],
             straight + [(1, j) for j in range(1, 6)], []]
    preds = []
    for cells in cases:
        p = inp.copy()
        for c in cells:
            p[c] = MAZE_PATH
        preds.append(p)
    n = len(preds)
    b = Boards(np.repeat(inp[None], n, 0), np.repeat(tgt[None], n, 0),
               np.repeat((inp != MAZE_OPEN)[None], n, 0))
    v, o = _check_maze(b, np.stack(preds), 1)
    assert list(v) == [True, True, False, False, False, False, False]
    assert list(o) == [True, False, False, False, False, False, False]


def test_maze_metrics_reference_vocabulary():
    # the reference's Maze-OOD tokens: EMPTY 0, PATH 1, WALL 2, ENDPOINT 3 (maze.py:71)
    b0 = maze_boards(20, 13, seed=9)
    remap = np.array([0, 2, 3, 3, 1])  # OPEN, WALL, START, GOAL, PATH -> the reference's
    b = Boards(remap[b0.inputs], remap[b0.targets], b0.given)
    rng = np.random.default_rng(2)
    preds = remap[_maze_preds(b0, 2, rng)]
    task = MazeTask(path_token=1, endpoint_tokens=(3,))
    v, _ = _check_maze(b, preds, 2, task=task, path=1, ends=(3,))
    assert v[::4].all()


def test_sudoku_valid_matches_oracle():
    rng = np.random.default_rng(0)
    b = sudoku_boards(64, seed=4)
    k = 3
    preds = np.repeat(b.targets, k, 0).copy()
    for r in range(len(preds)):
        if r % 3 == 1:
            i, j = rng.integers(0, 9, size=2)
            preds[r, i, j] = rng.integers(0, 11)
        elif r % 3 == 2:
            preds[r] = rng.integers(1, 10, size=(9, 9))
    got = SudokuTask().metrics(preds, b, k=k)
    want = OM.sudoku_valid(preds, np.repeat(b.inputs, k, 0), np.repeat(b.given, k, 0))
    assert np.array_equal(got["valid"], want)
    assert want[::3].all() and not want[2::3].any()


def test_prune_rows_equals_full_layout():
    rng = np.random.default_rng(5)
    N, K, cells = 12, 32, 20
    pat = rng.integers(0, 4, size=(4, cells))
    dec = pat[rng.integers(0, 4, size=(N, K))].astype(np.int32)
    conf = (rng.integers(0, 6, size=(N, K)) / 6).astype(np.float32)
    alive = rng.random((N, K)) < 0.7
    alive[0] = False
    alive[1] = False
    alive[1, 5] = True
    full = prune_select(torch.from_numpy(dec).to(DEV), torch.from_numpy(conf).to(DEV),
                        torch.from_numpy(alive).to(DEV), 2, 7, 3).cpu().numpy().reshape(-1)
    flat = np.nonzero(alive.reshape(-1))[0]
    keep = prune_select_rows(torch.from_numpy(dec.reshape(N * K, cells)[flat]).to(DEV),
                             torch.from_numpy(conf.reshape(-1)[flat]).to(DEV),
                             torch.from_numpy(flat).to(DEV), N, K, 2, 7, 3).cpu().numpy()
    assert np.array_equal(keep, full[flat])
    assert not full[~alive.reshape(-1)].any()


def _model():
    m = perturbed_model("maze_c16", 0, *DYN["maze_c16"])
    return copy.deepcopy(m).to(DEV)


def test_rollout_reports_task_metrics():
    md = _model()
    b = maze_boards(6, 13, seed=1)
    K = 4
    res = R.rollout(md, MazeTask(), b, R.RolloutConfig(depth=20, k=K), seed=3)
    N, _, H, W = res.pred.shape
    assert set(res.metrics) == {"exact", "cell_acc", "valid", "optimal"}
    flat = res.pred.reshape(N * K, H, W)
    rep = lambda a: np.repeat(a, K, 0)  # noqa: E731
    v, o = OM.maze_metrics(flat, rep(b.inputs), rep(b.targets), rep(b.given), MAZE_PATH, ENDS)
    assert np.array_equal(res.metrics["valid"].reshape(-1), v)
    assert np.array_equal(res.metrics["optimal"].reshape(-1), o)
    sc = R.score_candidates(MazeTask(), res, b)
    assert all(sc[k].shape == (N, K) for k in sc)
    # the same metrics from the decoded boards alone
    res.metrics = None
    again = R.score_candidates(MazeTask(), res, b)
    for name in ("exact", "valid", "optimal"):
        assert np.array_equal(again[name], sc[name])
    assert np.allclose(again["cell_acc"], sc["cell_acc"])
    # conf@K on any metric
    R.conf_at_k(sc["valid"], res.conf, res.alive, [1, 2, 4])


def test_record_boards_trace():
    md = _model()
    b = maze_boards(5, 11, seed=2)
    refs = [R.rollout(md, MazeTask(), b, R.RolloutConfig(depth=d, k=3), seed=1).pred[:, 0]
            for d in (4, 8, 12)]
    rc = R.RolloutConfig(depth=12, k=3, record_every=4, record_boards=3)
    res = R.rollout(md, MazeTask(), b, rc, seed=1)
    assert res.boards_trace.shape == (3, 3, 11, 11)
    for t in range(3):
        assert np.array_equal(res.boards_trace[:, t], refs[t][:3])
    # boards split over passes (max_cells: two boards a pass) and fewer boards than
    # record_boards: the missing boards stay zero
    rc2 = R.RolloutConfig(depth=12, k=3, record_every=4, record_boards=9, max_cells=3 * 121 * 2)
    res2 = R.rollout(md, MazeTask(), b, rc2, seed=1)
    assert res2.boards_trace.shape == (9, 3, 11, 11)
    for t in range(3):
        assert np.array_equal(res2.boards_trace[:5, t], refs[t])
    assert not res2.boards_trace[5:].any()


def test_short_depth_prunes_nothing():
    md = _model()
    b = maze_boards(2, 9, seed=0)
    res = R.rollout(md, MazeTask(), b, R.RolloutConfig(depth=3, k=8, pruning={"m": 4}), seed=0)
    assert res.alive.all()
