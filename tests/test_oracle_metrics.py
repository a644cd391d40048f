"""The oracle's task metrics pinned on hand-built boards whose verdict is fixed by the definition
(reference src/nca/tasks/maze.py:251-295, 843-866; src/nca/tasks/sudoku.py:151-164, 987-995),
on the generators' targets (shortest paths and solved grids, valid by construction), and
against this package's host `is_valid_solution`."""

from __future__ import annotations

import numpy as np
import pytest

from ncas_amd.model import MAZE_GOAL, MAZE_OPEN, MAZE_PATH, MAZE_START, MAZE_WALL
from ncas_amd.tasks import bfs, is_valid_solution, maze_boards, sudoku_boards
from oracle import metrics as OM

ENDS = (MAZE_START, MAZE_GOAL)


def _open(h=5, w=5, start=(0, 0), goal=(0, 4), path=((0, 1), (0, 2), (0, 3))):
    inputs = np.full((h, w), MAZE_OPEN, np.int64)
    inputs[start], inputs[goal] = MAZE_START, MAZE_GOAL
    targets = inputs.copy()
    for c in path:
        targets[c] = MAZE_PATH
    return inputs, targets, inputs != MAZE_OPEN


def _pred(inputs, cells):
    p = inputs.copy()
    for c in cells:
        p[c] = MAZE_PATH
    return p


def _score(inputs, targets, given, pred):
    v, o = OM.maze_metrics(pred[None], inputs[None], targets[None], given[None], MAZE_PATH, ENDS)
    return bool(v[0]), bool(o[0])


STRAIGHT = [(0, 1), (0, 2), (0, 3)]
DETOUR = [(1, 0), (1, 1), (1, 2), (1, 3), (1, 4)]


@pytest.mark.parametrize("cells,want", [
    (STRAIGHT, (True, True)),                              # the target path itself
    (DETOUR, (True, False)),                               # valid, 7 cells against 5
    (STRAIGHT + [(3, 1), (3, 2), (4, 1), (4, 2)], (False, False)),  # plus a detached 2x2 cycle
    ([(0, 1), (0, 3)], (False, False)),                    # a gap: four cells of degree one
    (STRAIGHT + [(1, 2)], (False, False)),                 # a spur: degree three
    (STRAIGHT + [(1, 1), (1, 2), (1, 3)], (False, False)), # a path two cells wide
    ([], (False, False)),                                  # no path cells
    (STRAIGHT + [(4, 4)], (False, False)),                 # an isolated cell: degree zero
])
def test_maze_hand_built(cells, want):
    inputs, targets, given = _open()
    assert _score(inputs, targets, given, _pred(inputs, cells)) == want


def test_maze_endpoint_rules():
    # adjacent endpoints and no path cells: a valid two-cell path, optimal when the target agrees
    inputs, targets, given = _open(start=(2, 2), goal=(2, 3), path=())
    assert _score(inputs, targets, given, inputs.copy()) == (True, True)
    # a path through an endpoint: that endpoint has degree two
    inputs, targets, given = _open(start=(0, 2), goal=(0, 4), path=((0, 3),))
    assert _score(inputs, targets, given, _pred(inputs, [(0, 1), (0, 3)])) == (False, False)
    # three endpoint cells
    inputs, targets, given = _open()
    inputs[4, 4] = MAZE_START
    assert _score(inputs, targets, given, _pred(inputs, STRAIGHT)) == (False, False)
    # one endpoint cell only
    inputs, targets, given = _open()
    inputs[0, 4] = MAZE_OPEN
    assert _score(inputs, targets, given, _pred(inputs, STRAIGHT + [(0, 4)])) == (False, False)


def test_maze_given_cells_are_not_path():
    # a path token decoded on a given (wall) cell is not part of the predicted path
    inputs, targets, given = _open()
    inputs[1, 2] = MAZE_WALL
    given = inputs != MAZE_OPEN
    pred = _pred(inputs, STRAIGHT + [(1, 2)])
    assert _score(inputs, targets, given, pred) == (True, True)


def test_maze_generated_targets_valid_and_optimal():
    for extra in (0.0, 0.1):
        b = maze_boards(40, 15, seed=3, extra_openings=extra)
        v, o = OM.maze_metrics(b.targets, b.inputs, b.targets, b.given, MAZE_PATH, ENDS)
        assert v.all() and o.all()


def test_maze_optimal_is_shortest_length():
    # a valid predicted path is optimal exactly when it has BFS distance + 1 cells
    rng = np.random.default_rng(0)
    b = maze_boards(30, 11, seed=5, extra_openings=0.3)
    for n in range(len(b)):
        inp, tgt = b.inputs[n], b.targets[n]
        s = tuple(np.argwhere(inp == MAZE_START)[0])
        g = tuple(np.argwhere(inp == MAZE_GOAL)[0])
        dist, _ = bfs(inp != MAZE_WALL, s)
        # a random simple walk from s to g: depth-first search in a random neighbour order
        free = inp != MAZE_WALL
        path, seen = [s], {s}

        def dfs(c):
            if c == g:
                return True
            nb = [(c[0] + a, c[1] + d) for a, d in ((-1, 0), (1, 0), (0, -1), (0, 1))]
            rng.shuffle(nb)
            for q in nb:
                if 0 <= q[0] < 11 and 0 <= q[1] < 11 and free[q] and q not in seen:
                    seen.add(q)
                    path.append(q)
                    if dfs(q):
                        return True
                    path.pop()
            return False

        assert dfs(s)
        pred = _pred(inp, [c for c in path if inp[c] == MAZE_OPEN])
        v, o = OM.maze_metrics(pred[None], inp[None], tgt[None], b.given[n][None], MAZE_PATH,
                               ENDS)
        mask = OM.path_cells(pred, inp, b.given[n], MAZE_PATH, ENDS)
        # an induced simple path is valid; its optimality is its length
        if v[0]:
            assert o[0] == (int(mask.sum()) == dist[g] + 1)
        else:
            # a walk that is not an induced path has two non-consecutive cells side by side
            pos = {c: i for i, c in enumerate(path)}
            assert any(abs(pos[c] - pos[q]) > 1 for c in path
                       for q in ((c[0] + 1, c[1]), (c[0], c[1] + 1)) if q in pos)


def _pattern_grid():
    i, j = np.meshgrid(np.arange(9), np.arange(9), indexing="ij")
    return (3 * (i % 3) + i // 3 + j) % 9 + 1


def test_sudoku_hand_built():
    g = _pattern_grid()
    none = np.zeros((9, 9), bool)
    assert OM.sudoku_valid(g[None], g[None], none[None])[0]
    latin = (np.add.outer(np.arange(9), np.arange(9)) % 9) + 1  # rows, columns ok; boxes not
    assert not OM.sudoku_valid(latin[None], latin[None], none[None])[0]
    bad = g.copy()
    bad[0, 0], bad[0, 1] = bad[0, 1], bad[0, 0]  # the row stays a permutation, columns break
    assert not OM.sudoku_valid(bad[None], bad[None], none[None])[0]
    for v in (0, 10):
        bad = g.copy()
        bad[4, 4] = v
        assert not OM.sudoku_valid(bad[None], bad[None], none[None])[0]
    # given cells take the input: a wrong decode on a clue does not matter, on a free cell it does
    given = np.zeros((9, 9), bool)
    given[0, 0] = True
    pred = g.copy()
    pred[0, 0] = 0
    assert OM.sudoku_valid(pred[None], g[None], given[None])[0]
    assert not OM.sudoku_valid(pred[None], g[None], none[None])[0]


def test_sudoku_against_host_check():
    b = sudoku_boards(50, seed=2)
    assert OM.sudoku_valid(b.targets, b.inputs, b.given).all()
    rng = np.random.default_rng(1)
    preds = b.targets.copy()
    for n in range(len(preds)):
        for _ in range(int(rng.integers(0, 3))):
            r, c = rng.integers(0, 9, size=2)
            preds[n, r, c] = rng.integers(0, 10)
    want = [is_valid_solution(np.where(b.given[n], b.inputs[n], preds[n])) for n in range(50)]
    assert list(OM.sudoku_valid(preds, b.inputs, b.given)) == want
    assert 0 < sum(want) < 50
