"""Input generators (the library's batched host code, no GPU needed): invariants of the seeded
mazes and Sudoku grids (reference src/nca/tasks/maze.py:251-309, 317-445 and
src/nca/tasks/sudoku.py:151, 290-294), independence from the thread count, and the on-disk
Boards format (maze.py:494-512)."""

from __future__ import annotations

import numpy as np
import pytest

from ncas_amd.model import MAZE_GOAL, MAZE_OPEN, MAZE_PATH, MAZE_START, MAZE_WALL
from ncas_amd.tasks import Boards, bfs, is_valid_solution, maze_boards, sudoku_boards


def _open_edges(passable):
    return int((passable[1:] & passable[:-1]).sum() + (passable[:, 1:] & passable[:, :-1]).sum())


@pytest.mark.parametrize("size", [13, 30])
def test_perfect_mazes_are_trees_with_a_shortest_path_target(size):
    b = maze_boards(6, size, seed=3)
    assert b.inputs.shape == (6, size, size)
    for n in range(6):
        inp, tgt = b.inputs[n], b.targets[n]
        passable = inp != MAZE_WALL
        # corridors of a recursive-backtracker maze form a spanning tree of the open cells
        assert _open_edges(passable) == passable.sum() - 1
        src = tuple(np.argwhere(inp == MAZE_START)[0])
        dst = tuple(np.argwhere(inp == MAZE_GOAL)[0])
        dist, _ = bfs(passable, src)
        assert (dist >= 0).sum() == passable.sum()  # connected
        on_path = (tgt == MAZE_PATH) | (tgt == MAZE_START) | (tgt == MAZE_GOAL)
        assert on_path.sum() == dist[dst] + 1 == b.meta["path_len"][n]
        # the path is a simple chain: the endpoints have one path neighbour, the rest two
        pad = np.pad(on_path, 1)
        nb = pad[:-2, 1:-1].astype(int) + pad[2:, 1:-1] + pad[1:-1, :-2] + pad[1:-1, 2:]
        ends = nb[on_path] == 1
        assert ends.sum() == (2 if dist[dst] > 0 else 0)
        # inputs show the maze without the path; given = everything but open cells
        assert np.array_equal(np.where(tgt == MAZE_PATH, MAZE_OPEN, tgt), inp)
        assert np.array_equal(b.given[n], inp != MAZE_OPEN)


def test_hard_mazes_have_loops_and_long_paths():
    b = maze_boards(4, 30, seed=5, extra_openings=0.1, min_path_len=20)
    for n in range(4):
        passable = b.inputs[n] != MAZE_WALL
        assert _open_edges(passable) > passable.sum() - 1
        assert b.meta["path_len"][n] >= 20


def test_maze_generator_is_seeded():
    a, b = maze_boards(3, 13, seed=9), maze_boards(3, 13, seed=9)
    assert np.array_equal(a.inputs, b.inputs) and np.array_equal(a.targets, b.targets)
    assert not np.array_equal(a.inputs, maze_boards(3, 13, seed=10).inputs)


def test_sudoku_boards_are_valid_with_17_to_30_clues():
    b = sudoku_boards(64, seed=1)
    counts = b.given.reshape(64, -1).sum(1)
    assert counts.min() >= 17 and counts.max() <= 30 and len(set(counts.tolist())) > 5
    for n in range(64):
        assert is_valid_solution(b.targets[n])
        assert np.array_equal(b.inputs[n][b.given[n]], b.targets[n][b.given[n]])
        assert np.all(b.inputs[n][~b.given[n]] == 0)
    assert np.array_equal(sudoku_boards(8, seed=1).targets, b.targets[:8])


def test_is_valid_solution_rejects_broken_grids():
    g = sudoku_boards(1, seed=2).targets[0].copy()
    assert is_valid_solution(g)
    g[0, 0], g[0, 1] = g[0, 1], g[0, 0]
    assert not is_valid_solution(g)
    assert not is_valid_solution(np.zeros((9, 9), np.int64))


def test_boards_repeat_is_board_major():
    b = sudoku_boards(3, seed=4)
    r = b.repeat(4)
    assert len(r) == 12
    for n in range(3):
        for t in range(4):
            assert np.array_equal(r.inputs[n * 4 + t], b.inputs[n])
    assert np.array_equal(r.meta["n_clues"], np.repeat(b.meta["n_clues"], 4))
    s = b.subset([2, 0])
    assert np.array_equal(s.targets, b.targets[[2, 0]])
    with pytest.raises(AssertionError):
        Boards(b.inputs, b.targets[:2], b.given)


def test_generators_do_not_depend_on_the_thread_count():
    a = maze_boards(24, 21, seed=7, extra_openings=0.1, threads=1)
    b = maze_boards(24, 21, seed=7, extra_openings=0.1, threads=5)
    assert np.array_equal(a.inputs, b.inputs) and np.array_equal(a.targets, b.targets)
    assert np.array_equal(a.meta["path_len"], b.meta["path_len"])
    s1, s2 = sudoku_boards(40, seed=3, threads=1), sudoku_boards(40, seed=3, threads=8)
    assert np.array_equal(s1.inputs, s2.inputs) and np.array_equal(s1.targets, s2.targets)
    # a board depends only on (seed, index): the first boards of a larger set are the same
    assert np.array_equal(maze_boards(5, 21, seed=7, extra_openings=0.1).inputs, a.inputs[:5])


def test_large_batches_of_hard_mazes():
    b = maze_boards(1000, 30, seed=0, extra_openings=0.10)
    assert b.inputs.shape == (1000, 30, 30)
    assert (b.meta["path_len"] >= 2).all() and (b.inputs == MAZE_START).sum() == 1000
    big = maze_boards(2, 201, seed=1)
    passable = big.inputs[0] != MAZE_WALL
    assert _open_edges(passable) == passable.sum() - 1


def test_boards_save_load_and_task_cache(tmp_path):
    from ncas_amd.tasks import get_task

    b = maze_boards(7, 13, seed=2)
    b.save(tmp_path / "m.npz")
    c = Boards.load(tmp_path / "m.npz")
    assert np.array_equal(c.inputs, b.inputs) and np.array_equal(c.given, b.given)
    assert np.array_equal(c.meta["path_len"], b.meta["path_len"])
    task = get_task("maze_hard")
    first = task.load("train", tmp_path, n=6, size=30, seed=4)
    path = task.cache_path(tmp_path, "train", 6, 30, 4)
    assert path.endswith(".npz") and (tmp_path / path.split("/")[-1]).exists()
    again = task.load("train", tmp_path, n=6, size=30, seed=4)
    assert np.array_equal(first.targets, again.targets)
    s = get_task("sudoku").load("val", tmp_path, n=5, size=9, seed=1)
    assert np.array_equal(s.meta["n_clues"], s.given.sum(axis=(1, 2)))
