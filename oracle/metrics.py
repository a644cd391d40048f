"""Task metrics of decoded boards restated in numpy (oracle: test infrastructure only).

Maze "valid" / "optimal" (reference src/nca/tasks/maze.py:843-866 with path_validity at
maze.py:251-295): the predicted path P is the decoded path-token cells that are not given plus
the inputs' endpoint cells. P is valid when the inputs hold exactly two endpoint cells, both
have exactly one 4-neighbour in P, every other cell of P has exactly two, and P is connected.
The reference checks connectivity with the walk that those degrees force from one endpoint (it
must reach the other after visiting all of P); here connectivity is a breadth-first search over
P, so the restatement does not share the walk with the GPU kernel. Under the degree conditions
the two are the same test: the component of an endpoint is a path ending at the only other
degree-one cell, so the walk visits exactly that component. "optimal": valid and |P| equal to
the target's path-token cells plus the endpoints.

Sudoku "valid" (reference src/nca/tasks/sudoku.py:151-164, 987-995): the grid with the inputs on
the given cells and the decode elsewhere holds each of 1..9 exactly once in every row, column
and 3x3 box (so no value outside 1..9).
"""

from __future__ import annotations

from collections import deque

import numpy as np


def path_cells(pred, inputs, given, path_token: int, endpoint_tokens) -> np.ndarray:
    """(H, W) bool: the predicted path cells plus the endpoint cells."""
    ends = np.isin(inputs, endpoint_tokens)
    return ((np.asarray(pred) == path_token) & ~np.asarray(given, dtype=bool)) | ends


def path_valid(mask: np.ndarray, ends: list[tuple[int, int]]) -> bool:
    """Is `mask` one simple 4-connected path between the two cells of `ends`?"""
    m = np.asarray(mask, dtype=bool)
    if len(ends) != 2 or ends[0] == ends[1]:
        return False
    H, W = m.shape
    cells = list(zip(*np.nonzero(m)))

    def nbrs(i, j):
        for a, b in ((i - 1, j), (i + 1, j), (i, j - 1), (i, j + 1)):
            if 0 <= a < H and 0 <= b < W and m[a, b]:
                yield a, b

    deg = {c: sum(1 for _ in nbrs(*c)) for c in cells}
    if any(not m[e] for e in ends):
        return False
    ones = [c for c in cells if deg[c] == 1]
    if sorted(ones) != sorted(ends) or any(deg[c] not in (1, 2) for c in cells):
        return False
    seen = {ends[0]}
    q = deque([ends[0]])
    while q:
        for nb in nbrs(*q.popleft()):
            if nb not in seen:
                seen.add(nb)
                q.append(nb)
    return len(seen) == len(cells)


def maze_metrics(pred, inputs, targets, given, path_token: int, endpoint_tokens
                 ) -> tuple[np.ndarray, np.ndarray]:
    """(valid, optimal) bool arrays over the boards of pred / inputs / targets / given
    (N, H, W)."""
    pred, inputs, targets = (np.asarray(a) for a in (pred, inputs, targets))
    N = len(pred)
    valid = np.zeros(N, bool)
    optimal = np.zeros(N, bool)
    for n in range(N):
        m = path_cells(pred[n], inputs[n], given[n], path_token, endpoint_tokens)
        ends = [tuple(int(v) for v in e) for e in np.argwhere(np.isin(inputs[n], endpoint_tokens))]
        valid[n] = path_valid(m, ends)
        ref_len = int((targets[n] == path_token).sum()) + len(ends)
        optimal[n] = valid[n] and int(m.sum()) == ref_len
    return valid, optimal


def sudoku_valid(pred, inputs, given) -> np.ndarray:
    """(N,) bool: the filled grids satisfy every Sudoku constraint."""
    g = np.where(np.asarray(given, dtype=bool), inputs, pred).reshape(-1, 9, 9)
    out = np.zeros(len(g), bool)
    want = np.arange(1, 10)
    for n, grid in enumerate(g):
        units = [grid[i, :] for i in range(9)] + [grid[:, j] for j in range(9)]
        units += [grid[r:r + 3, c:c + 3].ravel() for r in (0, 3, 6) for c in (0, 3, 6)]
        out[n] = all(np.array_equal(np.sort(u), want) for u in units)
    return out
