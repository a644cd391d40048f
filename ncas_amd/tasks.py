"""Boards and seeded input generators for the NCA workloads (host numpy).

`Boards` keeps the reference's container (reference src/nca/tasks/base.py:27-86): `(N, H, W)`
int64 `inputs` / `targets`, bool `given`, per-board `meta`.

Generators (the reference's own are pure-Python loops, reference src/nca/tasks/maze.py:317-445,
src/nca/tasks/sudoku.py:290-294):

* `maze_boards` - perfect mazes by randomised depth-first search (recursive backtracker) on a
  k x k lattice, drawn on a (2k+1) x (2k+1) grid (cropped to an even size like the reference's
  hard mazes), optionally with a fraction of the removable interior walls knocked out; start
  and goal on open cells (for hard mazes at BFS distance >= min_path_len - 1); targets mark the
  BFS shortest path. Tokens: OPEN=0, WALL=1, START=2, GOAL=3, PATH=4; given = walls, start,
  goal (the reference's `inputs != EMPTY`, maze.py:932).
* `sudoku_boards` - random valid solved grids (a valid base pattern under the validity-
  preserving symmetry group: digit relabelling, row / column permutations within bands /
  stacks, band / stack permutations, transposition) with a uniformly random number of clues
  in [17, 30] kept at uniformly random cells. Uniqueness of the solution is not required.
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field

import numpy as np

from .model import MAZE_GOAL, MAZE_OPEN, MAZE_PATH, MAZE_START, MAZE_WALL


@dataclass
class Boards:
    inputs: np.ndarray
    targets: np.ndarray
    given: np.ndarray
    meta: dict = field(default_factory=dict)

    def __post_init__(self) -> None:
        assert self.inputs.shape == self.targets.shape == self.given.shape, "shape mismatch"
        assert self.inputs.ndim == 3, "boards must be (N, H, W)"
        self.inputs = self.inputs.astype(np.int64)
        self.targets = self.targets.astype(np.int64)
        self.given = self.given.astype(bool)

    def __len__(self) -> int:
        return self.inputs.shape[0]

    @property
    def shape(self) -> tuple[int, int]:
        return self.inputs.shape[1], self.inputs.shape[2]

    def subset(self, idx) -> Boards:
        idx = np.asarray(idx)
        meta = {k: (v[idx] if isinstance(v, np.ndarray) and v.shape[:1] == (len(self),) else v)
                for k, v in self.meta.items()}
        return Boards(self.inputs[idx], self.targets[idx], self.given[idx], meta)

    def repeat(self, k: int) -> Boards:
        """Board n becomes rows n*k .. n*k+k-1 (reference tasks/base.py:66-77)."""
        n = len(self)
        meta = {key: (np.repeat(v, k, axis=0) if isinstance(v, np.ndarray) and v.shape[:1] == (n,)
                      else v) for key, v in self.meta.items()}
        return Boards(np.repeat(self.inputs, k, 0), np.repeat(self.targets, k, 0),
                      np.repeat(self.given, k, 0), meta)


# ---------------------------------------------------------------------------------- tasks
class Task:
    """What the rollout, the trainer and the metrics need to know about a board family
    (reference src/nca/tasks/base.py:89-149): given cells show their input token in decoded
    boards (`fill_given`), the scored cells are the mutable ones (`eval_mask`), "exact" is the
    main metric, and there is no augmentation."""

    name = "task"
    main_metric = "exact"
    fill_given = True

    def eval_mask(self, boards: Boards) -> np.ndarray:
        return ~boards.given

    def augment(self, boards: Boards, rng: np.random.Generator) -> Boards:
        return boards

    def metrics(self, pred: np.ndarray, boards: Boards) -> dict[str, np.ndarray]:
        """Per-board "exact" (every scored cell right) and "cell_acc" of predicted tokens
        (N, H, W)."""
        scored = self.eval_mask(boards)
        right = (pred == boards.targets) & scored
        n = scored.sum(axis=(1, 2))
        hits = right.sum(axis=(1, 2))
        return {"exact": hits == n, "cell_acc": hits / np.maximum(n, 1)}


class MazeTask(Task):
    """Mazes of `maze_boards` (open / wall / start / goal inputs, the BFS path as target)."""

    name = "maze"

    def __init__(self, extra_openings: float = 0.0, min_path_len: int | None = None):
        self.extra_openings, self.min_path_len = extra_openings, min_path_len

    def generate(self, n: int, size: int, seed: int) -> Boards:
        return maze_boards(n, size, seed, self.extra_openings, self.min_path_len)


class SudokuTask(Task):
    """Sudoku boards of `sudoku_boards` (clues as inputs, the solved grid as target)."""

    name = "sudoku"

    def __init__(self, clues: tuple[int, int] = (17, 30)):
        self.clues = tuple(clues)

    def generate(self, n: int, size: int, seed: int) -> Boards:
        if size != 9:
            raise ValueError("sudoku boards are 9x9")
        return sudoku_boards(n, seed, self.clues)


def get_task(name: str, **kwargs) -> Task:
    """"maze", "maze_hard" (10 % extra openings) or "sudoku"."""
    if name == "maze":
        return MazeTask(**kwargs)
    if name == "maze_hard":
        return MazeTask(**{"extra_openings": 0.10, **kwargs})
    if name == "sudoku":
        return SudokuTask(**kwargs)
    raise ValueError(f"unknown task {name!r} (maze | maze_hard | sudoku)")


# ---------------------------------------------------------------------------------- mazes
def carve_perfect_maze(k: int, rng: np.random.Generator) -> np.ndarray:
    """(2k+1, 2k+1) uint8 grid of WALL / OPEN: a spanning tree of the k x k lattice grown by
    randomised depth-first search (a neighbour drawn uniformly at every extension)."""
    grid = np.full((2 * k + 1, 2 * k + 1), MAZE_WALL, dtype=np.uint8)
    grid[1::2, 1::2] = MAZE_OPEN
    if k <= 1:
        return grid
    seen = np.zeros((k, k), dtype=bool)
    start = (int(rng.integers(k)), int(rng.integers(k)))
    seen[start] = True
    stack = [start]
    while stack:
        i, j = stack[-1]
        nbrs = [(i + di, j + dj) for di, dj in ((-1, 0), (1, 0), (0, -1), (0, 1))
                if 0 <= i + di < k and 0 <= j + dj < k and not seen[i + di, j + dj]]
        if not nbrs:
            stack.pop()
            continue
        ni, nj = nbrs[int(rng.integers(len(nbrs)))]
        seen[ni, nj] = True
        grid[i + ni + 1, j + nj + 1] = MAZE_OPEN  # the wall between (i, j) and (ni, nj)
        stack.append((ni, nj))
    return grid


def bfs(passable: np.ndarray, src: tuple[int, int]) -> tuple[np.ndarray, np.ndarray]:
    """Distances (-1 = unreachable) and BFS parents (flat index, -1) from src, neighbour order
    up, down, left, right."""
    H, W = passable.shape
    dist = np.full((H, W), -1, dtype=np.int64)
    parent = np.full((H, W), -1, dtype=np.int64)
    dist[src] = 0
    q = deque([src])
    while q:
        i, j = q.popleft()
        for di, dj in ((-1, 0), (1, 0), (0, -1), (0, 1)):
            a, b = i + di, j + dj
            if 0 <= a < H and 0 <= b < W and passable[a, b] and dist[a, b] < 0:
                dist[a, b] = dist[i, j] + 1
                parent[a, b] = i * W + j
                q.append((a, b))
    return dist, parent


def maze_boards(n: int, size: int, seed: int = 0, extra_openings: float = 0.0,
                min_path_len: int | None = None, max_tries: int = 1000) -> Boards:
    rng = np.random.default_rng(seed)
    k = size // 2
    inputs = np.zeros((n, size, size), np.int64)
    targets = np.zeros((n, size, size), np.int64)
    plen = np.zeros(n, np.int64)
    for b in range(n):
        for _ in range(max_tries):
            grid = carve_perfect_maze(k, rng)
            if extra_openings > 0:
                ii, jj = np.nonzero(grid == MAZE_WALL)
                inner = (ii > 0) & (jj > 0) & (ii < 2 * k) & (jj < 2 * k) & ((ii + jj) % 2 == 1)
                cand = np.stack([ii[inner], jj[inner]], 1)
                m = int(round(extra_openings * len(cand)))
                if m:
                    pick = cand[rng.choice(len(cand), size=m, replace=False)]
                    grid[pick[:, 0], pick[:, 1]] = MAZE_OPEN
            grid = np.ascontiguousarray(grid[:size, :size])
            passable = grid != MAZE_WALL
            free = np.argwhere(passable)
            src = tuple(int(v) for v in free[rng.integers(len(free))])
            dist, parent = bfs(passable, src)
            need = 1 if min_path_len is None else min_path_len - 1
            far = np.argwhere(dist >= need)
            if len(far) == 0:
                continue
            dst = tuple(int(v) for v in far[rng.integers(len(far))])
            tgt = grid.astype(np.int64)
            cur = dst[0] * size + dst[1]
            length = 1
            while parent.flat[cur] >= 0:
                cur = int(parent.flat[cur])
                tgt.flat[cur] = MAZE_PATH
                length += 1
            inp = grid.astype(np.int64)
            inp[src] = MAZE_START
            inp[dst] = MAZE_GOAL
            tgt[src] = MAZE_START
            tgt[dst] = MAZE_GOAL
            inputs[b], targets[b], plen[b] = inp, tgt, length
            break
        else:
            raise RuntimeError("could not generate a maze satisfying min_path_len")
    return Boards(inputs, targets, inputs != MAZE_OPEN, {"path_len": plen})


# ---------------------------------------------------------------------------------- sudoku
def random_solution(rng: np.random.Generator) -> np.ndarray:
    """A random valid solved 9x9 grid (values 1..9)."""
    r = np.arange(9)
    base = (3 * (r[:, None] % 3) + r[:, None] // 3 + r[None, :]) % 9  # valid Latin-box pattern
    rows = np.concatenate([3 * b + rng.permutation(3) for b in rng.permutation(3)])
    cols = np.concatenate([3 * s + rng.permutation(3) for s in rng.permutation(3)])
    g = base[rows][:, cols]
    if rng.integers(2):
        g = g.T
    return rng.permutation(9)[g] + 1


def is_valid_solution(grid: np.ndarray) -> bool:
    g = np.asarray(grid, dtype=np.int64).reshape(9, 9)
    if g.min() < 1 or g.max() > 9:
        return False
    full = set(range(1, 10))
    for k in range(9):
        box = g[3 * (k // 3): 3 * (k // 3) + 3, 3 * (k % 3): 3 * (k % 3) + 3]
        if set(g[k].tolist()) != full or set(g[:, k].tolist()) != full or set(box.ravel().tolist()) != full:
            return False
    return True


def sudoku_boards(n: int, seed: int = 0, clues: tuple[int, int] = (17, 30)) -> Boards:
    rng = np.random.default_rng(seed)
    sol = np.zeros((n, 9, 9), np.int64)
    inp = np.zeros((n, 9, 9), np.int64)
    for b in range(n):
        s = random_solution(rng)
        m = int(rng.integers(clues[0], clues[1] + 1))
        keep = rng.choice(81, size=m, replace=False)
        flat = np.zeros(81, np.int64)
        flat[keep] = s.ravel()[keep]
        sol[b], inp[b] = s, flat.reshape(9, 9)
    return Boards(inp, sol, inp != 0, {"n_clues": (inp != 0).sum((1, 2))})
