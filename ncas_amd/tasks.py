"""Boards, tasks and batched seeded input generators for the NCA workloads.

`Boards` is the reference's board container (reference src/nca/tasks/base.py:27-86): `(N, H, W)`
int64 `inputs` / `targets`, bool `given`, per-board `meta` arrays. `Boards.save` / `Boards.load`
keep a set on disk as an uncompressed-or-compressed `.npz` with the keys `inputs`, `targets`,
`given` and the per-board meta arrays (the reference's cached datasets, maze.py:494-512), read
back without unpickling.

Generators (the reference's are per-board Python loops, maze.py:317-445, sudoku.py:290-294) run
in the library's native code on all host threads, one counter-based random stream per board, so
a board depends only on (seed, board index):

* `maze_boards` - perfect mazes by randomised depth-first search (recursive backtracker) on a
  k x k lattice, drawn on a (2k+1) x (2k+1) grid (cropped to an even size like the reference's
  hard mazes), optionally with a fraction of the interior walls between two lattice cells
  knocked out; start and goal on open cells (for hard mazes at BFS distance >= min_path_len - 1);
  targets mark the BFS shortest path. Tokens: OPEN=0, WALL=1, START=2, GOAL=3, PATH=4;
  given = walls, start, goal (the reference's `inputs != EMPTY`, maze.py:932).
* `sudoku_boards` - random valid solved grids (a valid base pattern under the validity-
  preserving symmetries: digit relabelling, row / column permutations within bands / stacks,
  band / stack permutations, transposition) with a uniformly random number of clues in
  [17, 30] kept at uniformly random cells. Uniqueness of the solution is not required.

`Task` objects (`get_task`) give the scored cells, the metrics and `load(split, root, n, size,
seed)`, which reads a cached `.npz` or generates and caches the set. Metrics are computed on the
GPU for every (board, trial) row: "exact" and "cell_acc" for every task, plus the mazes' path
"valid" / "optimal" (`nca_maze_metrics`) and Sudoku's "valid" (`nca_sudoku_valid`).
"""

from __future__ import annotations

import ctypes
import os
from collections import deque
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib
from .model import MAZE_GOAL, MAZE_OPEN, MAZE_PATH, MAZE_START, MAZE_WALL


@dataclass
class Boards:
    inputs: np.ndarray
    targets: np.ndarray
    given: np.ndarray
    meta: dict = field(default_factory=dict)

    def __post_init__(self) -> None:
        shapes = {np.shape(self.inputs), np.shape(self.targets), np.shape(self.given)}
        if len(shapes) != 1 or len(next(iter(shapes))) != 3:
            raise AssertionError(f"boards must share one (N, H, W) shape, got {shapes}")
        self.inputs = np.asarray(self.inputs).astype(np.int64, copy=False)
        self.targets = np.asarray(self.targets).astype(np.int64, copy=False)
        self.given = np.asarray(self.given).astype(bool, copy=False)

    def __len__(self) -> int:
        return len(self.inputs)

    @property
    def shape(self) -> tuple[int, int]:
        return tuple(self.inputs.shape[1:])

    def _per_board(self, fn) -> dict:
        """The meta dict with `fn` applied to the per-board arrays (first dimension N)."""
        n = len(self)
        return {k: fn(v) if isinstance(v, np.ndarray) and len(v) == n and v.ndim else v
                for k, v in self.meta.items()}

    def subset(self, idx) -> Boards:
        idx = np.asarray(idx)
        return Boards(self.inputs[idx], self.targets[idx], self.given[idx],
                      self._per_board(lambda v: v[idx]))

    def repeat(self, k: int) -> Boards:
        """Board n becomes rows n*k .. n*k + k - 1 (reference tasks/base.py:66-77)."""
        rep = lambda v: np.repeat(v, k, axis=0)  # noqa: E731
        return Boards(rep(self.inputs), rep(self.targets), rep(self.given), self._per_board(rep))

    def save(self, path) -> None:
        """Write the set as an .npz (inputs, targets, given and the per-board meta arrays)."""
        arrays = {"inputs": self.inputs, "targets": self.targets, "given": self.given}
        arrays.update({k: v for k, v in self._per_board(lambda v: v).items()
                       if isinstance(v, np.ndarray)})
        np.savez_compressed(path, **arrays)

    @classmethod
    def load(cls, path) -> Boards:
        with np.load(path, allow_pickle=False) as z:
            meta = {k: z[k] for k in z.files if k not in ("inputs", "targets", "given")}
            return cls(z["inputs"], z["targets"], z["given"], meta)


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

    def generate(self, n: int, size: int, seed: int) -> Boards:
        raise NotImplementedError

    def cache_path(self, root, split: str, n: int, size: int, seed: int) -> str:
        return os.path.join(root, f"{self.name}_{split}_{size}_n{n}_seed{seed}.npz")

    def load(self, split: str, root, n: int, size: int, seed: int = 0) -> Boards:
        """The split's boards from `root`'s cached .npz, generated and cached on a miss
        (reference tasks/maze.py:505-512)."""
        path = self.cache_path(root, split, n, size, seed)
        if os.path.exists(path):
            return Boards.load(path)
        boards = self.generate(n, size, seed)
        os.makedirs(root, exist_ok=True)
        boards.save(path)
        return boards

    def device_metrics(self, pred: torch.Tensor, inputs: torch.Tensor, targets: torch.Tensor,
                       given: torch.Tensor, scored: torch.Tensor, k: int = 1
                       ) -> dict[str, torch.Tensor]:
        """Per-row metrics of decoded boards on the GPU: pred (rows, H, W) int64 tokens; inputs,
        targets (boards, H, W) int64, given and scored (boards, H, W) bool, with row r on board
        r // k. "exact": every scored cell right; "cell_acc": the fraction of scored cells right
        (reference tasks/base.py:126-149)."""
        B, H, W = targets.shape
        right = (pred.view(B, k, H, W) == targets[:, None]) & scored[:, None]
        hits = right.sum(dim=(2, 3))
        n = scored.sum(dim=(1, 2))[:, None]
        return {"exact": (hits == n).view(-1), "cell_acc": (hits / n.clamp_min(1)).view(-1)}

    def metrics(self, pred, boards: Boards, k: int = 1) -> dict[str, np.ndarray]:
        """The metrics of decoded boards pred (len(boards) * k, H, W), row r scored against board
        r // k (the reference's `metrics(pred, boards)` for k = 1), computed on the current GPU
        with one copy of the results to the host."""
        dev = torch.device("cuda", torch.cuda.current_device())
        bt = self.board_tensors(boards, dev)
        p = torch.as_tensor(pred)
        p = (p if p.is_cuda else _lib.upload(np.ascontiguousarray(p.numpy()), dev)).to(torch.int64)
        out = self.device_metrics(p.reshape(-1, *boards.shape).contiguous(), *bt, k=k)
        host = {name: v.cpu().numpy() for name, v in out.items()}
        return host

    def board_tensors(self, boards: Boards, device) -> tuple[torch.Tensor, ...]:
        """(inputs, targets, given, scored) of `boards` on the device."""
        up = lambda a: _lib.upload(np.ascontiguousarray(a), device)  # noqa: E731
        return (up(boards.inputs), up(boards.targets), up(boards.given),
                up(np.asarray(self.eval_mask(boards), dtype=bool)))


class MazeTask(Task):
    """Mazes of `maze_boards` (open / wall / start / goal inputs, the BFS path as target).

    Metrics add "valid" (the decoded path cells plus the two endpoints form one simple
    4-connected path between the endpoints) and "optimal" (valid and as long as the target path)
    of reference tasks/maze.py:843-866, computed by `nca_maze_metrics`. `path_token` and
    `endpoint_tokens` name the vocabulary: this build's maze tokens by default, the reference's
    (PATH 1, ENDPOINT 3) for its Maze-OOD boards."""

    name = "maze"
    path_token = MAZE_PATH
    endpoint_tokens = (MAZE_START, MAZE_GOAL)

    def __init__(self, extra_openings: float = 0.0, min_path_len: int | None = None,
                 path_token: int | None = None, endpoint_tokens: tuple[int, ...] | None = None):
        self.extra_openings, self.min_path_len = extra_openings, min_path_len
        if extra_openings:
            self.name = f"maze_x{extra_openings:g}"
        if path_token is not None:
            self.path_token = int(path_token)
        if endpoint_tokens is not None:
            self.endpoint_tokens = tuple(int(t) for t in endpoint_tokens)
        if not 1 <= len(self.endpoint_tokens) <= 2:
            raise ValueError("endpoint_tokens: one or two tokens")

    def generate(self, n: int, size: int, seed: int) -> Boards:
        return maze_boards(n, size, seed, self.extra_openings, self.min_path_len)

    def device_metrics(self, pred, inputs, targets, given, scored, k: int = 1):
        out = super().device_metrics(pred, inputs, targets, given, scored, k)
        rows, H, W = pred.shape
        valid = torch.empty(rows, dtype=torch.uint8, device=pred.device)
        optimal = torch.empty_like(valid)
        ends = self.endpoint_tokens + self.endpoint_tokens[-1:]
        g8 = given.to(torch.uint8).contiguous()
        _lib.check(_lib.load().nca_maze_metrics(
            pred.data_ptr(), inputs.contiguous().data_ptr(), targets.contiguous().data_ptr(),
            g8.data_ptr(), rows, int(k), H, W, int(self.path_token), int(ends[0]), int(ends[1]),
            valid.data_ptr(), optimal.data_ptr(), _lib.stream_of(pred.device)),
            "nca_maze_metrics")
        out["valid"], out["optimal"] = valid.bool(), optimal.bool()
        return out


class SudokuTask(Task):
    """Sudoku boards of `sudoku_boards` (clues as inputs, the solved grid as target). Metrics add
    "valid" (the grid filled with the clues satisfies every row, column and box constraint,
    reference tasks/sudoku.py:987-995), computed by `nca_sudoku_valid`."""

    name = "sudoku"

    def __init__(self, clues: tuple[int, int] = (17, 30)):
        self.clues = tuple(clues)

    def generate(self, n: int, size: int, seed: int) -> Boards:
        if size != 9:
            raise ValueError("sudoku boards are 9x9")
        return sudoku_boards(n, seed, self.clues)

    def device_metrics(self, pred, inputs, targets, given, scored, k: int = 1):
        out = super().device_metrics(pred, inputs, targets, given, scored, k)
        rows, H, W = pred.shape
        if (H, W) != (9, 9):
            raise ValueError("sudoku boards are 9x9")
        valid = torch.empty(rows, dtype=torch.uint8, device=pred.device)
        g8 = given.to(torch.uint8).contiguous()
        _lib.check(_lib.load().nca_sudoku_valid(
            pred.data_ptr(), inputs.contiguous().data_ptr(), g8.data_ptr(), rows, int(k),
            valid.data_ptr(), _lib.stream_of(pred.device)), "nca_sudoku_valid")
        out["valid"] = valid.bool()
        return out


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
def _threads(threads: int | None) -> int:
    return 0 if threads is None else int(threads)


def maze_boards(n: int, size: int, seed: int = 0, extra_openings: float = 0.0,
                min_path_len: int | None = None, max_tries: int = 1000,
                threads: int | None = None) -> Boards:
    """`n` seeded mazes of `size` x `size` (native code, `threads` host threads, all by default).
    meta["path_len"] is the number of cells on the shortest path, both ends included."""
    inputs = np.empty((n, size, size), np.int64)
    targets = np.empty((n, size, size), np.int64)
    given = np.empty((n, size, size), np.uint8)
    plen = np.empty(n, np.int64)
    P = ctypes.c_void_p
    _lib.check(_lib.load().nca_maze_boards(
        int(n), int(size), int(seed) & 0xFFFFFFFFFFFFFFFF, float(extra_openings),
        int(min_path_len or 0), int(max_tries), P(inputs.ctypes.data), P(targets.ctypes.data),
        P(given.ctypes.data), P(plen.ctypes.data), _threads(threads)), "nca_maze_boards")
    return Boards(inputs, targets, given.astype(bool), {"path_len": plen})


def bfs(passable: np.ndarray, src: tuple[int, int]) -> tuple[np.ndarray, np.ndarray]:
    """Distances (-1 = unreachable) and BFS parents (flat index, -1) from src over passable
    cells, neighbour order up, down, left, right (reference maze.py:251-295 scores paths the
    same way)."""
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


# ---------------------------------------------------------------------------------- sudoku
def is_valid_solution(grid: np.ndarray) -> bool:
    """A solved 9x9 grid: every row, column and 3x3 box holds 1..9 once (reference
    sudoku.py:151)."""
    g = np.asarray(grid, dtype=np.int64).reshape(9, 9)
    if g.min() < 1 or g.max() > 9:
        return False
    boxes = g.reshape(3, 3, 3, 3).transpose(0, 2, 1, 3).reshape(9, 9)
    digits = np.arange(1, 10)
    return all(np.array_equal(np.sort(u, axis=1), np.tile(digits, (9, 1))) for u in (g, g.T, boxes))


def sudoku_boards(n: int, seed: int = 0, clues: tuple[int, int] = (17, 30),
                  threads: int | None = None) -> Boards:
    """`n` seeded Sudoku boards (native code): targets are valid solved grids, inputs keep a
    uniformly random number of clues in `clues` (inclusive) at uniformly random cells, 0 elsewhere;
    meta["n_clues"] is that number."""
    inputs = np.empty((n, 9, 9), np.int64)
    targets = np.empty((n, 9, 9), np.int64)
    given = np.empty((n, 9, 9), np.uint8)
    P = ctypes.c_void_p
    _lib.check(_lib.load().nca_sudoku_boards(
        int(n), int(seed) & 0xFFFFFFFFFFFFFFFF, int(clues[0]), int(clues[1]),
        P(inputs.ctypes.data), P(targets.ctypes.data), P(given.ctypes.data), _threads(threads)),
        "nca_sudoku_boards")
    g = given.astype(bool)
    return Boards(inputs, targets, g, {"n_clues": g.sum(axis=(1, 2))})
