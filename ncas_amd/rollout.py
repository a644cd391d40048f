"""Inference over boards: K stochastic trials per board, D fused steps, conf@K selection.

`rollout(model, task, boards, rc, seed)` mirrors the reference's evaluation engine (reference
src/nca/rollout.py:85-305) for the features of the HIP path: depth, K trials flattened
board-major (row = board * K + trial, rollout.py:143-146), uniform or confidence-gated firing
(`p_low`, `tau`, `given_confident`), bf16 (`amp`), chunking by `max_cells`, traces every
`record_every` steps and the final decoded boards / board confidence / fired-cell counts.
Fire masks come from the Philox rule keyed on the global row index and step, so results do
not depend on `max_cells` or on where the trace boundaries fall. The steps between two trace
points run as one launch of the LDS-resident kernel (`inference.rollout_steps`).

Everything a rollout reports is computed on the GPU (decode, board confidence, the per-board
exact / cell-accuracy scores over `task.eval_mask`, fired-cell counts) and kept there until one
copy to the host at the end of the call (the reference copies at every record step,
rollout.py:277-288). Pruning (niche-capped halving of the K trials, reference rollout.py:
249-275) selects on the GPU and compacts the surviving rows. Test-time noise and damage are not
implemented and raise ValueError.

`conf_at_k` / `pass_at_k` are the reference's selection metrics (rollout.py:317-350) computed on
the GPU: the conf@K choice is the `nca_conf_select` wavefront reduction, and the metric of the
chosen trial, the any-of-k test of pass@K and the (weighted) means are device reductions.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib
from .inference import rollout_steps
from .readout import conf_select, readout


@dataclass
class RolloutConfig:
    depth: int
    k: int = 1
    fire_rate: float | None = None
    p_low: float | None = None
    tau: float | None = None
    given_confident: bool = True
    noise: dict | None = None
    damage_at: int | None = None
    damage: dict = field(default_factory=lambda: {"n": 1, "r_min": 0.1, "r_max": 0.4})
    pruning: dict | None = None
    record_every: int = 0
    record_boards: int = 0
    max_cells: int = 2_000_000
    amp: bool = False
    local_clock: bool = True
    engine: dict | None = None


@dataclass
class RolloutResult:
    pred: np.ndarray  # (N, K, H, W) decoded boards
    conf: np.ndarray  # (N, K) final board confidence
    alive: np.ndarray  # (N, K) bool
    cell_updates: np.ndarray  # (N, K) fired cells over the rollout
    steps: np.ndarray  # recorded steps (T,)
    trace_exact: np.ndarray | None
    trace_cell_acc: np.ndarray | None
    trace_conf: np.ndarray | None
    trace_updates: np.ndarray | None
    boards_trace: np.ndarray | None = None  # (record_boards, T, H, W) trial 0's decodes
    damage_masks: np.ndarray | None = None
    metrics: dict | None = None  # task metrics of the final boards, name -> (N, K)

    @property
    def n_boards(self) -> int:
        return self.pred.shape[0]


def decode_tokens(model, x, given, inputs, fill_given: bool = True):
    """Decoded tokens (B, H, W) and board confidence (B,) of states x. With `fill_given` (maze,
    Sudoku) given cells show their input token (reference rollout.py:74-82)."""
    _, conf, idx = readout(model, x)
    dec = model.token_table("tokens", x.device)[idx.long()]
    return (torch.where(given, inputs, dec) if fill_given else dec), conf


def _eval_mask(task, boards) -> np.ndarray:
    """The scored cells (reference tasks/base.py:126-132): the task's eval_mask, by default the
    mutable cells."""
    if task is not None and hasattr(task, "eval_mask"):
        return np.asarray(task.eval_mask(boards), dtype=bool)
    return ~boards.given


class _Batch:
    """The rows one pass of `rollout` still runs, on the device: the state and its clamp, the
    boards' tokens repeated per trial, the fired-cell counts and `flat`, the (board, trial) index
    of each row in the whole result (board-major, reference rollout.py:143-146). Dropping rows
    (pruning) keeps every per-row tensor aligned."""

    ROW_KEYS = ("x", "given4", "clamp", "inputs", "targets", "given", "scored", "updates", "flat")

    def __init__(self, model, task, **rows):
        self.model, self.task = model, task
        self.fill_given = getattr(task, "fill_given", True)
        for k in self.ROW_KEYS:
            setattr(self, k, rows[k])

    def __len__(self) -> int:
        return self.x.shape[0]

    def score(self) -> tuple[torch.Tensor, torch.Tensor, dict]:
        """(decoded boards, board confidence, task metrics) of the current states; the metrics
        are the task's per-row device metrics (exact, cell_acc, and e.g. valid / optimal)."""
        dec, conf = decode_tokens(self.model, self.x, self.given, self.inputs, self.fill_given)
        metrics = self.task.device_metrics(dec, self.inputs, self.targets, self.given,
                                           self.scored)
        return dec, conf, metrics

    def keep(self, rows: torch.Tensor) -> None:
        """Keep only `rows` (a sorted index tensor), in order."""
        for k in self.ROW_KEYS:
            setattr(self, k, getattr(self, k).index_select(0, rows))
        self.x = self.x.contiguous()


class _Outputs:
    """Everything a rollout reports, on the device until `to_host`: the final decode, confidence,
    alive flag, fired counts and task metrics per (board, trial) row, the per-record-step traces
    and the decoded boards of trial 0 of the first `n_boards_trace` boards."""

    TRACES = (("exact", torch.bool), ("cell", torch.float32), ("conf", torch.float32),
              ("upd", torch.float64))

    def __init__(self, rows: int, H: int, W: int, T: int, n_boards_trace: int, device):
        self.rows, self.T, self.device = rows, T, device
        self.pred = torch.empty((rows, H, W), dtype=torch.int64, device=device)
        self.conf = torch.empty((rows,), dtype=torch.float32, device=device)
        self.upd = torch.empty((rows,), dtype=torch.float64, device=device)
        self.alive = torch.ones((rows,), dtype=torch.bool, device=device)
        self.metrics: dict[str, torch.Tensor] = {}
        self.trace = ({k: torch.zeros((rows, T), dtype=dt, device=device) for k, dt in self.TRACES}
                      if T else None)
        self.boards = (torch.zeros((n_boards_trace, T, H, W), dtype=torch.int64, device=device)
                       if n_boards_trace and T else None)

    def final(self, b: _Batch, rows: torch.Tensor, dec, conf, metrics, t_from: int) -> None:
        """The last values of the batch rows `rows` (positions in b): a trajectory that ends
        before the last record step keeps them in the later trace columns."""
        flat = b.flat[rows]
        self.pred[flat] = dec[rows]
        self.conf[flat] = conf[rows]
        self.upd[flat] = b.updates[rows]
        for name, v in metrics.items():
            if name not in self.metrics:
                self.metrics[name] = torch.zeros((self.rows,), dtype=v.dtype, device=self.device)
            self.metrics[name][flat] = v[rows]
        if self.trace is not None and t_from < self.T:
            vals = (metrics["exact"], metrics["cell_acc"].float(), conf, b.updates)
            for (k, _), v in zip(self.TRACES, vals):
                self.trace[k][flat, t_from:] = v[rows][:, None]

    def record(self, b: _Batch, t_rec: int, dec, conf, metrics, K: int, board0: int,
               n_boards: int) -> None:
        """Trace column t_rec of the batch's rows, and trial 0's decoded board of the traced
        boards among the pass's boards board0 .. board0 + n_boards - 1 (reference
        rollout.py:277-288)."""
        for (k, _), v in zip(self.TRACES, (metrics["exact"], metrics["cell_acc"].float(), conf,
                                            b.updates)):
            self.trace[k][b.flat, t_rec] = v
        nb = 0 if self.boards is None else min(n_boards, self.boards.shape[0] - board0)
        if nb > 0:
            # the current decodes go into the result first, so a trial 0 pruned earlier shows
            # its last decode, as in the reference
            self.pred[b.flat] = dec
            first = torch.arange(board0, board0 + nb, device=self.device) * K
            self.boards[board0:board0 + nb, t_rec] = self.pred[first]

    def to_host(self, N: int, K: int, H: int, W: int, steps) -> RolloutResult:
        host = lambda t: t.cpu().numpy()  # noqa: E731
        tr = self.trace
        return RolloutResult(
            host(self.pred).reshape(N, K, H, W), host(self.conf).reshape(N, K),
            host(self.alive).reshape(N, K), host(self.upd).reshape(N, K), np.array(steps),
            *((host(tr[k]).reshape(N, K, self.T) for k, _ in self.TRACES) if tr is not None
              else (None, None, None, None)),
            boards_trace=None if self.boards is None else host(self.boards),
            metrics={k: host(v).reshape(N, K) for k, v in self.metrics.items()},
        )


def _schedule(rc: RolloutConfig) -> tuple[list[int], set[int]]:
    """(record steps, pruning steps). Record every `record_every` steps and at the end (reference
    rollout.py:116-118); prune at the m - 1 equidistant steps i * (depth // m), i = 1 .. m - 1,
    which never include step 0 (reference rollout.py:163-167, 249)."""
    steps = []
    if rc.record_every > 0:
        steps = list(range(rc.record_every, rc.depth + 1, rc.record_every))
        if not steps or steps[-1] != rc.depth:
            steps.append(rc.depth)
    prune = set()
    if rc.pruning:
        m = int(rc.pruning["m"])
        prune = {i * (rc.depth // m) for i in range(1, m)} - {0}
    return steps, prune


@torch.no_grad()
def rollout(model, task, boards, rc: RolloutConfig, seed: int = 0, task_ids=None,
            progress: bool = False) -> RolloutResult:
    """Run every board `rc.k` times (reference rollout.py:86-306). With `rc.pruning`
    ({"m", "n_cap"}) the ensemble of each board is halved at m - 1 equidistant steps
    (`pruning.prune_select_rows` on the running rows) and the pruned trajectories leave the batch;
    a pruned trajectory keeps its last state's decode, confidence, counts and metrics, also in
    the traces of the later record steps. After a pruning step the surviving rows are
    renumbered 0, 1, ... in the pass for the Philox row counter. `rc.record_boards` keeps trial
    0's decoded board of the first boards at every record step (`boards_trace`)."""
    if rc.noise is not None or rc.damage_at is not None:
        raise ValueError("test-time noise and damage are not implemented by the HIP rollout")
    if task_ids is not None or model.cfg.time_steps:
        raise ValueError("task / time embeddings are not implemented by the HIP rollout")
    from .pruning import prune_select_rows
    from .tasks import Task

    model.eval()
    device = model.device
    if device.type != "cuda":
        raise ValueError("the HIP rollout needs the model on the GPU")
    task = task if task is not None else Task()
    N = len(boards)
    H, W = boards.shape
    K = rc.k
    per_pass = max(1, rc.max_cells // (K * H * W))
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    precision = "bf16" if rc.amp else "fp32"
    steps, prune_steps = _schedule(rc)
    n_cap = int(rc.pruning.get("n_cap", 3)) if rc.pruning else 3
    bounds = sorted({rc.depth, *steps, *prune_steps})
    out = _Outputs(N * K, H, W, len(steps), rc.record_boards, device)
    scored_all = _eval_mask(task, boards)
    event = 0
    for start in range(0, N, per_pass):
        stop_b = min(N, start + per_pass)
        base = start * K
        sub = boards.subset(np.arange(start, stop_b))
        up = lambda a: _lib.upload(np.repeat(a, K, 0), device)  # noqa: E731
        inputs, given = up(sub.inputs), up(sub.given)
        x, given4, clamp = model.init_state(inputs, given, None, gen)
        B = len(sub) * K
        b = _Batch(model, task, x=x.float().contiguous(), given4=given4, clamp=clamp,
                   inputs=inputs, targets=up(sub.targets), given=given,
                   scored=up(scored_all[start:stop_b]),
                   updates=torch.zeros(B, dtype=torch.float64, device=device),
                   flat=torch.arange(base, base + B, device=device))
        t, t_rec = 0, 0
        for stop in bounds:
            b.x, _, fired = rollout_steps(
                model, b.x, b.given4, b.clamp, stop - t, seed=seed, p_fire=rc.fire_rate,
                p_low=rc.p_low, tau=rc.tau, given_confident=rc.given_confident,
                row0=base, step0=t, precision=precision, out=b.x, want_conf=False,
                want_fired=True,
            )
            b.updates += fired.double()
            t = stop
            scores = None
            if stop in prune_steps:
                scores = b.score()
                dec, conf, _ = scores
                keep = prune_select_rows(dec, conf, b.flat - base, len(sub), K, n_cap, seed,
                                         event)
                event += 1
                gone = (~keep).nonzero().squeeze(1)  # one host wait per pruning step
                if len(gone):
                    out.final(b, gone, *scores, t_rec)
                    out.alive[b.flat[gone]] = False
                    b.keep(keep.nonzero().squeeze(1))
                    scores = None
            if t_rec < len(steps) and stop == steps[t_rec]:
                out.record(b, t_rec, *(scores or b.score()), K, start, len(sub))
                t_rec += 1
        out.final(b, torch.arange(len(b), device=device), *b.score(), len(steps))
    return out.to_host(N, K, H, W, steps)


def score_candidates(task, res: RolloutResult, boards) -> dict[str, np.ndarray]:
    """Task metrics of every (board, trial) of a rollout result: dict of (N, K) arrays
    (reference rollout.py:309-314). `rollout` computes them on the GPU with the final states;
    for a result without them they are computed from `res.pred` on the GPU."""
    if res.metrics:
        return res.metrics
    N, K, H, W = res.pred.shape
    return {k: v.reshape(N, K) for k, v in task.metrics(res.pred.reshape(N * K, H, W), boards,
                                                         k=K).items()}


def _device_metric(metric, alive, weights):
    dev = torch.device("cuda", torch.cuda.current_device())
    m = _lib.upload(np.ascontiguousarray(metric), dev)
    a = None if alive is None else _lib.upload(np.ascontiguousarray(alive, dtype=bool), dev)
    w = None if weights is None else _lib.upload(np.asarray(weights, np.float64), dev)
    return m, a, w


def _mean(v, w):
    v = v.double()
    return v.mean() if w is None else (v * w).sum() / w.sum()


def conf_at_k(metric, conf, alive, ks, weights=None) -> dict[int, float]:
    """Conf@k for every k in ks from one run of K trials (reference rollout.py:317-334): per
    board, the alive trial of highest board confidence among the first k (the first one on
    ties: `nca_conf_select`), and the (weighted) mean of its metric. Computed on the GPU; one
    copy of the results to the host."""
    N, K = np.shape(metric)
    m, a, w = _device_metric(metric, alive, weights)
    c = _lib.upload(np.ascontiguousarray(conf, dtype=np.float32), m.device)
    rows = torch.arange(N, device=m.device)
    kk = [min(int(k), K) for k in ks]
    vals = torch.stack([_mean(m[rows, conf_select(c, a, k)], w) for k in kk]).tolist()
    return dict(zip(kk, vals))


def pass_at_k(metric, alive, ks, weights=None) -> dict[int, float]:
    """Pass@k (reference rollout.py:337-350): the (weighted) fraction of boards with a correct
    alive trial among the first k. Computed on the GPU; one copy to the host."""
    N, K = np.shape(metric)
    m, a, w = _device_metric(metric, alive, weights)
    ok = m.bool() & (a if a is not None else True)
    kk = [min(int(k), K) for k in ks]
    vals = torch.stack([_mean(ok[:, :k].any(dim=1), w) for k in kk]).tolist()
    return dict(zip(kk, vals))


def select_at_k(conf: torch.Tensor, alive: torch.Tensor | None, k: int) -> torch.Tensor:
    """conf_at_k's per-board choice on the GPU: (N,) trial index."""
    return conf_select(conf, alive, k)
