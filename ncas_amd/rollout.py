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
    boards_trace: np.ndarray | None = None
    damage_masks: np.ndarray | None = None

    @property
    def n_boards(self) -> int:
        return self.pred.shape[0]


def decode_tokens(model, x, given, inputs, fill_given: bool = True):
    """Decoded tokens (B, H, W) and board confidence (B,) of states x. With `fill_given` (maze,
    Sudoku) given cells show their input token (reference rollout.py:74-82)."""
    _, conf, idx = readout(model, x)
    tokens = torch.tensor(model.cfg.output_tokens, device=x.device)
    dec = tokens[idx.long()]
    return (torch.where(given, inputs, dec) if fill_given else dec), conf


class _Scorer:
    """Per-row scores of a pass, on the device: decoded board, cell accuracy and exactness over
    the scored cells, board confidence (reference rollout.py:181-184)."""

    def __init__(self, model, task, inputs, targets, given, scored):
        self.model, self.inputs, self.targets, self.given = model, inputs, targets, given
        self.fill_given = getattr(task, "fill_given", True)
        self.scored = scored
        self.n_scored = scored.sum(dim=(1, 2)).clamp_min(1)

    def __call__(self, x):
        dec, conf = decode_tokens(self.model, x, self.given, self.inputs, self.fill_given)
        correct = ((dec == self.targets) & self.scored).sum(dim=(1, 2))
        return dec, correct / self.n_scored, correct == self.n_scored, conf


def _eval_mask(task, boards) -> np.ndarray:
    """The scored cells (reference tasks/base.py:126-132): the task's eval_mask, by default the
    mutable cells."""
    if task is not None and hasattr(task, "eval_mask"):
        return np.asarray(task.eval_mask(boards), dtype=bool)
    return ~boards.given


@torch.no_grad()
def rollout(model, task, boards, rc: RolloutConfig, seed: int = 0, task_ids=None,
            progress: bool = False) -> RolloutResult:
    """Run every board `rc.k` times (reference rollout.py:86-306). With `rc.pruning`
    ({"m", "n_cap"}) the ensemble of each board is halved at m - 1 equidistant steps
    (`pruning.prune_select`) and the pruned trajectories leave the batch (rows compacted on the
    GPU); a pruned trajectory keeps its last state's decode, confidence and counts, also in the
    traces of the later record steps. After a pruning step the surviving rows are renumbered
    0, 1, ... in the pass for the Philox row counter."""
    if rc.noise is not None or rc.damage_at is not None:
        raise ValueError("test-time noise and damage are not implemented by the HIP rollout")
    if task_ids is not None or model.cfg.time_steps:
        raise ValueError("task / time embeddings are not implemented by the HIP rollout")
    from .pruning import prune_select

    model.eval()
    device = model.device
    if device.type != "cuda":
        raise ValueError("the HIP rollout needs the model on the GPU")
    N = len(boards)
    H, W = boards.shape
    K = rc.k
    per_pass = max(1, rc.max_cells // (K * H * W))
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    precision = "bf16" if rc.amp else "fp32"
    record = rc.record_every > 0
    steps = list(range(rc.record_every, rc.depth + 1, rc.record_every)) if record else []
    if record and (not steps or steps[-1] != rc.depth):
        steps.append(rc.depth)
    T = len(steps)
    prune_steps, n_cap = set(), 3
    if rc.pruning:
        m = int(rc.pruning["m"])
        n_cap = int(rc.pruning.get("n_cap", 3))
        stride = rc.depth // m
        prune_steps = {i * stride for i in range(1, m)}
    bounds = sorted({rc.depth, *steps, *prune_steps})
    rows_total = N * K
    # every output lives on the device until the end of the call
    pred = torch.empty((rows_total, H, W), dtype=torch.int64, device=device)
    conf_out = torch.empty((rows_total,), dtype=torch.float32, device=device)
    upd_out = torch.empty((rows_total,), dtype=torch.float64, device=device)
    alive_out = torch.ones((rows_total,), dtype=torch.bool, device=device)
    tr = {k: torch.zeros((rows_total, T), dtype=dt, device=device) for k, dt in
          (("exact", torch.bool), ("cell", torch.float32), ("conf", torch.float32),
           ("upd", torch.float64))} if record else None
    scored_all = _eval_mask(task, boards)
    event = 0
    for start in range(0, N, per_pass):
        stop_b = min(N, start + per_pass)
        n = stop_b - start
        sub = boards.subset(np.arange(start, stop_b))
        base = start * K
        inputs = _lib.upload(np.repeat(sub.inputs, K, 0), device)
        targets = _lib.upload(np.repeat(sub.targets, K, 0), device)
        given = _lib.upload(np.repeat(sub.given, K, 0), device)
        scored = _lib.upload(np.repeat(scored_all[start:stop_b], K, 0), device)
        x, given4, clamp = model.init_state(inputs, given, None, gen)
        x = x.float().contiguous()
        B = n * K
        idx = torch.arange(base, base + B, device=device)  # flat (board, trial) row of each row
        updates = torch.zeros(B, dtype=torch.float64, device=device)
        t, t_rec = 0, 0

        def store(rows, dec, cell, exact, conf, upd, t_from):
            pred[rows] = dec
            conf_out[rows] = conf
            upd_out[rows] = upd
            if record and t_from < T:
                tr["exact"][rows, t_from:] = exact[:, None]
                tr["cell"][rows, t_from:] = cell.float()[:, None]
                tr["conf"][rows, t_from:] = conf[:, None]
                tr["upd"][rows, t_from:] = upd[:, None]

        for stop in bounds:
            x, _, fired = rollout_steps(
                model, x, given4, clamp, stop - t, seed=seed, p_fire=rc.fire_rate,
                p_low=rc.p_low, tau=rc.tau, given_confident=rc.given_confident,
                row0=base, step0=t, precision=precision, out=x, want_conf=False,
                want_fired=True,
            )
            updates += fired.double()
            t = stop
            score = _Scorer(model, task, inputs, targets, given, scored)
            if stop in prune_steps:
                dec, cell, exact, conf = score(x)
                local = idx - base  # row of the (board, trial) in the pass's full layout
                dec_full = torch.zeros((B, H, W), dtype=torch.int64, device=device)
                conf_full = torch.full((B,), -float("inf"), device=device)
                alive_full = torch.zeros(B, dtype=torch.bool, device=device)
                dec_full[local], conf_full[local], alive_full[local] = dec, conf, True
                keep = prune_select(dec_full.view(n, K, H * W), conf_full.view(n, K),
                                    alive_full.view(n, K), n_cap, seed, event).view(B)[local]
                event += 1
                drop = ~keep
                store(idx[drop], dec[drop], cell[drop], exact[drop], conf[drop], updates[drop],
                      t_rec)
                alive_out[idx[drop]] = False
                sel = keep.nonzero().squeeze(1)  # one host wait per pruning step
                x, given4, clamp = x[sel].contiguous(), given4[sel], clamp[sel]
                inputs, targets, given, scored = inputs[sel], targets[sel], given[sel], scored[sel]
                updates, idx = updates[sel], idx[sel]
                score = _Scorer(model, task, inputs, targets, given, scored)
            if record and t_rec < T and stop == steps[t_rec]:
                _, cell, exact, conf = score(x)
                tr["exact"][idx, t_rec] = exact
                tr["cell"][idx, t_rec] = cell.float()
                tr["conf"][idx, t_rec] = conf
                tr["upd"][idx, t_rec] = updates
                t_rec += 1
        dec, cell, exact, conf = _Scorer(model, task, inputs, targets, given, scored)(x)
        store(idx, dec, cell, exact, conf, updates, T)
    host = lambda t: t.cpu().numpy()  # noqa: E731
    return RolloutResult(
        host(pred).reshape(N, K, H, W), host(conf_out).reshape(N, K),
        host(alive_out).reshape(N, K), host(upd_out).reshape(N, K), np.array(steps),
        *((host(tr[k]).reshape(N, K, T) for k in ("exact", "cell", "conf", "upd")) if record
          else (None, None, None, None)),
    )


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
