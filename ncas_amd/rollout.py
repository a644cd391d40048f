"""Inference over boards: K stochastic trials per board, D fused steps, conf@K selection.

`rollout(model, task, boards, rc, seed)` mirrors the reference's evaluation engine (reference
src/nca/rollout.py:85-305) for the features of the HIP path: depth, K trials flattened
board-major (row = board * K + trial, rollout.py:143-146), uniform or confidence-gated firing
(`p_low`, `tau`, `given_confident`), bf16 (`amp`), chunking by `max_cells`, traces every
`record_every` steps and the final decoded boards / board confidence / fired-cell counts.
Fire masks come from the Philox rule keyed on the global row index and step, so results do
not depend on `max_cells` or on where the trace boundaries fall. The steps between two trace
points run as one launch of the LDS-resident kernel (`inference.rollout_steps`).

Test-time noise, damage and pruning are not implemented and raise ValueError.

`conf_at_k` / `pass_at_k` are the reference's selection metrics (rollout.py:317-350);
`select_at_k` is the same per-board choice computed on the GPU.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

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


def decode_tokens(model, x, given, inputs):
    """Decoded tokens (B, H, W); given cells show their input token (rollout.py:74-82)."""
    _, conf, idx = readout(model, x)
    tokens = torch.tensor(model.cfg.output_tokens, device=x.device)
    dec = tokens[idx.long()]
    return torch.where(given, inputs, dec), conf


@torch.no_grad()
def rollout(model, task, boards, rc: RolloutConfig, seed: int = 0, task_ids=None,
            progress: bool = False) -> RolloutResult:
    if rc.noise is not None or rc.damage_at is not None or rc.pruning:
        raise ValueError("noise, damage and pruning are not implemented by the HIP rollout")
    if task_ids is not None or model.cfg.time_steps:
        raise ValueError("task / time embeddings are not implemented by the HIP rollout")
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
    out_pred = np.zeros((N, K, H, W), np.int64)
    out_conf = np.zeros((N, K), np.float32)
    out_alive = np.ones((N, K), bool)
    out_upd = np.zeros((N, K), np.float64)
    tr = {k: (np.zeros((N, K, T), dt) if record else None) for k, dt in
          (("exact", bool), ("cell", np.float32), ("conf", np.float32), ("upd", np.float64))}
    fill_given = getattr(task, "fill_given", True)
    for start in range(0, N, per_pass):
        sub = boards.subset(np.arange(start, min(N, start + per_pass)))
        n = len(sub)
        B = n * K
        inputs = torch.from_numpy(np.repeat(sub.inputs, K, 0)).to(device)
        targets = torch.from_numpy(np.repeat(sub.targets, K, 0)).to(device)
        given = torch.from_numpy(np.repeat(sub.given, K, 0)).to(device)
        mutable = (~given).float()
        n_mut = mutable.sum(dim=(1, 2)).clamp_min(1)
        x, given4, clamp = model.init_state(inputs, given, None, gen)
        x = x.float().contiguous()
        updates = torch.zeros(B, dtype=torch.float64, device=device)
        t = 0
        for t_rec, stop in enumerate(steps + ([] if record else [rc.depth])):
            x, _, fired = rollout_steps(
                model, x, given4, clamp, stop - t, seed=seed, p_fire=rc.fire_rate,
                p_low=rc.p_low, tau=rc.tau, given_confident=rc.given_confident,
                row0=start * K, step0=t, precision=precision, out=x, want_conf=False,
                want_fired=True,
            )
            updates += fired.double()
            t = stop
            if record:
                dec, conf = decode_tokens(model, x, given, inputs) if fill_given else (None, None)
                correct = ((dec == targets).float() * mutable).sum(dim=(1, 2))
                sl = slice(start, start + n)
                tr["exact"][sl, :, t_rec] = (correct == n_mut).view(n, K).cpu().numpy()
                tr["cell"][sl, :, t_rec] = (correct / n_mut).view(n, K).cpu().numpy()
                tr["conf"][sl, :, t_rec] = conf.view(n, K).cpu().numpy()
                tr["upd"][sl, :, t_rec] = updates.view(n, K).cpu().numpy()
        dec, conf = decode_tokens(model, x, given, inputs)
        out_pred[start:start + n] = dec.view(n, K, H, W).cpu().numpy()
        out_conf[start:start + n] = conf.view(n, K).cpu().numpy()
        out_upd[start:start + n] = updates.view(n, K).cpu().numpy()
    return RolloutResult(out_pred, out_conf, out_alive, out_upd, np.array(steps), tr["exact"],
                         tr["cell"], tr["conf"], tr["upd"])


def conf_at_k(metric, conf, alive, ks, weights=None) -> dict[int, float]:
    """Conf@k (reference rollout.py:317-334): per board the alive trial of highest board
    confidence among the first k (first maximum), mean metric."""
    N, K = metric.shape
    out = {}
    for k in ks:
        k = min(k, K)
        c = np.where(alive[:, :k], conf[:, :k], -np.inf)
        best = c.argmax(axis=1)
        out[k] = float(np.average(metric[np.arange(N), best], weights=weights))
    return out


def pass_at_k(metric, alive, ks, weights=None) -> dict[int, float]:
    """Pass@k (reference rollout.py:337-350)."""
    N, K = metric.shape
    return {
        min(k, K): float(np.average((metric[:, : min(k, K)] & alive[:, : min(k, K)]).any(axis=1),
                                    weights=weights))
        for k in ks
    }


def select_at_k(conf: torch.Tensor, alive: torch.Tensor | None, k: int) -> torch.Tensor:
    """conf_at_k's per-board choice on the GPU: (N,) trial index."""
    return conf_select(conf, alive, k)
