"""BPTT training on the HIP path: the chunk forward/backward operator, the reference engine's
`train_iteration`, its loss weights and the replay pool.

* `bptt_chunk(model, x, given4, clamp, targets, weights, ...)` - forward a chunk of
  `len(weights)` steps keeping only its states (C ABI `nca_bptt_forward`), then the fused
  backward that recomputes perception and hidden activations from those states
  (`nca_bptt_backward`). Returns the final state, the loss, the parameter gradients and the
  gradient of the initial state. Replaces the chunk of the reference's
  `Engine.train_iteration` (reference src/nca/engine/engine.py:478-497) that autograd or
  `torch.utils.checkpoint` segments would otherwise differentiate.
* `Engine(model, rollout, chunk, amp).train_iteration(batch, seeds, c0, weights, grad_clip,
  apply_update) -> (x, loss, grad_norm)` - the reference's interface (engine.py:366-517):
  no-grad prefix [0, c0), the chunk with gradient, clipping, the update callback, no-grad
  suffix; fire masks from per-step Philox keys `seeds` (as from `rng.step_seeds`).
* `loss_weights(window, chunk)` - reference src/nca/engine/train.py:60-69.
* `ReplayPool` - the replay buffer of reference src/nca/pool.py:26-204 (sample / write_back /
  state_dict) for (B, H, W) token boards, on the model's device.

The loss is the per-cell cross-entropy of the mlp head's logits (reference train.py:183-193)
averaged over cells (or a loss mask), weighted per chunk step and normalised by the sum of
the weights (step.py:243-245, engine.py:490). Gradients of bf16 cells are those of the rounded
forward with straight-through rounding, computed in fp32.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .inference import rollout_steps
from .rng import fire_desc

_GRAD_NAMES = ("kernels", "w1", "b1", "w2", "b2", "head_w", "head_b")


def _params(model):
    """The model's parameters in the C ABI's order (kernels, w1, b1, w2, b2, head_w, head_b)."""
    return (model.perceive.weight, model.update.fc1.weight, model.update.fc1.bias,
            model.update.fc2.weight, model.update.fc2.bias, model.head.weight, model.head.bias)


def loss_weights(window, chunk: int, device=None) -> torch.Tensor:
    """Per-chunk-step loss weights for `loss_window` ("all", "last" or an integer w)
    (reference src/nca/engine/train.py:60-69)."""
    w = torch.zeros(chunk, device=device)
    if window == "all":
        w[:] = 1.0
    elif window == "last":
        w[-1] = 1.0
    else:
        w[chunk - int(window):] = 1.0
    return w


@dataclass
class ChunkResult:
    x: torch.Tensor              # final state (B, C, H, W)
    loss: torch.Tensor           # scalar (device)
    grads: dict                  # name -> gradient shaped like the parameter
    grad_x0: torch.Tensor | None
    states_bytes: int            # bytes of the kept chunk states
    workspace_bytes: int         # bytes of the backward's workspace


def bptt_chunk(model, x, given4, clamp, targets, weights, *, seed: int = 0, step_seeds=None,
               masks=None, p_fire: float | None = None, row0: int = 0, step0: int = 0,
               precision: str = "fp32", loss_mask=None, grad_final=None,
               want_grad_x0: bool = False) -> ChunkResult:
    """Forward + backward of one BPTT chunk of `len(weights)` steps on the GPU.

    targets: (B, H, W) class indices in [0, n_out) (`model.output_index(tokens)`); masks:
    injected fire masks (n, B, 1, H, W), else Philox keyed on `step_seeds` (n,) or `seed`."""
    cfg = model.cfg
    if cfg.head != "mlp":
        raise ValueError("the BPTT loss is the cross-entropy of an mlp head")
    dev = _lib.require_device(x, given4, clamp, targets, masks, loss_mask, grad_final)
    B, C, H, W = x.shape
    n = len(weights)
    w_host = np.ascontiguousarray(np.asarray(
        weights.detach().cpu() if torch.is_tensor(weights) else weights, dtype=np.float32))
    pk = model.packed(precision, dev)
    L = _lib.load()
    xs = x.detach().to(torch.float32).contiguous()
    g8 = given4.detach().to(torch.uint8).contiguous()
    cl = clamp.detach().to(torch.float32).contiguous()
    tg = targets.detach().to(torch.int32).contiguous()
    lm = None if loss_mask is None else loss_mask.detach().to(torch.float32).contiguous()
    gf = None if grad_final is None else grad_final.detach().to(torch.float32).contiguous()
    m8 = None
    if masks is not None:
        if masks.shape[0] != n or masks[0].numel() != B * H * W:
            raise ValueError("masks must be (n, B, 1, H, W)")
        m8 = (masks.detach() != 0).to(torch.uint8).contiguous()
    ss = None
    if step_seeds is not None:
        ss = _lib.upload(np.asarray(step_seeds, dtype=np.int64), dev)
        if ss.numel() != n:
            raise ValueError("step_seeds must have one key per chunk step")
    fd = fire_desc(seed, cfg.fire_rate if p_fire is None else p_fire, None, None, True, row0,
                   step0, ss, m8)
    states = torch.empty((n + 1, B, C, H, W), dtype=torch.float32, device=dev)
    stream = _lib.stream_of(dev)
    _lib.check(L.nca_bptt_forward(ctypes.byref(pk.desc), pk.buf.data_ptr(), B, H, W,
                                  xs.data_ptr(), g8.data_ptr(), cl.data_ptr(), ctypes.byref(fd),
                                  n, states.data_ptr(), stream), "nca_bptt_forward")
    # fp32 master weights for the backward GEMMs (rounded to bf16 on load for bf16 cells)
    params = _params(model)
    master = [p.detach().to(dev, torch.float32).contiguous() for p in params]
    wts = _lib.CellWeights(master[0].data_ptr(), master[1].data_ptr(), master[2].data_ptr(),
                           master[3].data_ptr(), master[4].data_ptr(), master[5].data_ptr(),
                           master[6].data_ptr(), None)
    grads = {name: torch.empty(p.shape, dtype=torch.float32, device=dev)
             for name, p in zip(_GRAD_NAMES, params)}
    gs = _lib.CellGrads(*[grads[k].data_ptr() for k in _GRAD_NAMES])
    gx0 = torch.empty_like(xs) if want_grad_x0 else None
    loss = torch.empty((), dtype=torch.float32, device=dev)
    lossd = _lib.BpttLoss(tg.data_ptr(), _lib.ptr(lm), w_host.ctypes.data_as(ctypes.c_void_p))
    ws_bytes = L.nca_bptt_workspace_bytes(ctypes.byref(pk.desc), B, H, W, n)
    if ws_bytes == 0:
        _lib.check(_lib.NCA_ERR_UNSUPPORTED, "nca_bptt_workspace_bytes")
    ws = torch.empty((ws_bytes // 4,), dtype=torch.float32, device=dev)
    _lib.check(L.nca_bptt_backward(ctypes.byref(pk.desc), pk.buf.data_ptr(), ctypes.byref(wts), B,
                                   H, W, states.data_ptr(), g8.data_ptr(), ctypes.byref(fd), n,
                                   ctypes.byref(lossd), _lib.ptr(gf), ctypes.byref(gs),
                                   _lib.ptr(gx0), loss.data_ptr(), ws.data_ptr(), ws_bytes,
                                   stream), "nca_bptt_backward")
    # no wait: the host arrays were read during the calls, and the device buffers freed here are
    # reused only by later work on the same stream
    return ChunkResult(states[n].clone(), loss, grads, gx0, states.numel() * 4, ws_bytes)


class Engine:
    """The reference engine's training interface (reference src/nca/engine/engine.py:168-517)
    on the HIP kernels: `rollout` steps per iteration with the BPTT chunk of `chunk` steps at
    `[c0, c0 + chunk)`; bf16 when `amp`."""

    def __init__(self, model, rollout: int, chunk: int, amp: bool = False, p_fire=None):
        model.kernel_support()
        if model.cfg.head != "mlp":
            raise ValueError("Engine trains mlp-head cells (cross-entropy loss)")
        if not 1 <= chunk <= rollout:
            raise ValueError("need 1 <= chunk <= rollout")
        self.model, self.N, self.Nc, self.amp = model, rollout, chunk, amp
        self.p_fire = model.cfg.fire_rate if p_fire is None else p_fire
        self.last_chunk: ChunkResult | None = None

    @property
    def precision(self) -> str:
        return "bf16" if self.amp else "fp32"

    def _run(self, x, batch, seeds):
        if len(seeds) == 0:
            return x
        with torch.no_grad():
            y, _, _ = rollout_steps(self.model, x, batch["given4"], batch["clamp"], len(seeds),
                                    step_seeds=seeds, p_fire=self.p_fire,
                                    precision=self.precision, want_conf=False)
        return y

    def train_iteration(self, batch: dict, seeds, c0: int, weights, grad_clip,
                        apply_update=None):
        """Roll the batch out for `rollout` steps with the BPTT chunk at `[c0, c0 + chunk)`,
        add the chunk loss's gradients to the parameters' `.grad`, clip them to `grad_clip`
        (if not None) and call `apply_update(grad_norm)`. Returns (final state, loss, grad norm)
        as device tensors (reference engine.py:366-517, update_after_rollout)."""
        model = self.model
        seeds = np.asarray(seeds, dtype=np.int64)
        if len(seeds) != self.N:
            raise ValueError(f"need {self.N} step seeds")
        if not 0 <= c0 <= self.N - self.Nc:
            raise ValueError("the chunk must lie inside the rollout")
        x = self._run(batch["x"], batch, seeds[:c0])
        targets = model.output_index(batch["targets"])
        res = bptt_chunk(model, x, batch["given4"], batch["clamp"], targets, weights,
                         step_seeds=seeds[c0:c0 + self.Nc], p_fire=self.p_fire,
                         precision=self.precision, loss_mask=batch.get("loss_mask"))
        self.last_chunk = res
        for name, p in zip(_GRAD_NAMES, _params(model)):
            g = res.grads[name].reshape(p.shape).to(p.dtype)
            p.grad = g if p.grad is None else p.grad + g
        if grad_clip is not None:
            gn = torch.nn.utils.clip_grad_norm_(model.parameters(), grad_clip)
        else:
            gn = res.loss.new_zeros(())
        x = self._run(res.x, batch, seeds[c0 + self.Nc:])
        if apply_update is not None:
            apply_update(gn)
        return x, res.loss, gn


class ReplayPool:
    """Replay buffer of (state, board) pairs (reference src/nca/pool.py:26-204) for boards given
    as numpy (N, H, W) token grids with a boolean `given` mask (`tasks.Boards`)."""

    def __init__(self, model, boards, size: int, rng: np.random.Generator,
                 generator: torch.Generator | None = None):
        self.model, self.boards, self.size, self.rng = model, boards, size, rng
        self.generator = generator
        self.device = model.device
        fresh = self.fresh(size)
        self.x, self.given4, self.clamp = fresh["x"], fresh["given4"], fresh["clamp"]
        self.inputs, self.targets = fresh["inputs"], fresh["targets"]
        self.age = torch.zeros(size, dtype=torch.long, device=self.device)

    def fresh(self, n: int) -> dict:
        """`n` fresh boards drawn uniformly with freshly initialised states (pool.py:58-87)."""
        idx = self.rng.integers(0, len(self.boards), size=n)
        sub = self.boards.subset(idx)
        inputs = _lib.upload(sub.inputs, self.device)
        targets = _lib.upload(sub.targets, self.device)
        given = _lib.upload(sub.given, self.device)
        x, given4, clamp = self.model.init_state(inputs, given, None, self.generator)
        return dict(x=x.detach(), given4=given4, clamp=clamp, inputs=inputs, targets=targets)

    def sample(self, batch_size: int, seed_ratio: float):
        """`batch_size` pool entries without replacement, the first round(seed_ratio * batch)
        replaced by fresh boards (pool.py:90-131). Returns (indices, batch dict of copies)."""
        idx = self.rng.choice(self.size, size=batch_size, replace=False)
        di = _lib.upload(idx, self.device)
        batch = {k: getattr(self, k).index_select(0, di)
                 for k in ("x", "given4", "clamp", "inputs", "targets", "age")}
        n_fresh = int(round(seed_ratio * batch_size))
        if n_fresh > 0:
            f = self.fresh(n_fresh)
            for k in ("x", "given4", "clamp", "inputs", "targets"):
                batch[k][:n_fresh] = f[k]
            batch["age"][:n_fresh] = 0
        return idx, batch

    def write_back(self, idx, batch: dict) -> None:
        """Store the post-rollout states back (pool.py:166-179)."""
        di = _lib.upload(idx, self.device)
        with torch.no_grad():
            self.x[di] = batch["x"].detach()
        for k in ("given4", "clamp", "inputs", "targets"):
            getattr(self, k)[di] = batch[k]
        self.age[di] = batch["age"] + 1

    def state_dict(self) -> dict:
        return {k: getattr(self, k) for k in ("x", "given4", "clamp", "inputs", "targets", "age")}

    def load_state_dict(self, d: dict) -> None:
        for k, v in d.items():
            setattr(self, k, v.to(self.device))
