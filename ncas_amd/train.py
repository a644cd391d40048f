"""BPTT training on the HIP path: the chunk operator, the reference engine's training interface,
its loss weights and the replay pool.

* `bptt_chunk(model, x, given4, clamp, targets, weights, ...)` - forward a chunk of
  `len(weights)` steps keeping only its states (C ABI `nca_bptt_forward_ws`), then the fused
  backward that recomputes perception and hidden activations from those states
  (`nca_bptt_backward`). Returns the final state, the loss, the parameter gradients and the
  gradient of the initial state. Replaces the chunk of the reference's
  `Engine.train_iteration` (reference src/nca/engine/engine.py:478-497) that autograd or
  `torch.utils.checkpoint` segments would otherwise differentiate.
* `EngineConfig` / `Engine(model, cfg, train_cfg, device)` - the reference engine's
  constructor and `train_iteration(batch, seeds, c0, weights, grad_clip, apply_update) ->
  (x, loss, grad_norm)` (reference engine.py:59-155, 167-207, 366-517): a no-grad fp32 prefix
  [0, c0), the chunk with gradient (bf16 when `train_cfg["amp"]`), clipping, the update callback
  (after the rollout or right after the backward, `update_after_rollout`), a no-grad fp32 suffix.
  The chunk runs on the fused chunk operator when the loss is the cross-entropy of an mlp head
  and no step noise is drawn; otherwise step by step through the differentiable HIP step
  (`step.make_step`), with the loss of every step computed by torch on the GPU.
* `loss_weights(window, chunk)` - the per-step weights of `train.loss_window` (reference
  src/nca/engine/train.py:60-69).
* `ReplayPool` - the replay buffer of reference src/nca/pool.py:26-204 for (N, H, W) token
  boards: fresh boards, sampling with fresh replacements, write-back with ages, target swaps,
  state_dict.

Fire masks come from Philox keyed on (per-step seed; row, step, cell), the same rule as every
kernel, with global step indices: step s of the iteration uses seed `seeds[s]` and counter step
s, whether it runs in the prefix, the chunk or the suffix. Step noise (reference
src/nca/engine/rng.py:51-76: with probability p_t per board, N(0, sigma^2) on a p_s fraction of
its cells) is drawn from a torch generator seeded with the step's seed.

The chunk loss is sum_t w_t * step_loss(x_{t+1}) / max(sum_t w_t, 1) (reference
src/nca/engine/step.py:243-245, engine.py:490) with step_loss the mean (or loss-mask weighted
mean) over cells of the per-cell loss of reference src/nca/train.py:183-207 ("ce", "mse",
"mse_mean"). Gradients of bf16 cells are those of the rounded forward with straight-through
rounding, computed in fp32.
"""

from __future__ import annotations

import ctypes
from dataclasses import asdict, dataclass

import numpy as np
import torch
import torch.nn.functional as F

from . import _lib
from .inference import rollout_steps
from .rng import fire_desc, fire_mask

_GRAD_NAMES = ("kernels", "w1", "b1", "w2", "b2", "head_w", "head_b")


def _params(model):
    """The model's parameters in the C ABI's order (kernels, w1, b1, w2, b2, head_w, head_b)."""
    return (model.perceive.weight, model.update.fc1.weight, model.update.fc1.bias,
            model.update.fc2.weight, model.update.fc2.bias, model.head.weight, model.head.bias)


def loss_weights(window, chunk: int, device=None) -> torch.Tensor:
    """(chunk,) float weights of the chunk's steps for `train.loss_window` (reference
    src/nca/engine/train.py:60-69): "all" supervises every step, "last" the final one, an integer
    w the last w steps. The first supervised step of an integer window follows Python's rule
    for a slice start (chunk - w, wrapped once when negative, then clipped at 0), which is what
    the reference's slice assignment does."""
    if window == "all":
        first = 0
    elif window == "last":
        first = chunk - 1
    else:
        first = chunk - int(window)
        if first < 0:
            first = max(first + chunk, 0)
    return (torch.arange(chunk, device=device) >= first).to(torch.float32)


@dataclass
class ChunkResult:
    x: torch.Tensor              # final state (B, C, H, W)
    loss: torch.Tensor           # scalar (device)
    grads: dict                  # name -> gradient shaped like the parameter
    grad_x0: torch.Tensor | None
    states_bytes: int            # bytes of the kept chunk states
    workspace_bytes: int         # bytes of the backward's workspace
    halo_failed: torch.Tensor | None = None  # device bool: a wait of the forward's board
    #                pieces ran out and the forward was recomputed on whole boards (the states
    #                are right either way)
    back_repaired: torch.Tensor | None = None  # device bool: the same for the one-launch
    #                backward's pieces (the gradients were recomputed on whole boards)


def bptt_chunk(model, x, given4, clamp, targets, weights, *, seed: int = 0, step_seeds=None,
               masks=None, p_fire: float | None = None, row0: int = 0, step0: int = 0,
               precision: str = "fp32", loss_mask=None, grad_final=None,
               want_grad_x0: bool = False, accumulate_into=None) -> ChunkResult:
    """Forward + backward of one BPTT chunk of `len(weights)` steps on the GPU.

    targets: (B, H, W) class indices in [0, n_out) (`model.output_index(tokens)`); masks:
    injected fire masks (n, B, 1, H, W), else Philox keyed on `step_seeds` (n,) or `seed`, with
    counter steps step0 .. step0 + n - 1. `weights` is read on the host (a host array avoids a
    device-to-host copy). With `accumulate_into` (the parameters' fp32 gradient tensors, in the
    model's parameter order) the gradients are added into those tensors, as autograd adds into
    .grad, and the result's `grads` is None."""
    cfg = model.cfg
    if cfg.head != "mlp":
        raise ValueError("the fused chunk's loss is the cross-entropy of an mlp head")
    dev = _lib.require_device(x, given4, clamp, targets, masks, loss_mask, grad_final)
    B, C, H, W = x.shape
    n = len(weights)
    w_host = np.ascontiguousarray(np.asarray(
        weights.detach().cpu() if torch.is_tensor(weights) else weights, dtype=np.float32))
    pk = model.packed(precision, dev)
    L = _lib.load()
    xs = x.detach().to(torch.float32).contiguous()
    g8 = (given4.detach().view(torch.uint8) if given4.dtype == torch.bool else given4.detach().to(torch.uint8)).contiguous()
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
    ws_bytes = L.nca_bptt_workspace_bytes(ctypes.byref(pk.desc), B, H, W, n)
    if ws_bytes == 0:
        _lib.check(_lib.NCA_ERR_UNSUPPORTED, "nca_bptt_workspace_bytes")
    ws = torch.empty((ws_bytes // 4,), dtype=torch.float32, device=dev)
    # the forward may run boards in pieces of rows, exchanging rows through the workspace (which
    # the backward then overwrites)
    _lib.check(L.nca_bptt_forward_ws(ctypes.byref(pk.desc), pk.buf.data_ptr(), B, H, W,
                                     xs.data_ptr(), g8.data_ptr(), cl.data_ptr(), ctypes.byref(fd),
                                     n, states.data_ptr(), ws.data_ptr(), ws_bytes, stream),
               "nca_bptt_forward_ws")
    # fp32 master weights for the backward GEMMs (rounded to bf16 on load for bf16 cells)
    params = _params(model)
    master = [p.detach().to(dev, torch.float32).contiguous() for p in params]
    wts = _lib.CellWeights(*[m.data_ptr() for m in master], None)
    if accumulate_into is not None:
        acc = list(accumulate_into)
        if len(acc) != len(params) or any(
                a.dtype != torch.float32 or a.device != dev or not a.is_contiguous() or a.shape != p.shape
                for a, p in zip(acc, params)):
            raise ValueError("accumulate_into: the parameters' contiguous fp32 gradients on the device")
        grads = None
        gs = _lib.CellGrads(*[a.data_ptr() for a in acc], 1)
    else:
        grads = {name: torch.empty(p.shape, dtype=torch.float32, device=dev)
                 for name, p in zip(_GRAD_NAMES, params)}
        gs = _lib.CellGrads(*[grads[k].data_ptr() for k in _GRAD_NAMES], 0)
    gx0 = torch.empty_like(xs) if want_grad_x0 else None
    loss = torch.empty((), dtype=torch.float32, device=dev)
    lossd = _lib.BpttLoss(tg.data_ptr(), _lib.ptr(lm), w_host.ctypes.data_as(ctypes.c_void_p))
    _lib.check(L.nca_bptt_backward(ctypes.byref(pk.desc), pk.buf.data_ptr(), ctypes.byref(wts), B,
                                   H, W, states.data_ptr(), g8.data_ptr(), ctypes.byref(fd), n,
                                   ctypes.byref(lossd), _lib.ptr(gf), ctypes.byref(gs),
                                   _lib.ptr(gx0), loss.data_ptr(), ws.data_ptr(), ws_bytes,
                                   stream), "nca_bptt_backward")
    # the status words of the forward's pieces (bytes 0 .. 3, which the backward leaves alone) and of
    # the one-launch backward's (bytes 8 .. 11; zero when it did not run in pieces), in one test
    flags = ws[:3].view(torch.int32)[0::2] != 0
    halo_failed, back_repaired = flags[0:1], flags[1:2]
    # no wait: the host arrays were read during the calls, and the device buffers freed here are
    # reused only by later work on the same stream
    return ChunkResult(states[n].clone(), loss, grads, gx0, states.numel() * 4, ws_bytes,
                       halo_failed, back_repaired)


# ------------------------------------------------------------------------------ losses
def cell_loss(model, x, targets, kind: str) -> torch.Tensor:
    """(B, H, W) loss of every cell (reference src/nca/train.py:183-193): squared distance of the
    output slice to the target token's embedding, summed ("mse") or averaged ("mse_mean") over
    the output channels, or the cross-entropy of the mlp head's logits ("ce")."""
    cfg = model.cfg
    out = x[:, cfg.out_slice]
    if kind in ("mse", "mse_mean"):
        sq = (out - model.target_embedding(targets)).square()
        return sq.sum(dim=1) if kind == "mse" else sq.mean(dim=1)
    if kind == "ce":
        if cfg.head != "mlp":
            raise ValueError("the cross-entropy loss needs an mlp head")
        logits = F.conv2d(out, model.head.weight, model.head.bias)
        return F.cross_entropy(logits, model.output_index(targets), reduction="none")
    raise ValueError(f"unknown loss {kind!r} (ce | mse | mse_mean)")


def step_loss(model, x, targets, kind: str, loss_mask=None) -> torch.Tensor:
    """`cell_loss` averaged over the cells, or over the loss mask's weight (reference
    src/nca/train.py:196-207)."""
    per_cell = cell_loss(model, x, targets, kind)
    if loss_mask is None:
        return per_cell.mean()
    return (per_cell * loss_mask).sum() / loss_mask.sum().clamp_min(1)


# ------------------------------------------------------------------------------ the engine
@dataclass
class EngineConfig:
    """The reference's engine options (reference src/nca/engine/engine.py:59-92), same fields
    and defaults, so that a training config's `engine:` section loads unchanged. On the HIP
    engine the backend switches and the compile / checkpoint / graph options have no effect:
    there is one fused backend, and the BPTT chunk keeps only its states and recomputes the rest
    in its backward. `update_after_rollout` is honoured; `microbatch` is refused (the chunk's
    memory is states only, so a batch does not need splitting)."""

    backend: str = "fused"
    compile: bool = False
    block: int = 1
    compile_mode: str | None = None
    compile_backward_only: bool = False
    checkpoint_segment: int | str | None = "auto"
    checkpoint_candidates: tuple = (1, 2, 4, 8, 16, 32)
    vram_budget: float = 0.85
    update_after_rollout: bool = True
    project_before_pad: bool | None = None
    fused_mix: bool | None = None
    fused_update: bool | None = None
    kernel_mix: bool = False
    kernel_backward: bool | str = False
    triton_mix: bool = False
    microbatch: int | None = None
    checkpoint_recursive: bool = False
    channels_last: bool = False
    normalized_backward: bool = False
    compile_update: bool = False
    sparse_mlp: bool = False
    sparse_sobel: bool = False
    cache_fire: bool = False
    checkpoint_mlp: bool = False
    skip_zero_loss: bool = False
    linear_mlp: bool = False
    clone_microbatch_grads: bool = False
    linear_value: bool = False
    attention_split_k: int = 1
    iteration_graph: bool = False
    triton_mlp: bool = False
    dynamo_cache_size: int = 64

    def __post_init__(self) -> None:
        if self.backend not in ("reference", "fused", "hip"):
            raise ValueError(f"unknown backend {self.backend!r} (reference | fused | hip)")
        if self.block < 1:
            raise ValueError("block must be >= 1")
        if self.microbatch is not None:
            raise ValueError("microbatch is not implemented by the HIP engine (the chunk keeps "
                             "only its states, so the batch is not split)")
        self.checkpoint_candidates = tuple(int(c) for c in self.checkpoint_candidates)

    @classmethod
    def from_dict(cls, d: dict | None) -> EngineConfig:
        return cls(**(d or {}))

    def to_dict(self) -> dict:
        return asdict(self)


@dataclass
class StepDraw:
    """The random tensors of one step (reference src/nca/engine/rng.py:42-48)."""

    fire: torch.Tensor                 # (B, 1, H, W) float in {0, 1}
    noise: torch.Tensor | None         # (B, C, H, W) or None
    noise_mask: torch.Tensor | None    # (B, 1, H, W) bool or None


def _noise_active(noise: dict | None) -> bool:
    return noise is not None and all(noise[k] > 0 for k in ("sigma", "p_t", "p_s"))


class Engine:
    """The reference engine's training interface (reference src/nca/engine/engine.py:167-517)
    on the HIP kernels. `train_cfg` is the resolved `train` section: `rollout`, `chunk`, `amp`,
    `loss`, and `noise` / `perturb` for step noise."""

    def __init__(self, model, cfg: EngineConfig | None, train_cfg: dict, device=None):
        from .step import make_step

        model.kernel_support()
        self.model = model
        self.cfg = cfg if cfg is not None else EngineConfig()
        self.tr = train_cfg
        self.device = torch.device(device) if device is not None else model.device
        self.N, self.Nc = int(train_cfg["rollout"]), int(train_cfg["chunk"])
        if not 1 <= self.Nc <= self.N:
            raise ValueError("need 1 <= chunk <= rollout")
        self.loss_kind = train_cfg.get("loss", "ce")
        if self.loss_kind not in ("ce", "mse", "mse_mean"):
            raise ValueError(f"unknown loss {self.loss_kind!r} (ce | mse | mse_mean)")
        if self.loss_kind == "ce" and model.cfg.head != "mlp":
            raise ValueError("the cross-entropy loss needs an mlp head")
        if self.loss_kind != "ce" and model.cfg.head not in ("l2", "cosine"):
            raise ValueError("the MSE losses compare the output slice with token embeddings: "
                             "they need an embedding head (l2)")
        self.step = make_step(model)
        self.segment = None  # what the reference's EngineState reports: no checkpoint segments
        self.last_chunk: ChunkResult | None = None
        self._weights_host = None

    @property
    def p_fire(self) -> float:
        return self.model.cfg.fire_rate

    @property
    def noise_cfg(self) -> dict | None:
        """Step noise of the rollout (reference engine.py:215-219): `noise` unless `perturb` is
        off; None when inactive."""
        noise = self.tr.get("noise") if self.tr.get("perturb", True) else None
        return noise if _noise_active(noise) else None

    @property
    def fused_chunk(self) -> bool:
        """Does the chunk run on the fused chunk operator (else step by step)?"""
        return self.loss_kind == "ce" and self.model.cfg.head == "mlp" and self.noise_cfg is None

    def to_dict(self) -> dict:
        return {"config": self.cfg.to_dict(), "fused_chunk": self.fused_chunk, "segment": None}

    # ------------------------------------------------------------------ random draws
    def draw(self, seed: int, step: int, shape) -> StepDraw:
        """Fire mask and noise of global step `step` whose seed is `seed`."""
        B, C, H, W = shape
        fire = fire_mask(B, H, W, int(seed), int(step), self.p_fire, device=self.device)
        noise = self.noise_cfg
        if noise is None:
            return StepDraw(fire, None, None)
        gen = torch.Generator(device=self.device)
        gen.manual_seed(int(seed))
        dev = self.device
        hit = torch.rand((B, 1, 1, 1), generator=gen, device=dev) < noise["p_t"]
        cells = torch.rand((B, 1, H, W), generator=gen, device=dev) < noise["p_s"]
        mask = hit & cells
        g = torch.randn((B, C, H, W), generator=gen, device=dev)
        return StepDraw(fire, g * (noise["sigma"] * mask.to(g.dtype)), mask)

    # ------------------------------------------------------------------ running steps
    def forward_steps(self, x, given4, clamp, seeds, step0: int):
        """The steps `seeds` (global steps step0, step0 + 1, ...) without gradient, in fp32 (the
        reference runs the steps outside the chunk without autocast, engine.py:285-292): one
        fused launch, or step by step when step noise is drawn."""
        if len(seeds) == 0:
            return x
        with torch.no_grad():
            if self.noise_cfg is None:
                y, _, _ = rollout_steps(self.model, x, given4, clamp, len(seeds),
                                        step_seeds=np.asarray(seeds, dtype=np.int64),
                                        step0=step0, p_fire=self.p_fire, precision="fp32",
                                        want_conf=False)
                return y
            for i, s in enumerate(seeds):
                d = self.draw(s, step0 + i, x.shape)
                x = self.step(x, given4, clamp, d.fire, d.noise, d.noise_mask)
            return x

    def _host_weights(self, weights) -> np.ndarray:
        """The loss weights on the host, copied once per weights tensor version (the training
        loop passes the same tensor every iteration)."""
        if not torch.is_tensor(weights):
            return np.asarray(weights, dtype=np.float32)
        c = self._weights_host
        key = (id(weights), weights._version, weights.data_ptr())
        if c is None or c[0] != key:
            c = (key, weights.detach().cpu().numpy().astype(np.float32))
            self._weights_host = c
        return c[1]

    def _chunk_steps(self, x, batch, seeds, step0, weights, precision):
        """The chunk step by step through the differentiable step; returns (x, loss)."""
        model = self.model
        given4, clamp, targets = batch["given4"], batch["clamp"], batch["targets"]
        loss_mask = batch.get("loss_mask")
        x = x.detach()
        total = None
        for i, s in enumerate(seeds):
            d = self.draw(s, step0 + i, x.shape)
            x = self.step(x, given4, clamp, d.fire, d.noise, d.noise_mask)
            if weights[i] == 0:
                continue
            term = float(weights[i]) * step_loss(model, x, targets, self.loss_kind, loss_mask)
            total = term if total is None else total + term
        if total is None:  # no supervised step: a zero loss that still reaches the parameters
            total = sum(p.sum() for p in model.parameters()) * 0.0
        return x, total / max(float(np.sum(weights)), 1.0)

    def train_iteration(self, batch: dict, seeds, c0: int, weights, grad_clip,
                        apply_update=None):
        """Roll the batch out for `rollout` steps with the BPTT chunk at `[c0, c0 + chunk)`,
        add the chunk loss's gradients to the parameters' `.grad`, clip them to `grad_clip`
        (if not None) and call `apply_update(grad_norm)` after the rollout or, with
        `update_after_rollout` off, right after the backward. Returns (final state, loss, grad
        norm) as device tensors, with no host synchronisation (reference engine.py:366-517)."""
        model = self.model
        seeds = np.asarray(seeds, dtype=np.int64)
        if len(seeds) != self.N:
            raise ValueError(f"need {self.N} step seeds")
        if not 0 <= c0 <= self.N - self.Nc:
            raise ValueError("the chunk must lie inside the rollout")
        given4, clamp = batch["given4"], batch["clamp"]
        lo, hi = c0, c0 + self.Nc
        w = self._host_weights(weights)
        if len(w) != self.Nc:
            raise ValueError("need one loss weight per chunk step")
        precision = "bf16" if self.tr.get("amp", False) else "fp32"
        x = self.forward_steps(batch["x"], given4, clamp, seeds[:lo], 0)
        if self.fused_chunk:
            params = _params(model)
            # the gradients are added straight into .grad where every parameter has an fp32 one
            # (optim.FusedUpdate's views of its flat buffer), else into .grad afterwards
            into = [p.grad for p in params]
            direct = all(g is not None and g.dtype == torch.float32 and g.is_contiguous() and g.device == x.device
                         for g in into)
            res = bptt_chunk(model, x, given4, clamp, model.output_index(batch["targets"], torch.int32), w,
                             step_seeds=seeds[lo:hi], step0=lo, p_fire=self.p_fire,
                             precision=precision, loss_mask=batch.get("loss_mask"),
                             accumulate_into=into if direct else None)
            self.last_chunk = res
            if not direct:
                # added into existing gradients in place (one launch), so a gradient that is a view
                # of a flat buffer stays one
                grads = [res.grads[n].reshape(p.shape).to(p.dtype) for n, p in zip(_GRAD_NAMES, params)]
                have = [(p.grad, g) for p, g in zip(params, grads) if p.grad is not None]
                if have:
                    torch._foreach_add_([a for a, _ in have], [g for _, g in have])
                for p, g in zip(params, grads):
                    if p.grad is None:
                        p.grad = g
            x, loss = res.x, res.loss
        else:
            with torch.enable_grad():
                x, loss = self._chunk_steps(x, batch, seeds[lo:hi], lo, w, precision)
                loss.backward()
            x, loss = x.detach(), loss.detach()
        if grad_clip is not None:
            gn = torch.nn.utils.clip_grad_norm_(model.parameters(), grad_clip)
        else:
            gn = self.__dict__.get("_zero_norm")
            if gn is None or gn.device != loss.device:
                gn = self._zero_norm = loss.new_zeros(())
        if apply_update is not None and not self.cfg.update_after_rollout:
            apply_update(gn)
        x = self.forward_steps(x, given4, clamp, seeds[hi:], hi)
        if apply_update is not None and self.cfg.update_after_rollout:
            apply_update(gn)
        return x, loss, gn


# ------------------------------------------------------------------------------ replay pool
class ReplayPool:
    """Replay buffer of (state, board) pairs (reference src/nca/pool.py:26-204) for boards given
    as numpy (N, H, W) token grids with a boolean `given` mask (`tasks.Boards`), kept on the
    model's device. Entries carry the state x, given4, clamp, inputs, targets, an optional
    loss_mask (from the boards' meta) and their age in rollouts."""

    KEYS = ("x", "given4", "clamp", "inputs", "targets", "loss_mask")

    def __init__(self, model, boards, size: int, rng: np.random.Generator,
                 generator: torch.Generator | None = None, task=None, augment: bool = False):
        self.model, self.boards, self.size, self.rng = model, boards, size, rng
        self.generator, self.task, self.augment = generator, task, augment
        self.device = model.device
        # tensors of their own (fresh's are views of one upload, which a checkpoint cannot hold)
        for key, value in self.fresh(size).items():
            setattr(self, key, None if value is None else value.clone())
        self.age = torch.zeros(size, dtype=torch.long, device=self.device)

    def _upload_many(self, arrays) -> list:
        """Host arrays on the device in one copy (one buffer, each array at a 16-byte boundary),
        as contiguous tensors of their dtypes and shapes (views of that buffer)."""
        arrays = [np.ascontiguousarray(a) for a in arrays]
        offs, total = [], 0
        for a in arrays:
            offs.append(total)
            total += (a.nbytes + 15) & ~15
        host = np.zeros(max(total, 1), np.uint8)
        for a, o in zip(arrays, offs):
            host[o:o + a.nbytes] = a.reshape(-1).view(np.uint8)
        dev = _lib.upload_beside(host, self.device)
        return [dev[o:o + a.nbytes].view(torch.from_numpy(a[:0].reshape(-1)).dtype).view(a.shape)
                for a, o in zip(arrays, offs)]

    def fresh(self, n: int, extra=()) -> dict:
        """`n` boards drawn uniformly (with replacement) from the board set, augmented when the
        pool has a task that augments, each with a freshly initialised state. The boards' arrays
        (and the host arrays in `extra`, returned under "_extra") go to the device in one copy."""
        picks = self.rng.integers(0, len(self.boards), size=n)
        chosen = self.boards.subset(picks)
        if self.augment and self.task is not None:
            chosen = self.task.augment(chosen, self.rng)
        lm = chosen.meta.get("loss_mask")
        host = [chosen.inputs, chosen.given, chosen.targets]
        if lm is not None:
            host.append(np.asarray(lm, np.float32))
        dev = self._upload_many(host + list(extra))
        inputs, given, targets = dev[:3]
        x, given4, clamp = self.model.init_state(inputs, given, None, self.generator)
        out = {"x": x.detach(), "given4": given4, "clamp": clamp, "inputs": inputs, "targets": targets,
               "loss_mask": None if lm is None else dev[3]}
        if extra:
            out["_extra"] = dev[len(host):]
        return out

    def _rows(self, items, n_rows: int) -> None:
        """One launch of nca_pool_rows over (src, dst, src_row, dst_row, mode) items (a pool on a
        CPU device indexes with torch)."""
        if self.device.type != "cuda":
            with torch.no_grad():
                for src, dst, srow, drow, mode in items:
                    if srow is not None:
                        sel = srow >= 0
                        dst[sel] = 0 if mode == 2 else src[srow[sel]]
                    else:
                        dst[drow] = src + 1 if mode == 1 else src
            return
        arr = (_lib.PoolRowCopy * len(items))()
        for i, (src, dst, srow, drow, mode) in enumerate(items):
            if src is not None and (src.dtype != dst.dtype or src.shape[1:] != dst.shape[1:]):
                raise ValueError("pool rows: dtype or row shape mismatch")
            if not dst.is_contiguous() or (src is not None and not src.is_contiguous()):
                raise ValueError("pool rows: tensors must be contiguous")
            arr[i] = _lib.PoolRowCopy(None if src is None else src.data_ptr(), dst.data_ptr(),
                                      None if srow is None else srow.data_ptr(),
                                      None if drow is None else drow.data_ptr(),
                                      dst[0].numel() * dst.element_size(), mode)
        _lib.check(_lib.load().nca_pool_rows(arr, len(items), n_rows, _lib.stream_of(self.device)),
                   "nca_pool_rows")

    def sample(self, batch_size: int, seed_ratio: float):
        """`batch_size` distinct pool entries (copies), of which the first
        round(seed_ratio * batch_size) are replaced by fresh boards of age 0. Returns (pool
        indices, batch dict)."""
        idx = self.rng.choice(self.size, size=batch_size, replace=False)
        n_new = int(round(seed_ratio * batch_size))
        # row maps: the pool rows (idx), the pool row of each batch row (-1 for the fresh ones)
        # and the fresh row of each batch row (-1 for the others); one upload with the boards
        maps = np.full((3, batch_size), -1, np.int64)
        maps[0] = idx
        maps[1, n_new:] = idx[n_new:]
        maps[2, :n_new] = np.arange(n_new)
        if n_new > 0:
            new = self.fresh(n_new, extra=(maps,))
            maps_d = new.pop("_extra")[0]
        else:
            new, maps_d = {}, _lib.upload(maps, self.device)
        batch, items = {}, []
        for k in self.KEYS + ("age",):
            src = getattr(self, k)
            if src is None:
                batch[k] = None
                continue
            batch[k] = torch.empty((batch_size,) + tuple(src.shape[1:]), dtype=src.dtype, device=src.device)
            items.append((src, batch[k], maps_d[1], None, 0))
            if n_new > 0:
                if k == "age":
                    items.append((None, batch[k], maps_d[2], None, 2))  # fresh boards: age 0
                else:
                    items.append((new[k], batch[k], maps_d[2], None, 0))
        self._rows(items, batch_size)
        self._last_rows = (idx, maps_d[0])
        return idx, batch

    def replace_boards(self, batch: dict, which: np.ndarray) -> None:
        """Target swap with fresh boards: samples `which` get a new board (given cells, clamp
        values, inputs, targets, loss mask) and keep their state, re-clamped
        (reference pool.py:123-135)."""
        if len(which) == 0:
            return
        new = self.fresh(len(which))
        sel = _lib.upload(np.asarray(which), self.device)
        for k in ("given4", "clamp", "inputs", "targets", "loss_mask"):
            if batch.get(k) is not None:
                batch[k][sel] = new[k]
        batch["x"] = self.model.apply_clamp(batch["x"], batch["given4"], batch["clamp"])

    def swap_from_pool(self, batch: dict, which: np.ndarray) -> None:
        """Target swap from the pool (reference pool.py:137-165): samples `which` take the board
        of a uniformly drawn pool entry and that entry's input channels on its given cells; the
        rest of their state is kept and their age restarts at 0."""
        if len(which) == 0:
            return
        src = _lib.upload(self.rng.integers(0, self.size, size=len(which)), self.device)
        sel = _lib.upload(np.asarray(which), self.device)
        for k in ("given4", "clamp", "inputs", "targets", "loss_mask"):
            if batch.get(k) is not None:
                batch[k][sel] = getattr(self, k)[src]
        batch["age"][sel] = 0
        sl = self.model.cfg.in_slice
        g = batch["given4"][sel]
        batch["x"][sel, sl] = torch.where(g, self.x[src][:, sl], batch["x"][sel, sl])
        batch["x"] = self.model.apply_clamp(batch["x"], batch["given4"], batch["clamp"])

    def write_back(self, idx, batch: dict) -> None:
        """Store the batch's post-rollout states and boards at the pool indices they came from,
        one rollout older (reference pool.py:166-179)."""
        last = getattr(self, "_last_rows", None)
        rows = last[1] if last is not None and last[0] is idx else _lib.upload(np.asarray(idx, np.int64), self.device)
        items = []
        for k in self.KEYS:
            if getattr(self, k) is not None and batch.get(k) is not None:
                items.append((batch[k].detach().contiguous(), getattr(self, k), None, rows, 0))
        items.append((batch["age"].contiguous(), self.age, None, rows, 1))  # one rollout older
        self._rows(items, len(idx))

    def state_dict(self) -> dict:
        return {k: getattr(self, k) for k in self.KEYS + ("age",)}

    def load_state_dict(self, d: dict) -> None:
        for k, v in d.items():
            setattr(self, k, None if v is None else v.to(self.device))
