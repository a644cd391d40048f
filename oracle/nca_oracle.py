"""The NCA cell step and rollout restated in PyTorch-CPU (oracle: test infrastructure only).

Restates the reference's `src/nca/model.py` for the "kernels" perception + ReLU MLP cell with
no group normalisation and no time embedding (the cells of the north-star configurations and
of the reference's maze presets):

* `pad`            - model.py:140-152 (wall / wrap / zero, 1-cell border);
* `perceive`       - model.py:161-178 (K shared 3x3 kernels, cross-correlation, head-major
                     output `z[:, k*C + c]`, computed as `F.conv2d` over B*C single-channel
                     images exactly like the reference);
* `mlp`            - model.py:277-287 (1x1 fc1 -> ReLU -> 1x1 fc2);
* `step`           - model.py:503-559 (`x + fire * dx`, optional noise, clamp of the input
                     slice of given cells, model.py:430-438);
* `rollout`        - the per-step loop of rollout.py:203-247 / engine/inference.py:9-24 with
                     `x.float()` after every step (engine/step.py:240-242), fire masks drawn
                     from the Philox rule (`oracle/philox.py`) instead of torch's generator;
* `readout`        - model.py:596-633 through the C restatement (`nca_oracle.c`), whose fixed
                     operation order is what the GPU readout must match bit for bit;
* `chunk_loss`,
  `bptt_chunk`     - the BPTT chunk of engine.py:366-517: `n` steps with gradient, loss
                     sum_t w_t * step_loss(x_{t+1}) / sum_t w_t with the per-cell cross-entropy of
                     the mlp head's logits (train.py:183-207, step.py:243-245), differentiated by
                     torch autograd in fp64 (the parameters, and optionally x_0).

Precision modes: "fp32" and "fp64" compute everything in that type. "bf16" reproduces the
rounding points of the reference under `torch.autocast(bfloat16)` (engine/step.py:240-242,
ops.py:237): the perception input and the kernels are rounded to bf16 (autocast casts a conv's
operands), z, h (fc1 output, ReLU applied in bf16) and dx (fc2 output) are bf16, products are
exact in fp32 and accumulate in fp32, and the residual update and clamp stay fp32. The bf16
chunk's gradients go straight through the rounding points (`ste`); with `grad_round` the
gradients reaching dx, h and z are rounded to bf16 as in the reference's bf16 backward
(engine/triton_mlp.py:46-78), pinned against a written-out numpy backward in
tests/test_oracle_bptt.py.

Cells are described by `OracleCell`, a plain record of tensors, so that the oracle does not
depend on the product's classes.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F

from . import clib
from . import philox as np_philox

PADDING = ("zero", "wall", "wrap")


@dataclass
class OracleCell:
    channels: int
    heads: int
    hidden: int
    c_in: int
    in_offset: int
    c_out: int
    out_offset: int
    padding: str  # "zero" | "wall" | "wrap"
    head: str  # "mlp" | "l2"
    kernels: torch.Tensor  # (heads, 1, 3, 3)
    w1: torch.Tensor  # (hidden, heads * channels)
    b1: torch.Tensor  # (hidden,)
    w2: torch.Tensor  # (channels, hidden)
    b2: torch.Tensor  # (channels,)
    head_w: torch.Tensor  # mlp: (n_out, c_out) linear head; l2: (n_out, c_out) token embeddings
    head_b: torch.Tensor | None  # mlp: (n_out,)
    pad_vec: torch.Tensor  # (channels,) wall border value

    @property
    def head_kind(self) -> int:
        return {"mlp": 0, "l2": 1}[self.head]


def _bf(t: torch.Tensor) -> torch.Tensor:
    """Round to bf16 (round to nearest even) and return as fp32."""
    return t.to(torch.bfloat16).to(torch.float32)


def pad(x: torch.Tensor, mode: str, pad_vec: torch.Tensor | None) -> torch.Tensor:
    """model.py:140-152."""
    if mode == "wrap":
        return F.pad(x, (1, 1, 1, 1), mode="circular")
    xp = F.pad(x, (1, 1, 1, 1))
    if mode == "wall":
        v = pad_vec.to(xp.dtype)[None, :, None]
        xp[:, :, 0, :] = v
        xp[:, :, -1, :] = v
        xp[:, :, :, 0] = v
        xp[:, :, :, -1] = v
    return xp


def perceive(xp: torch.Tensor, kernels: torch.Tensor, H: int, W: int) -> torch.Tensor:
    """model.py:175-178: (B, C, H+2, W+2) -> (B, K*C, H, W), head-major."""
    B, C = xp.shape[:2]
    K = kernels.shape[0]
    z = F.conv2d(xp.reshape(B * C, 1, H + 2, W + 2), kernels.to(xp.dtype))
    return z.view(B, C, K, H, W).transpose(1, 2).reshape(B, K * C, H, W)


def _dtype(precision: str) -> torch.dtype:
    return torch.float64 if precision == "fp64" else torch.float32


class _RoundBF16(torch.autograd.Function):
    """Round to bf16 with an identity backward: the exact gradient of the rounded forward (the
    rounding is piecewise constant, so its derivative is taken as 1, i.e. straight-through)."""

    @staticmethod
    def forward(ctx, t):
        return t.to(torch.bfloat16).to(t.dtype)

    @staticmethod
    def backward(ctx, g):
        return g


class _RoundBF16Grad(torch.autograd.Function):
    """Round to bf16 in the forward and round the incoming gradient to bf16 in the backward: the
    gradient of a bf16 tensor of the reference's autocast step is itself bf16 (a bf16 op's
    backward produces bf16 gradients), so the gradients reaching dx (fc2's output), h (fc1's
    output) and z (the perception's output) are rounded there. The Triton MLP backward of the
    reference's fused engine rounds at the same points: G = grad(dx) in bf16, gh = bf16(G W2)
    masked by h > 0, gx = bf16(gh W1) (reference src/nca/engine/triton_mlp.py:46-78)."""

    @staticmethod
    def forward(ctx, t):
        return t.to(torch.bfloat16).to(t.dtype)

    @staticmethod
    def backward(ctx, g):
        return g.to(torch.bfloat16).to(g.dtype)


# fp32 summation orders of the bf16 step: torch's own, one rounding of the exact sum, and blocks
# of 32 or 8 products (each block's exact sum rounded to fp32, the blocks added in fp32 in
# ascending or, "r" prefix, descending order)
SUM_ORDERS = ("torch", "exact", "block32", "block8", "rblock32")


def _blocks(order: str) -> tuple[int, bool]:
    """(block width, descending) of a "block<N>" / "rblock<N>" order."""
    rev = order.startswith("r")
    return int(order[6 if rev else 5:]), rev


def _perceive_ordered(xp: torch.Tensor, k: torch.Tensor, H: int, W: int, order: str):
    """`perceive` with another fp32 summation order of the 9 taps: "exact" sums the (exact)
    products in fp64 and rounds once; the block orders add them one by one in fp32 in row-major
    tap order (descending for "r" orders)."""
    if order == "exact":
        return perceive(xp.double(), k.double(), H, W).to(xp.dtype)
    _, rev = _blocks(order)
    B, C = xp.shape[:2]
    K = k.shape[0]
    acc = torch.zeros((B, K, C, H, W), dtype=xp.dtype)
    taps = [(dy, dx) for dy in range(3) for dx in range(3)]
    for dy, dx in (taps[::-1] if rev else taps):
        tap = xp[:, None, :, dy:dy + H, dx:dx + W]
        acc = acc + tap * k[:, 0, dy, dx].to(xp.dtype)[None, :, None, None, None]
    return acc.reshape(B, K * C, H, W)


def _linear_ordered(a: torch.Tensor, w: torch.Tensor, b: torch.Tensor, order: str):
    """a @ w.T + b with another fp32 summation order: "exact" sums every dot product and its
    bias in fp64 and rounds once; a block order rounds each block of N products' exact sum to
    fp32 and adds the blocks one by one to the bias in fp32."""
    if order == "exact":
        return (a.double() @ w.double().T + b.double()).to(a.dtype)
    n, rev = _blocks(order)
    acc = b.to(a.dtype).expand(a.shape[0], w.shape[0]).clone()
    starts = list(range(0, a.shape[1], n))
    for k0 in (starts[::-1] if rev else starts):
        acc = acc + (a[:, k0:k0 + n].double() @ w[:, k0:k0 + n].double().T).to(a.dtype)
    return acc


def sense_update(cell: OracleCell, x: torch.Tensor, precision: str = "fp32",
                 dtype: torch.dtype | None = None, ste: bool = False,
                 grad_round: bool = False, order: str = "torch") -> torch.Tensor:
    """Perception + MLP: the proposed dx of every cell (model.py:489-495). `dtype` overrides the
    compute type (fp64 for gradients); `ste` makes the bf16 rounding points straight-through;
    `grad_round` (with `ste`) also rounds the gradients of z, h and dx to bf16, the reference's
    bf16 backward (the perception input's and the weights' gradients stay unrounded). `order`
    changes only the fp32 summation order of the stencil and the two linear layers ("torch":
    torch's conv2d and GEMM; the others: see `_perceive_ordered`, `_linear_ordered`),
    which measures how far two correct fp32 implementations of the same bf16 step drift apart."""
    B, C, H, W = x.shape
    dt = dtype or _dtype(precision)
    bf = precision == "bf16"
    if order not in SUM_ORDERS:
        raise ValueError(f"order {order!r}")
    _bf = _RoundBF16.apply if ste else globals()["_bf"]
    _bfg = _RoundBF16Grad.apply if (ste and grad_round) else _bf
    x = x.to(dt)
    xp = pad(x, cell.padding, cell.pad_vec.to(dt))
    k = cell.kernels.to(dt)
    if bf:
        xp, k = _bf(xp), _bf(k)
    z = perceive(xp, k, H, W) if order == "torch" else _perceive_ordered(xp, k, H, W, order)
    if bf:
        z = _bfg(z)
    rows = z.permute(0, 2, 3, 1).reshape(-1, z.shape[1])
    w1, b1, w2, b2 = (t.to(dt) for t in (cell.w1, cell.b1, cell.w2, cell.b2))
    if bf:
        w1, b1, w2, b2 = _bf(w1), _bf(b1), _bf(w2), _bf(b2)
    h = rows @ w1.T + b1 if order == "torch" else _linear_ordered(rows, w1, b1, order)
    if bf:
        h = _bfg(h)
    h = torch.relu(h)
    dx = h @ w2.T + b2 if order == "torch" else _linear_ordered(h, w2, b2, order)
    if bf:
        dx = _bfg(dx)
    return dx.reshape(B, H, W, C).permute(0, 3, 1, 2)


def apply_clamp(cell: OracleCell, x, given4, clamp):
    """model.py:430-438."""
    sl = slice(cell.in_offset, cell.in_offset + cell.c_in)
    out = x.clone()
    out[:, sl] = torch.where(given4, clamp.to(x.dtype), x[:, sl])
    return out


def step(cell: OracleCell, x, given4, clamp, fire, precision="fp32", noise=None, dtype=None, ste=False,
         grad_round=False, order="torch"):
    """One step (model.py:503-559 without time embedding / normalisation). fire: (B,1,H,W)."""
    dt = dtype or _dtype(precision)
    x = x.to(dt)
    dx = sense_update(cell, x, precision, dtype, ste, grad_round, order)
    u = x + fire.to(dt) * dx.to(dt)
    if noise is not None:
        u = u + noise.to(dt)
    return apply_clamp(cell, u, given4, clamp)


def readout(cell: OracleCell, x: torch.Tensor):
    """(conf_cell, conf_board, argmax) of fp32 states, fixed operation order (nca_oracle.c)."""
    return clib.readout(
        x.detach().to(torch.float32).contiguous().numpy(),
        cell.out_offset,
        cell.c_out,
        cell.head_kind,
        cell.head_w.detach().to(torch.float32).numpy(),
        None if cell.head_b is None else cell.head_b.detach().to(torch.float32).numpy(),
    )


def rollout(
    cell: OracleCell,
    x: torch.Tensor,
    given4: torch.Tensor,
    clamp: torch.Tensor,
    n_steps: int,
    precision: str = "fp32",
    seed: int = 0,
    row0: int = 0,
    step0: int = 0,
    p_fire: float = 0.5,
    p_low: float | None = None,
    tau: float | None = None,
    given_confident: bool = True,
    masks: torch.Tensor | None = None,
    trace=None,
    order: str = "torch",
):
    """`n_steps` steps from x with Philox fire masks (or injected `masks` (n, B, 1, H, W)).

    Returns (x_final fp32, fired per row (B,) int64). `trace(t, x)` is called after each step.
    `order`: the fp32 summation order of every step (`sense_update`).
    Adaptive firing (p_low, tau) reads the pre-step confidence of every cell, like
    rollout.py:220-222 -> model.py:589-593, with given cells counted as confident when
    `given_confident` (rollout.py:36).
    """
    B, C, H, W = x.shape
    x = x.to(_dtype(precision))
    fired = torch.zeros(B, dtype=torch.int64)
    g_np = given4.reshape(B, H * W).numpy().astype(np.uint8)
    for t in range(n_steps):
        if masks is not None:
            fire = masks[t].to(x.dtype)
        else:
            conf = None
            if p_low is not None and tau is not None:
                conf, _, _ = readout(cell, x.to(torch.float32))
            m = clib.fire_mask(
                seed, row0, B, step0 + t, H * W, p_fire, p_low, tau, conf,
                g_np if given_confident else None,
            )
            fire = torch.from_numpy(m.astype(np.float32)).reshape(B, 1, H, W).to(x.dtype)
        fired += fire.reshape(B, -1).sum(1).to(torch.int64)
        x = step(cell, x, given4, clamp, fire, precision, order=order)
        if precision != "fp64":
            x = x.float()
        if trace is not None:
            trace(t, x)
    return x, fired


def chunk_loss(cell: OracleCell, x0, given4, clamp, masks, targets, weights, precision="fp32",
               loss_mask=None, ste=True, final_cotangent=None, grad_round=False,
               dtype=torch.float64):
    """The BPTT chunk's loss (engine.py:474-490 with the chunk's run_block, step.py:236-245):
    `n` steps from x0 with fire masks `masks` (n, B, 1, H, W), then
    L = sum_t w_t * step_loss(x_{t+1}) / max(sum_t w_t, 1), where step_loss is the mean (or the
    loss_mask weighted mean, train.py:196-207) over cells of the cross-entropy of the mlp head's
    logits against `targets` (B, H, W) class indices (train.py:190-192). Computed in fp64,
    differentiable w.r.t. the cell's tensors and x0; bf16 cells round at the forward's points
    (straight-through when `ste`; with `grad_round` the gradients of z, h and dx are rounded to
    bf16 as in the reference's bf16 backward). `final_cotangent` adds sum(x_n * final_cotangent),
    whose gradient w.r.t. the last state is that cotangent (a later loss's gradient). `dtype`:
    the arithmetic type (fp64 for the parity checks; fp32 times the reference's CPU path)."""
    dt = dtype
    x = x0.to(dt)
    w = torch.as_tensor(weights, dtype=dt)
    total = x.new_zeros(())
    sl = slice(cell.out_offset, cell.out_offset + cell.c_out)
    for t in range(masks.shape[0]):
        x = step(cell, x, given4, clamp, masks[t], precision, dtype=dt, ste=ste, grad_round=grad_round)
        if w[t] == 0:
            continue
        logits = torch.einsum("vc,bchw->bvhw", cell.head_w.to(dt), x[:, sl]) \
            + cell.head_b.to(dt)[None, :, None, None]
        per_cell = F.cross_entropy(logits, targets.long(), reduction="none")
        if loss_mask is not None:
            lm = loss_mask.to(dt)
            step_l = (per_cell * lm).sum() / lm.sum().clamp_min(1)
        else:
            step_l = per_cell.mean()
        total = total + w[t] * step_l
    total = total / w.sum().clamp_min(1)
    if final_cotangent is not None:
        total = total + (x * final_cotangent.to(dt)).sum()
    return total


def bptt_chunk(cell: OracleCell, x0, given4, clamp, masks, targets, weights, precision="fp32",
               loss_mask=None, grad_x0=False, ste=True, final_cotangent=None, grad_round=False,
               dtype=torch.float64):
    """`chunk_loss` and its gradients by torch autograd in fp64 (`grad_round`: the reference's
    bf16 gradient rounding points, see `_RoundBF16Grad`; `dtype` float32 sums every product in
    fp32 instead, which measures how much the sums' precision alone moves the result).

    Returns (loss float, grads dict of `dtype` tensors: kernels, w1, b1, w2, b2, head_w, head_b,
    and x0 when grad_x0)."""
    dt = dtype
    names = ("kernels", "w1", "b1", "w2", "b2", "head_w", "head_b")
    params = {k: getattr(cell, k).detach().to(dt).clone().requires_grad_(True) for k in names}
    c = OracleCell(**{**cell.__dict__, **params})
    x = x0.detach().to(dt).clone().requires_grad_(grad_x0)
    loss = chunk_loss(c, x, given4, clamp, masks, targets, weights, precision, loss_mask, ste,
                      final_cotangent, grad_round, dtype=dt)
    wrt = [params[k] for k in names] + ([x] if grad_x0 else [])
    if not loss.requires_grad:  # every step weight is zero: a constant loss
        grads = [None] * len(wrt)
    else:
        grads = torch.autograd.grad(loss, wrt, allow_unused=True)
    out = {k: (g if g is not None else torch.zeros_like(params[k])) for k, g in zip(names, grads)}
    if grad_x0:
        out["x0"] = grads[-1] if grads[-1] is not None else torch.zeros_like(x)
    return float(loss.detach()), out


def conf_at_k(metric, conf, alive, ks, weights=None):
    """rollout.py:317-334 restated (np.argmax: first maximum)."""
    N, K = metric.shape
    out = {}
    for k in ks:
        k = min(k, K)
        c = np.where(alive[:, :k], conf[:, :k], -np.inf)
        best = c.argmax(axis=1)
        out[k] = float(np.average(metric[np.arange(N), best], weights=weights))
    return out


def pass_at_k(metric, alive, ks, weights=None):
    """rollout.py:337-350 restated."""
    N, K = metric.shape
    return {
        min(k, K): float(
            np.average((metric[:, : min(k, K)] & alive[:, : min(k, K)]).any(axis=1),
                       weights=weights)
        )
        for k in ks
    }


def fire_masks_np(seed, row0, rows, step, H, W, p):
    """Uniform-firing mask (rows, 1, H, W) float32 via the numpy Philox."""
    m = np_philox.fire_mask(seed, row0, rows, step, H * W, p)
    return torch.from_numpy(m.astype(np.float32)).reshape(rows, 1, H, W)
