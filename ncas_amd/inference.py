"""Fused forward rollouts: many NCA steps in one launch of the LDS-resident HIP kernel.

* `rollout_steps(model, x, given4, clamp, n_steps, ...)` - the rollout operator: `n_steps`
  steps of every row with Philox fire masks keyed on (seed, row, step, cell) (or injected
  masks), returning the final state, the board confidence of the final state and the number of
  fired cells per row. Replaces the per-step Python loops of the reference (reference
  src/nca/engine/inference.py:9-24, src/nca/rollout.py:203-247).
* `InferenceEngine(model, config, amp)(batch, seeds) -> (x, clock)` - the reference's
  forward-only runner (reference src/nca/engine/inference.py:27-71): one Philox key per step
  (`seeds`, as from `rng.step_seeds`), fire rate `model.cfg.fire_rate`, bf16 when `amp`.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from .rng import fire_desc


def rollout_steps(
    model,
    x: torch.Tensor,
    given4: torch.Tensor,
    clamp: torch.Tensor,
    n_steps: int,
    *,
    seed: int = 0,
    p_fire: float | None = None,
    p_low: float | None = None,
    tau: float | None = None,
    given_confident: bool = True,
    row0: int = 0,
    step0: int = 0,
    step_seeds=None,
    masks: torch.Tensor | None = None,
    precision: str = "fp32",
    out: torch.Tensor | None = None,
    want_conf: bool = True,
    want_fired: bool = False,
):
    """Returns (x_out, conf (B,) or None, fired (B,) int32 or None).

    `masks` (n_steps, B, 1, H, W) injects the fire masks; `step_seeds` (n_steps,) int64 gives
    one Philox key per step (otherwise `seed` keys every step). `out` may alias `x`."""
    dev = _lib.require_device(x, given4, clamp, masks, out)
    if torch.is_grad_enabled() and (
        x.requires_grad or any(p.requires_grad for p in model.parameters())
    ):
        raise NotImplementedError("the HIP rollout is forward-only; call it under torch.no_grad()")
    cfg = model.cfg
    B, C, H, W = x.shape
    if C != cfg.channels:
        raise ValueError(f"state has {C} channels, the model {cfg.channels}")
    if given4.shape != (B, 1, H, W):
        raise ValueError("given4 must be (B, 1, H, W)")
    if clamp.shape != (B, cfg.c_in, H, W):
        raise ValueError(f"clamp must be {(B, cfg.c_in, H, W)}")
    if n_steps < 0:
        raise ValueError("n_steps must be >= 0")
    pk = model.packed(precision, dev)
    xs = x.detach()
    if xs.dtype != torch.float32 or not xs.is_contiguous():
        xs = xs.to(torch.float32).contiguous()
    g8 = given4.detach().to(torch.uint8).contiguous()
    cl = clamp.detach().to(torch.float32).contiguous()
    m8 = None
    if masks is not None:
        if masks.shape[0] != n_steps or masks[0].numel() != B * H * W:
            raise ValueError("masks must be (n_steps, B, 1, H, W)")
        if p_low is not None:
            raise ValueError("adaptive firing draws its own masks")
        m8 = (masks.detach() != 0).to(torch.uint8).contiguous()
    ss = None
    if step_seeds is not None:
        ss = _lib.upload(np.asarray(step_seeds, dtype=np.int64), dev)
        if ss.numel() != n_steps:
            raise ValueError("step_seeds must have n_steps entries")
    if out is None:
        out = torch.empty_like(xs)
    elif out.shape != xs.shape or out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError("out must be a contiguous fp32 tensor shaped like x")
    conf = torch.empty((B,), dtype=torch.float32, device=dev) if want_conf else None
    fired = torch.empty((B,), dtype=torch.int32, device=dev) if want_fired else None
    fd = fire_desc(seed, cfg.fire_rate if p_fire is None else p_fire, p_low, tau,
                   given_confident, row0, step0, ss, m8)
    L = _lib.load()
    # rows that do not fit one workgroup's LDS run step by step through a workspace buffer
    ws_bytes = L.nca_rollout_workspace_bytes(ctypes.byref(pk.desc), B, H, W)
    ws = torch.empty((ws_bytes // 4,), dtype=torch.float32, device=dev) if ws_bytes else None
    _lib.check(
        L.nca_rollout_ws(
            ctypes.byref(pk.desc), pk.buf.data_ptr(), B, H, W, xs.data_ptr(), g8.data_ptr(),
            cl.data_ptr(), out.data_ptr(), ctypes.byref(fd), int(n_steps), None,
            _lib.ptr(conf), _lib.ptr(fired), _lib.ptr(ws), ws_bytes, _lib.stream_of(dev),
        ),
        "nca_rollout_ws",
    )
    return out, conf, fired


class InferenceEngine:
    """Forward-only multi-step runner (reference src/nca/engine/inference.py:27-71)."""

    def __init__(self, model, config=None, amp: bool = False, noise=None):
        if noise is not None:
            raise ValueError("rollout noise is not implemented by the HIP engine")
        model.kernel_support()
        self.model, self.config, self.amp, self.noise = model, config, amp, noise

    @torch.no_grad()
    def __call__(self, batch: dict, seeds):
        x = batch["x"]
        seeds = np.asarray(seeds, dtype=np.int64)
        out, _, _ = rollout_steps(
            self.model, x, batch["given4"], batch["clamp"], len(seeds), step_seeds=seeds,
            precision="bf16" if self.amp else "fp32", want_conf=False,
        )
        return out, None
