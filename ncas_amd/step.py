"""The step operator: a drop-in for the reference engine's step protocol.

`make_step(model, opts)` returns `step(x, given4, clamp, fire, noise, noise_mask, clock) -> x`,
the signature of the reference's `make_step` (reference src/nca/engine/step.py:74-209, call at
184-207): states (B, C, H, W) fp32, `given4` (B, 1, H, W) bool, `clamp` (B, c_in, H, W),
`fire` (B, 1, H, W) float, optional additive `noise` (B, C, H, W); a new tensor is returned and
the inputs are not modified. The step runs as one launch of the fused HIP kernel
(`nca_step`). Under bf16 autocast (or `precision="bf16"`) the kernel reproduces autocast's
rounding points; the result is fp32 like the reference's `x.float()` (step.py:242).

The HIP step is forward-only: calling it where autograd would need its backward raises.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib


@dataclass(frozen=True)
class StepOptions:
    """Accepted for signature compatibility with the reference's StepOptions
    (reference src/nca/engine/step.py:36-62); the HIP step is a single fused backend, so the
    ablation switches have no effect."""

    project_before_pad: bool = True
    fused_mix: bool = True
    fused_update: bool = True
    kernel_mix: bool = False
    kernel_backward: bool | str = False
    triton_mix: bool = False
    normalized_backward: bool = False
    compile_update: bool = False
    sparse_mlp: bool = False
    sparse_sobel: bool = False
    checkpoint_mlp: bool = False
    linear_mlp: bool = False
    linear_value: bool = False
    attention_split_k: int = 1
    triton_mlp: bool = False

    @classmethod
    def for_backend(cls, backend: str) -> StepOptions:
        if backend not in ("reference", "fused", "hip"):
            raise ValueError(f"unknown backend {backend!r} (reference | fused | hip)")
        return cls()


def _autocast_precision(device: torch.device, precision: str | None) -> str:
    if precision is not None:
        return precision
    if torch.is_autocast_enabled(device.type):
        dt = torch.get_autocast_dtype(device.type)
        if dt != torch.bfloat16:
            raise ValueError(f"autocast dtype {dt} is not implemented (bfloat16 only)")
        return "bf16"
    return "fp32"


def _needs_grad(model, *tensors) -> bool:
    if not torch.is_grad_enabled():
        return False
    if any(t is not None and t.requires_grad for t in tensors):
        return True
    return any(p.requires_grad for p in model.parameters())


def hip_step(model, x, given4, clamp, fire, noise=None, precision=None):
    """One fused step on the GPU (C ABI `nca_step`)."""
    dev = _lib.require_device(x, given4, clamp, fire, noise)
    if _needs_grad(model, x, clamp, noise):
        raise NotImplementedError(
            "the HIP step is forward-only; call it under torch.no_grad() / inference_mode()"
        )
    prec = _autocast_precision(dev, precision)
    cfg = model.cfg
    B, C, H, W = x.shape
    if C != cfg.channels:
        raise ValueError(f"state has {C} channels, the model {cfg.channels}")
    if given4.shape != (B, 1, H, W) or fire.shape[0] != B or fire.numel() != B * H * W:
        raise ValueError("given4 / fire must be (B, 1, H, W)")
    if clamp.shape != (B, cfg.c_in, H, W):
        raise ValueError(f"clamp must be {(B, cfg.c_in, H, W)}, got {tuple(clamp.shape)}")
    pk = model.packed(prec, dev)
    xs = x.detach().to(torch.float32).contiguous()
    g8 = given4.detach().to(torch.uint8).contiguous()
    cl = clamp.detach().to(torch.float32).contiguous()
    fi = fire.detach().to(torch.float32).contiguous()
    nz = None if noise is None else noise.detach().to(torch.float32).contiguous()
    if nz is not None and nz.shape != xs.shape:
        raise ValueError("noise must have the state's shape")
    out = torch.empty_like(xs)
    L = _lib.load()
    _lib.check(
        L.nca_step(ctypes.byref(pk.desc), pk.buf.data_ptr(), B, H, W, xs.data_ptr(),
                   g8.data_ptr(), cl.data_ptr(), fi.data_ptr(), _lib.ptr(nz), out.data_ptr(),
                   _lib.stream_of(dev)),
        "nca_step",
    )
    return out


def make_step(model, opts: StepOptions | None = None, precision: str | None = None):
    """Step function with the reference engine's signature (reference step.py:184-207).
    `noise_mask` is accepted and unused (it only matters with group normalisation, which the
    HIP cell does not have); `clock` must be None (no time embedding)."""
    model.kernel_support()

    def step(x, given4, clamp, fire, noise=None, noise_mask=None, clock=None):
        if clock is not None and model.cfg.time_steps:
            raise ValueError("time embeddings are not implemented")
        return hip_step(model, x, given4, clamp, fire, noise, precision)

    return step
