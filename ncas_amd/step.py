"""The step operator: a drop-in for the reference engine's step protocol.

`make_step(model, opts)` returns `step(x, given4, clamp, fire, noise, noise_mask, clock) -> x`,
the signature of the reference's `make_step` (reference src/nca/engine/step.py:74-209, call at
184-207): states (B, C, H, W) fp32, `given4` (B, 1, H, W) bool, `clamp` (B, c_in, H, W),
`fire` (B, 1, H, W) float, optional additive `noise` (B, C, H, W); a new tensor is returned and
the inputs are not modified. The step runs as one launch of the fused HIP kernel
(`nca_step`). Under bf16 autocast (or `precision="bf16"`) the kernel reproduces autocast's
rounding points; the result is fp32 like the reference's `x.float()` (step.py:242).

Under autograd (a state or a parameter that requires grad, grad mode on) the step is a node
whose backward runs on the GPU too (`nca_step_backward`): the gradients of the state, the clamp
values, the noise and the cell's parameters, like the reference's step (reference
tests/test_engine_ops.py:251-294). bf16 cells differentiate the rounded forward with
straight-through rounding, in fp32 arithmetic.
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


def _params(model):
    """The step's parameters in the C ABI's order: kernels, fc1 weight / bias, fc2 weight / bias."""
    u = model.update
    return (model.perceive.weight, u.fc1.weight, u.fc1.bias, u.fc2.weight, u.fc2.bias)


def _needs_grad(model, *tensors) -> bool:
    if not torch.is_grad_enabled():
        return False
    if any(t is not None and t.requires_grad for t in tensors):
        return True
    return any(p.requires_grad for p in _params(model))


def _check_shapes(model, x, given4, clamp, fire, noise):
    cfg = model.cfg
    B, C, H, W = x.shape
    if C != cfg.channels:
        raise ValueError(f"state has {C} channels, the model {cfg.channels}")
    if given4.shape != (B, 1, H, W) or fire.shape[0] != B or fire.numel() != B * H * W:
        raise ValueError("given4 / fire must be (B, 1, H, W)")
    if clamp.shape != (B, cfg.c_in, H, W):
        raise ValueError(f"clamp must be {(B, cfg.c_in, H, W)}, got {tuple(clamp.shape)}")
    if noise is not None and noise.shape != x.shape:
        raise ValueError("noise must have the state's shape")


def _forward(model, prec, dev, x, given4, clamp, fire, noise):
    """x_out = step(x) through `nca_step`; returns (x_out, the fp32 / u8 operands it read)."""
    B, _, H, W = x.shape
    pk = model.packed(prec, dev)
    xs = x.detach().to(torch.float32).contiguous()
    g8 = given4.detach().to(torch.uint8).contiguous()
    cl = clamp.detach().to(torch.float32).contiguous()
    fi = fire.detach().to(torch.float32).contiguous()
    nz = None if noise is None else noise.detach().to(torch.float32).contiguous()
    out = torch.empty_like(xs)
    _lib.check(
        _lib.load().nca_step(ctypes.byref(pk.desc), pk.buf.data_ptr(), B, H, W, xs.data_ptr(),
                             g8.data_ptr(), cl.data_ptr(), fi.data_ptr(), _lib.ptr(nz),
                             out.data_ptr(), _lib.stream_of(dev)),
        "nca_step",
    )
    return out, xs, g8, fi


def step_vjp(model, x, given4, fire, grad_out, precision: str = "fp32", want_grad_x: bool = True):
    """The vector-Jacobian product of one step through `nca_step_backward`: (grad_x or None,
    [grad of kernels, fc1.weight, fc1.bias, fc2.weight, fc2.bias]) for the cotangent `grad_out`
    of the step's output. `fire` (B, 1, H, W) is the step's fire value per cell."""
    dev = _lib.require_device(x, given4, fire, grad_out)
    B, C, H, W = x.shape
    L = _lib.load()
    pk = model.packed(precision, dev)
    xs = x.detach().to(torch.float32).contiguous()
    g8 = given4.detach().to(torch.uint8).contiguous()
    fi = fire.detach().to(torch.float32).contiguous()
    go = grad_out.detach().to(torch.float32).contiguous()
    params = _params(model)
    master = [p.detach().to(dev, torch.float32).contiguous() for p in params]
    wts = _lib.CellWeights(*[m.data_ptr() for m in master], None, None, None)
    grads = [torch.empty(p.shape, dtype=torch.float32, device=dev) for p in params]
    gs = _lib.CellGrads(*[g.data_ptr() for g in grads], None, None)
    gx = torch.empty_like(xs) if want_grad_x else None
    ws_bytes = L.nca_step_backward_workspace_bytes(ctypes.byref(pk.desc), B, H, W)
    if ws_bytes == 0:
        _lib.check(_lib.NCA_ERR_UNSUPPORTED, "nca_step_backward_workspace_bytes")
    ws = torch.empty((ws_bytes // 4,), dtype=torch.float32, device=dev)
    _lib.check(
        L.nca_step_backward(ctypes.byref(pk.desc), pk.buf.data_ptr(), ctypes.byref(wts), B, H, W,
                            xs.data_ptr(), g8.data_ptr(), fi.data_ptr(), go.data_ptr(),
                            ctypes.byref(gs), _lib.ptr(gx), ws.data_ptr(), ws_bytes,
                            _lib.stream_of(dev)),
        "nca_step_backward",
    )
    return gx, grads


class _HipStep(torch.autograd.Function):
    """One step as an autograd node: forward `nca_step`, backward `nca_step_backward` (the fused
    cell update's backward, reference src/nca/engine/ops.py:269-294, then the MLP's and the
    perception's). The clamp values get g on the input slice of given cells, the noise gets the
    gradient of the residual sum u (g with that slice zeroed), like the reference's where()."""

    @staticmethod
    def forward(ctx, model, prec, x, given4, clamp, fire, noise, *params):
        dev = x.device
        out, xs, g8, fi = _forward(model, prec, dev, x, given4, clamp, fire, noise)
        ctx.model, ctx.prec = model, prec
        ctx.dtypes = (x.dtype, clamp.dtype, None if noise is None else noise.dtype)
        ctx.save_for_backward(xs, g8, fi)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        xs, g8, fi = ctx.saved_tensors
        model, prec = ctx.model, ctx.prec
        need = ctx.needs_input_grad
        gx, gp = step_vjp(model, xs, g8, fi, grad_out, prec, want_grad_x=need[2])
        sl = model.cfg.in_slice
        given = g8.bool()
        g_clamp = g_noise = None
        if need[4]:
            g_clamp = torch.where(given, grad_out[:, sl], 0.0).to(ctx.dtypes[1])
        if need[6]:
            g_noise = grad_out.clone()
            g_noise[:, sl] = torch.where(given, 0.0, grad_out[:, sl])
            g_noise = g_noise.to(ctx.dtypes[2])
        gx = None if gx is None else gx.to(ctx.dtypes[0])
        gp = [g if n else None for g, n in zip(gp, need[7:])]
        return (None, None, gx, None, g_clamp, None, g_noise, *gp)


def hip_step(model, x, given4, clamp, fire, noise=None, precision=None):
    """One fused step on the GPU (C ABI `nca_step`); differentiable w.r.t. the state, the clamp
    values, the noise and the cell's parameters when autograd needs it (`nca_step_backward`)."""
    dev = _lib.require_device(x, given4, clamp, fire, noise)
    prec = _autocast_precision(dev, precision)
    _check_shapes(model, x, given4, clamp, fire, noise)
    if not _needs_grad(model, x, clamp, noise):
        return _forward(model, prec, dev, x, given4, clamp, fire, noise)[0]
    if fire.requires_grad:
        raise ValueError("the HIP step does not differentiate w.r.t. the fire mask")
    return _HipStep.apply(model, prec, x, given4, clamp, fire, noise, *_params(model))


def make_step(model, opts: StepOptions | None = None, precision: str | None = None):
    """Step function with the reference engine's signature (reference step.py:184-207).
    `noise_mask` is accepted and unused (it only matters with group normalisation, which the
    HIP cell does not have); `clock` must be None (no time embedding). Under autograd the
    step records a node whose backward runs on the GPU (`step_vjp`)."""
    model.kernel_support()

    def step(x, given4, clamp, fire, noise=None, noise_mask=None, clock=None):
        if clock is not None and model.cfg.time_steps:
            raise ValueError("time embeddings are not implemented")
        return hip_step(model, x, given4, clamp, fire, noise, precision)

    return step
