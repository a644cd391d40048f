"""The fused parameter update of the training step: clip + AdamW + EMA + zero_grad in one launch
(`nca_adamw_ema`), replacing clip_grad_norm_, the host test of the norm, torch.optim.AdamW,
the EMA loop and zero_grad of the reference's update (reference src/nca/engine/train.py:262-273).

`FusedUpdate(model, ema_model, lr, betas, eps, weight_decay)` moves every parameter of both
models into flat fp32 buffers (the parameters become views of them, in `model.parameters()`
order) with a flat gradient buffer behind the parameters' `.grad`, so that gradients added into
`.grad` in place land where the kernel reads them. `step(lr, ema_decay, max_norm)` queues the
update on the current stream and returns the device scalar holding the gradient norm before
clipping; whether the norm was finite, the count of applied AdamW steps and the count of skipped
iterations stay on the device, so the iteration needs no host synchronisation. The update is
deterministic (a fixed summation order for the norm), so a run resumed from `state_dict()`
repeats the uninterrupted run bit for bit. `state_dict()` has torch.optim.AdamW's layout
(per-parameter `step`, `exp_avg`, `exp_avg_sq`; one parameter group) plus the skipped count.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib


def _flatten(params, device) -> torch.Tensor:
    """Copy `params` into one flat fp32 buffer and make each parameter a view of its slice."""
    n = sum(p.numel() for p in params)
    flat = torch.empty(n, dtype=torch.float32, device=device)
    off = 0
    for p in params:
        k = p.numel()
        flat[off:off + k].copy_(p.detach().reshape(-1))
        p.data = flat[off:off + k].view(p.shape)
        off += k
    return flat


class FusedUpdate:
    def __init__(self, model, ema_model, lr: float, betas=(0.9, 0.999), eps: float = 1e-8,
                 weight_decay: float = 0.0):
        self.params = list(model.parameters())
        self.ema_params = list(ema_model.parameters()) if ema_model is not None else []
        if self.ema_params and [p.shape for p in self.ema_params] != [p.shape for p in self.params]:
            raise ValueError("the EMA model must have the model's parameter shapes")
        dev = self.params[0].device
        _lib.require_device(*self.params)
        if any(p.dtype != torch.float32 for p in self.params):
            raise ValueError("the fused update keeps fp32 master weights")
        self.lr, self.betas, self.eps, self.weight_decay = float(lr), tuple(betas), eps, weight_decay
        self.flat = _flatten(self.params, dev)
        self.ema = _flatten(self.ema_params, dev) if self.ema_params else None
        self.n = self.flat.numel()
        self.grad = torch.zeros_like(self.flat)
        self.exp_avg = torch.zeros_like(self.flat)
        self.exp_avg_sq = torch.zeros_like(self.flat)
        self.counters = torch.zeros(2, dtype=torch.int64, device=dev)  # applied, skipped
        self.grad_norm = torch.zeros((), dtype=torch.float32, device=dev)
        self._ws = torch.empty(_lib.ADAMW_WORKSPACE_BYTES, dtype=torch.uint8, device=dev)
        off = 0
        self._slices = []
        for p in self.params:
            k = p.numel()
            p.grad = self.grad[off:off + k].view(p.shape)
            self._slices.append(slice(off, off + k))
            off += k

    def step(self, lr: float | None = None, ema_decay: float | None = None,
             max_norm: float | None = None) -> torch.Tensor:
        """One update with this iteration's learning rate and EMA decay (None: no EMA); clips
        the gradient to max_norm first (None: no clipping)."""
        if ema_decay is not None and self.ema is None:
            raise ValueError("no EMA model")
        d = _lib.AdamWDesc(
            self.lr if lr is None else float(lr), float(self.betas[0]), float(self.betas[1]),
            float(self.eps), float(self.weight_decay),
            -1.0 if ema_decay is None else float(ema_decay),
            -1.0 if max_norm is None else float(max_norm))
        dev = self.flat.device
        _lib.check(_lib.load().nca_adamw_ema(
            self.flat.data_ptr(), self.grad.data_ptr(), self.exp_avg.data_ptr(),
            self.exp_avg_sq.data_ptr(), _lib.ptr(self.ema), self.n, ctypes.byref(d),
            self.counters.data_ptr(), self.grad_norm.data_ptr(), self._ws.data_ptr(),
            _lib.stream_of(dev)),
            "nca_adamw_ema")
        # the kernel wrote the parameters behind torch's back: bump their version counters, so
        # caches keyed on them (the models' packed weights) see the change
        torch.autograd.graph.increment_version(self.params + self.ema_params)
        return self.grad_norm

    def state_dict(self) -> dict:
        steps, skipped = (int(v) for v in self.counters.tolist())
        group = dict(lr=self.lr, betas=self.betas, eps=self.eps, weight_decay=self.weight_decay,
                     amsgrad=False, maximize=False, foreach=None, capturable=False,
                     differentiable=False, fused=None, params=list(range(len(self.params))))
        state = {i: {"step": torch.tensor(float(steps)),
                     "exp_avg": self.exp_avg[s].view(p.shape).clone(),
                     "exp_avg_sq": self.exp_avg_sq[s].view(p.shape).clone()}
                 for i, (s, p) in enumerate(zip(self._slices, self.params)) if steps}
        return {"state": state, "param_groups": [group], "skipped": skipped}

    def load_state_dict(self, sd: dict) -> None:
        state = sd.get("state", {})
        steps = 0
        self.exp_avg.zero_()
        self.exp_avg_sq.zero_()
        for i, s in enumerate(self._slices):
            st = state.get(i)
            if st is None:
                continue
            steps = int(float(st["step"]))
            self.exp_avg[s].copy_(st["exp_avg"].reshape(-1))
            self.exp_avg_sq[s].copy_(st["exp_avg_sq"].reshape(-1))
        self.counters.copy_(torch.tensor([steps, int(sd.get("skipped", 0))], dtype=torch.int64))
        g = sd["param_groups"][0]
        self.lr, self.betas = float(g["lr"]), tuple(g["betas"])
        self.eps, self.weight_decay = float(g["eps"]), float(g["weight_decay"])

    @property
    def skipped(self) -> torch.Tensor:
        """Device scalar: iterations whose gradient norm was not finite."""
        return self.counters[1]
