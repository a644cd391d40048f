"""The training batch's perturbations before a rollout (reference src/nca/perturb.py, applied by
src/nca/train.py:219-252): target swaps, damage discs, the clamp and the optional batch noise.

* `swap_rows(rng, B, p)` - the batch rows whose board is swapped (a uniform draw per row).
* `draw_discs(rng, hit, H, W, n, r_min, r_max, geometry)` - the damage discs of the boards in
  `hit` as an (n_discs, 4) array of (row, centre y, centre x, radius^2). The draws come from the
  run's numpy generator in the reference's order (per damaged board, per disc: the centre, then
  the radius), so a run's damage follows the same random stream; "ours" centres anywhere on the
  grid with radius r ~ U(r_min, r_max) min(H, W), "official" centres in [-0.5, 0.5]^2 on
  linspace(-1, 1) coordinates with r ~ U(r_min, r_max).
* `damage_clamp(model, x, given4, clamp, discs, fill, geometry)` - one pass over the state on the
  GPU (`nca_damage_clamp`): the cells inside a disc take `fill` in every channel, then the given
  cells' input channels take their clamp values. In place.
* `batch_noise(model, batch, bn, generator)` - the public code's optional batch noise: per board
  with probability p, N(0, sigma^2) on a ps fraction of the cells, every channel except the given
  cells' input channels, then the clamp.
"""

from __future__ import annotations

import numpy as np
import torch

from . import _lib


def swap_rows(rng: np.random.Generator, B: int, p: float) -> np.ndarray:
    return np.flatnonzero(rng.random(B) < p)


def draw_discs(rng: np.random.Generator, hit: np.ndarray, H: int, W: int, n: int,
               r_min: float, r_max: float, geometry: str = "ours") -> np.ndarray:
    """(n_discs, 4) float64 rows (board row, cy, cx, r^2) for every board of `hit`."""
    if geometry not in _lib.DAMAGE_GEOMETRY:
        raise ValueError(f"unknown damage geometry {geometry!r} (ours | official)")
    out = []
    scale = min(H, W)
    for row in np.flatnonzero(hit):
        for _ in range(n):
            if geometry == "official":
                cy, cx = rng.uniform(-0.5, 0.5, size=2)
                r = rng.uniform(r_min, r_max)
            else:
                cy = rng.uniform(0, H)
                cx = rng.uniform(0, W)
                r = rng.uniform(r_min, r_max) * scale
            out.append((float(row), float(cy), float(cx), float(r) * float(r)))
    return np.asarray(out, dtype=np.float64).reshape(-1, 4)


def damage_clamp(model, x: torch.Tensor, given4: torch.Tensor, clamp: torch.Tensor,
                 discs: np.ndarray, fill: float = 0.0, geometry: str = "ours") -> torch.Tensor:
    """Damage inside `discs` and the clamp, in place on the contiguous fp32 state x
    (B, C, H, W); returns x."""
    dev = _lib.require_device(x, given4, clamp)
    if x.dtype != torch.float32 or not x.is_contiguous():
        raise ValueError("x must be a contiguous float32 tensor")
    B, C, H, W = x.shape
    cfg = model.cfg
    sl = cfg.in_slice
    g8 = given4.reshape(B, H, W).to(torch.uint8).contiguous()
    cl = clamp.to(torch.float32).contiguous()
    if cl.shape != (B, sl.stop - sl.start, H, W):
        raise ValueError("clamp must be (B, c_in, H, W)")
    d = None
    if len(discs):
        d = _lib.upload(np.ascontiguousarray(discs, dtype=np.float64), dev)
    _lib.check(_lib.load().nca_damage_clamp(
        x.data_ptr(), B, C, H, W, _lib.ptr(d), len(discs), _lib.DAMAGE_GEOMETRY[geometry],
        float(fill), g8.data_ptr(), cl.data_ptr(), sl.stop - sl.start, sl.start,
        _lib.stream_of(dev)), "nca_damage_clamp")
    return x


def batch_noise(model, batch: dict, bn: dict, generator: torch.Generator) -> None:
    """The public code's batch noise (reference perturb.py:109-130), then the clamp."""
    x = batch["x"]
    B, C, H, W = x.shape
    dev = x.device
    boards = torch.rand((B, 1, 1, 1), generator=generator, device=dev) < bn["p"]
    cells = torch.rand((B, 1, H, W), generator=generator, device=dev) < bn["ps"]
    noise = torch.randn(x.shape, generator=generator, device=dev) * bn["sigma"]
    in_ch = torch.zeros((1, C, 1, 1), dtype=torch.bool, device=dev)
    in_ch[:, model.cfg.in_slice] = True
    keep = boards & cells & ~(batch["given4"] & in_ch)
    batch["x"] = model.apply_clamp(x + noise * keep.to(x.dtype), batch["given4"], batch["clamp"])
