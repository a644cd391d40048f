"""Counter-based fire masks (Philox4x32-10) on the GPU.

The reference gives every step a 62-bit seed and regenerates its fire mask from that seed
alone (reference src/nca/engine/rng.py:37-76). The HIP engine keys a Philox4x32-10 stream on
(seed; cell >> 2, step, row, 0) instead, so a mask depends only on (seed, row, step, cell):
`u = (word >> 8) * 2^-24`, fire where `u < p` (adaptive: `p_low` for cells whose confidence is
`> tau` or, with `given_confident`, given cells; reference model.py:584-593).
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib

SEED_BITS = 62


def step_seeds(rng: np.random.Generator, n: int) -> np.ndarray:
    """`n` independent step seeds (reference rng.py:37-39)."""
    return rng.integers(0, 2**SEED_BITS, size=n, dtype=np.int64)


def fire_desc(seed=0, p_fire=0.5, p_low=None, tau=None, given_confident=True, row0=0, step0=0,
              step_seeds=None, fire_in=None) -> _lib.FireDesc:
    adaptive = p_low is not None and tau is not None
    return _lib.FireDesc(
        int(seed) & 0xFFFFFFFFFFFFFFFF, _lib.ptr(step_seeds), _lib.ptr(fire_in), int(row0),
        int(step0), float(p_fire), float(p_low or 0.0), float(tau or 0.0), int(adaptive),
        int(bool(given_confident)),
    )


def fire_mask(rows: int, H: int, W: int, seed: int, step: int, p_fire: float, row0: int = 0,
              p_low=None, tau=None, conf_cell=None, given=None, given_confident=True,
              device=None) -> torch.Tensor:
    """(rows, 1, H, W) float32 fire mask of one step, drawn on the GPU."""
    dev = _lib.require_device(*(t for t in (conf_cell, given) if t is not None)) \
        if conf_cell is not None else torch.device(device or "cuda")
    if dev.type != "cuda":
        raise ValueError("fire masks are drawn on the GPU")
    fd = fire_desc(seed, p_fire, p_low, tau, given_confident, row0)
    if fd.adaptive and conf_cell is None:
        raise ValueError("adaptive firing needs conf_cell")
    cc = None if conf_cell is None else conf_cell.detach().to(torch.float32).contiguous()
    g8 = None if given is None else given.detach().to(torch.uint8).contiguous()
    out = torch.empty((rows, H, W), dtype=torch.uint8, device=dev)
    _lib.check(
        _lib.load().nca_fire_mask(rows, H, W, ctypes.byref(fd), int(step), _lib.ptr(cc),
                                  _lib.ptr(g8), out.data_ptr(), _lib.stream_of(dev)),
        "nca_fire_mask",
    )
    return out.view(rows, 1, H, W).to(torch.float32)
