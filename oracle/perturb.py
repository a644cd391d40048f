"""Damage discs rasterised in numpy (oracle: test infrastructure only).

The discs of the reference's `circular_masks` (reference src/nca/perturb.py:43-83) given as
(row, cy, cx, r^2) rows: "ours" marks the cells (i, j) with (i - cy)^2 + (j - cx)^2 <= r^2,
"official" the cells whose numpy linspace(-1, 1) coordinates (y_i, x_j) have
(y_i - cy)^2 + (x_j - cx)^2 < r^2. The union over a board's discs is its damage mask.
"""

from __future__ import annotations

import numpy as np


def disc_masks(discs: np.ndarray, B: int, H: int, W: int, geometry: str = "ours") -> np.ndarray:
    masks = np.zeros((B, H, W), dtype=bool)
    if geometry == "official":
        ys = np.linspace(-1.0, 1.0, H)[:, None]
        xs = np.linspace(-1.0, 1.0, W)[None, :]
    else:
        ys = np.arange(H, dtype=np.float64)[:, None]
        xs = np.arange(W, dtype=np.float64)[None, :]
    for row, cy, cx, r2 in np.asarray(discs, dtype=np.float64).reshape(-1, 4):
        d = (ys - cy) ** 2 + (xs - cx) ** 2
        masks[int(row)] |= (d < r2) if geometry == "official" else (d <= r2)
    return masks


def damage_clamp(x: np.ndarray, masks: np.ndarray, fill: float, given: np.ndarray,
                 clamp: np.ndarray, in_slice: slice) -> np.ndarray:
    """x (B, C, H, W): every channel of a damaged cell set to fill, then the given cells' input
    channels set to the clamp values (reference model.py:430-438)."""
    y = np.where(masks[:, None], np.float32(fill), x).astype(np.float32)
    y[:, in_slice] = np.where(given[:, None], clamp, y[:, in_slice])
    return y
