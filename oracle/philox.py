"""Philox4x32-10 and the fire-mask rule in numpy (oracle; see `nca_oracle.c` for the spec).

Salmon, Moraes, Dror, Shaw, "Parallel Random Numbers: As Easy as 1, 2, 3" (SC'11): ten rounds
of two 32x32->64 multiplications, with the key bumped by the Weyl constants between rounds.
The fire mask replaces the reference's `torch.rand(B, 1, H, W) < p` (reference
src/nca/engine/rng.py:66-69, src/nca/model.py:584-593) by a draw keyed on
(seed; cell >> 2, step, row, 0): word `cell & 3`, top 24 bits, scaled by 2^-24.
"""

from __future__ import annotations

import numpy as np

M0, M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
W0, W1 = np.uint64(0x9E3779B9), np.uint64(0xBB67AE85)
MASK = np.uint64(0xFFFFFFFF)
S32 = np.uint64(32)


def philox4x32_10(ctr, key):
    """Vectorised Philox4x32-10. ctr: 4 arrays (or ints) of uint32 values, key: 2 of them.
    Returns a (4, ...) uint32 array."""
    c0, c1, c2, c3 = (np.asarray(c, dtype=np.uint64) & MASK for c in ctr)
    k0, k1 = (np.asarray(k, dtype=np.uint64) & MASK for k in key)
    for _ in range(10):
        p0 = M0 * c0
        p1 = M1 * c2
        hi0, lo0 = p0 >> S32, p0 & MASK
        hi1, lo1 = p1 >> S32, p1 & MASK
        c0, c1, c2, c3 = hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0
        k0 = (k0 + W0) & MASK
        k1 = (k1 + W1) & MASK
    return np.stack(np.broadcast_arrays(c0, c1, c2, c3)).astype(np.uint32)


def cell_uniforms(seed: int, row0: int, rows: int, step: int, hw: int) -> np.ndarray:
    """u of every cell of rows [row0, row0 + rows) at `step`: (rows, hw) float32."""
    seed = int(seed) & 0xFFFFFFFFFFFFFFFF
    r = np.arange(row0, row0 + rows, dtype=np.uint64)[:, None]
    q = np.arange(hw, dtype=np.uint64)[None, :]
    words = philox4x32_10(
        (q >> np.uint64(2), np.uint64(step & 0xFFFFFFFF), r, np.uint64(0)),
        (np.uint64(seed & 0xFFFFFFFF), np.uint64(seed >> 32)),
    )  # (4, rows, hw)
    w = np.take_along_axis(words, (q & np.uint64(3)).astype(np.int64)[None].repeat(rows, 1), 0)[0]
    return (w >> np.uint32(8)).astype(np.float32) * np.float32(2.0**-24)


def fire_mask(
    seed: int,
    row0: int,
    rows: int,
    step: int,
    hw: int,
    p: float,
    p_low: float | None = None,
    tau: float | None = None,
    conf: np.ndarray | None = None,
    given: np.ndarray | None = None,
) -> np.ndarray:
    """(rows, hw) uint8 fire mask. With p_low/tau/conf: adaptive firing (model.py:589-593)."""
    u = cell_uniforms(seed, row0, rows, step, hw)
    prob = np.full(u.shape, np.float32(p), dtype=np.float32)
    if p_low is not None and tau is not None and conf is not None:
        confident = np.asarray(conf, dtype=np.float32).reshape(rows, hw) > np.float32(tau)
        if given is not None:
            confident |= np.asarray(given, dtype=bool).reshape(rows, hw)
        prob = np.where(confident, np.float32(p_low), prob)
    return (u < prob).astype(np.uint8)
