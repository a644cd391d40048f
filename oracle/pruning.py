"""Niche-capped diversity pruning restated in numpy (oracle: test infrastructure only).

Follows the reference's `niche_capped_pruning` (reference src/nca/pruning.py:22-65) step by step:
per board with a > 1 alive trials, target = a // 2; alive trials grouped into niches by
identical decoded boards (a dict in first-member order); each niche's members sorted by
confidence, highest first (Python's stable sort: ties keep the lower trial first) and cut to
n_cap; then round-robin over the niches in a random order, depth by depth, until target
survivors are chosen or a round adds nothing. The one substitution: the niche order is not
numpy's `rng.permutation` but the niches sorted by a Philox4x32-10 word keyed on
(seed; first member, event, board, 1), ties by first member - the rule the GPU kernel
(`nca_prune_select`) uses, so that both draw the same order.
"""

from __future__ import annotations

import numpy as np

from .philox import philox4x32_10


def niche_key(seed: int, event: int, board: int, rep: int) -> int:
    seed = int(seed) & 0xFFFFFFFFFFFFFFFF
    w = philox4x32_10((rep, event, board, 1), (seed & 0xFFFFFFFF, seed >> 32))
    return int(w[0])


def niche_capped_pruning(decoded, conf, alive, n_cap: int, seed: int, event: int,
                         order_fn=None) -> np.ndarray:
    """decoded (N, K, ...) ints, conf (N, K), alive (N, K) bool -> new alive (N, K) bool.
    `order_fn(board, representatives) -> niche order` replaces the Philox order (tests)."""
    dec = np.asarray(decoded)
    N, K = dec.shape[:2]
    cf = np.asarray(conf, dtype=np.float32)
    al = np.asarray(alive, dtype=bool).copy()
    for n in range(N):
        idx = np.nonzero(al[n])[0]
        if len(idx) <= 1:
            continue
        target = len(idx) // 2
        niches: dict[bytes, list[int]] = {}
        for k in idx:
            niches.setdefault(dec[n, k].tobytes(), []).append(int(k))
        capped = [sorted(members, key=lambda k: -cf[n, k])[:n_cap] for members in niches.values()]
        reps = [members[0] for members in niches.values()]
        if order_fn is None:
            keys = [niche_key(seed, event, n, r) for r in reps]
            order = sorted(range(len(capped)), key=lambda j: (keys[j], reps[j]))
        else:
            order = order_fn(n, reps)
        survivors: list[int] = []
        depth = 0
        while len(survivors) < target:
            added = False
            for j in order:
                if depth < len(capped[j]):
                    survivors.append(capped[j][depth])
                    added = True
                    if len(survivors) >= target:
                        break
            if not added:
                break
            depth += 1
        new = np.zeros(K, dtype=bool)
        new[survivors] = True
        al[n] = new
    return al


def pruned_compute_fraction(m: int) -> float:
    """Share of the unpruned K x D compute with m - 1 halvings (reference pruning.py:68-70):
    (2 - 2^-(m-1)) / m."""
    return (2 - 2.0 ** (-(m - 1))) / m
