"""Niche-capped diversity pruning on the GPU (reference src/nca/pruning.py:22-70).

`prune_select(decoded, conf, alive, n_cap, seed, event)` is the selection of the trials that
survive a halving of a board's ensemble (C ABI `nca_prune_select`): trials with identical decoded
boards form a niche, each niche keeps at most n_cap of its most confident members, and the
survivors (half the alive trials) are taken round-robin across the niches in a random order
keyed on (seed; niche, event, board). `prune_select_rows` takes the running rows of a compacted
batch directly; `rollout()` calls it at its pruning steps and drops the pruned rows, so the
kernels of the later steps run on fewer rows.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib


def prune_select(decoded: torch.Tensor, conf: torch.Tensor, alive: torch.Tensor, n_cap: int,
                 seed: int, event: int) -> torch.Tensor:
    """decoded (N, K, ...) integer boards, conf (N, K), alive (N, K) bool on the GPU -> the new
    alive mask (N, K) bool."""
    dev = _lib.require_device(decoded, conf, alive)
    N, K = conf.shape
    d = decoded.detach().reshape(N, K, -1).to(torch.int32).contiguous()
    c = conf.detach().to(torch.float32).contiguous()
    a = alive.detach().to(torch.uint8).contiguous()
    out = torch.empty((N, K), dtype=torch.uint8, device=dev)
    _lib.check(_lib.load().nca_prune_select(d.data_ptr(), c.data_ptr(), a.data_ptr(), N, K,
                                            d.shape[2], int(n_cap),
                                            int(seed) & 0xFFFFFFFFFFFFFFFF, int(event),
                                            out.data_ptr(), _lib.stream_of(dev)),
               "nca_prune_select")
    return out.bool()


def prune_select_rows(decoded: torch.Tensor, conf: torch.Tensor, row_trial: torch.Tensor,
                      n_boards: int, k: int, n_cap: int, seed: int, event: int) -> torch.Tensor:
    """The same selection on a compacted batch: decoded (rows, ...) and conf (rows,) of the
    alive trials, row_trial (rows,) their flat (board, trial) index board * k + trial, strictly
    increasing -> (rows,) bool, True where the row's trial survives (C ABI
    `nca_prune_select_rows`). Equals `prune_select` on the full layout with the absent trials
    dead."""
    dev = _lib.require_device(decoded, conf, row_trial)
    rows = conf.shape[0]
    d = decoded.detach().reshape(rows, -1).to(torch.int32).contiguous()
    c = conf.detach().to(torch.float32).contiguous()
    r = row_trial.detach().to(torch.int64).contiguous()
    out = torch.empty((rows,), dtype=torch.uint8, device=dev)
    _lib.check(_lib.load().nca_prune_select_rows(
        d.data_ptr(), c.data_ptr(), r.data_ptr(), rows, int(n_boards), int(k),
        d.shape[1] if rows else 1, int(n_cap), int(seed) & 0xFFFFFFFFFFFFFFFF, int(event),
        out.data_ptr(), _lib.stream_of(dev)), "nca_prune_select_rows")
    return out.bool()


def pruned_compute_fraction(m: int) -> float:
    """Share of the unpruned K x D compute that m - 1 equidistant halvings leave
    (reference pruning.py:68-70): (2 - 2^-(m-1)) / m."""
    return (2 - 2.0 ** (-(m - 1))) / m
