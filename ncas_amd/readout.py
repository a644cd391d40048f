"""Readout and selection on the GPU.

* `readout(model, x)` - per-cell confidence, board confidence and argmax class of fp32 states
  (reference src/nca/model.py:596-633): mlp head -> max softmax, l2 head -> max
  1 / (1 + |x - e_v|), board confidence = mean over all H*W cells, argmax = first maximum.
  The kernel uses a fixed operation order (fma chains, a Cephes-method exp, a sequential
  cell sum) so that its results are reproducible bit for bit.
* `conf_select(conf, alive, k)` - conf@K's per-board choice (reference src/nca/rollout.py:
  317-334): the first maximum of the alive trials' confidence among the first k trials, one
  wavefront per board.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib


def readout(model, x: torch.Tensor):
    dev = _lib.require_device(x)
    B, C, H, W = x.shape
    if C != model.cfg.channels:
        raise ValueError(f"state has {C} channels, the model {model.cfg.channels}")
    pk = model.packed("fp32", dev)
    xs = x.detach().to(torch.float32).contiguous()
    cc = torch.empty((B, H, W), dtype=torch.float32, device=dev)
    cb = torch.empty((B,), dtype=torch.float32, device=dev)
    am = torch.empty((B, H, W), dtype=torch.int32, device=dev)
    L = _lib.load()
    _lib.check(
        L.nca_readout(ctypes.byref(pk.desc), pk.buf.data_ptr(), B, H, W, xs.data_ptr(),
                      cc.data_ptr(), cb.data_ptr(), am.data_ptr(), _lib.stream_of(dev)),
        "nca_readout",
    )
    return cc, cb, am


def conf_select(conf: torch.Tensor, alive: torch.Tensor | None = None, k: int | None = None):
    """(N,) int64 index of the selected trial of each board."""
    dev = _lib.require_device(conf, alive)
    N, K = conf.shape
    k = K if k is None else min(int(k), K)
    c = conf.detach().to(torch.float32).contiguous()
    a = None if alive is None else alive.detach().to(torch.uint8).contiguous()
    best = torch.empty((N,), dtype=torch.int32, device=dev)
    _lib.check(
        _lib.load().nca_conf_select(c.data_ptr(), _lib.ptr(a), N, K, k, best.data_ptr(),
                                    _lib.stream_of(dev)),
        "nca_conf_select",
    )
    return best.long()
