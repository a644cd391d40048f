"""Parity of the streamed C=32 kernel (bf16 cells with 32 channels and 256 hidden units on boards
up to 31 wide, one board per workgroup: the 30x30 hard-maze rollout), on the GPU through the C ABI.

* States within max-abs 2e-2 of the CPU oracle (bf16) over multi-step rollouts with the same
  Philox masks, fired counts exact, the in-kernel board confidence equal to the oracle's readout
  of the final state bit for bit; a fused rollout equals the same steps chained one launch at a
  time, bit for bit.
* Confidence-gated firing over many fused steps: the kernel decides each cell's next-step mask
  from its new state inside the launch; chained single steps (whose masks come from the state at
  the start of each launch) give the same bits, and each step matches the oracle's step from the
  same state.
* Edge cases: zero padding, the widest grid (W = 31), small grids near the size limit, step
  counts whose last tile is partial, a caller state that does not hold the clamp values yet,
  injected masks, and agreement with the halo-tiled path.
"""

from __future__ import annotations

import copy
import ctypes
import sys

import numpy as np
import pytest
import torch

sys.path.insert(0, __file__.rsplit("/", 1)[0])
from cells import DYN, initial_state, oracle_cell, perturbed_model  # noqa: E402

from ncas_amd import _lib  # noqa: E402
from ncas_amd.inference import rollout_steps  # noqa: E402
from ncas_amd.tasks import maze_boards  # noqa: E402
from oracle import clib  # noqa: E402
from oracle import nca_oracle as O  # noqa: E402

pytestmark = pytest.mark.gpu
TOL = 2e-2
DEV = torch.device("cuda:0")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    clib.build()
    yield
    _lib.load().nca_set_kernel_path(0)


def _say(*a):
    print(*a, flush=True)


def _maze(n, size, k=1, seed=0, sigma=0.15, extra=0.10, **overrides):
    m = perturbed_model("maze_hard_c32", seed, *DYN["maze_hard_c32"], **overrides)
    b = maze_boards(n, size, seed, extra_openings=extra)
    x, g4, cl = initial_state(m, b, k=k, sigma=sigma, seed=seed)
    return m, copy.deepcopy(m).to(DEV), x, g4, cl


def _random(H, W, B=3, seed=0, **overrides):
    m = perturbed_model("maze_hard_c32", seed, *DYN["maze_hard_c32"], **overrides)
    g = torch.Generator().manual_seed(H * 100 + W)
    x = torch.randn((B, 32, H, W), generator=g) * 0.3
    g4 = torch.rand((B, 1, H, W), generator=g) < 0.3
    cl = torch.randn((B, m.cfg.c_in, H, W), generator=g)
    return m, copy.deepcopy(m).to(DEV), x, g4, cl


def _takes_stream(md, B, H, W):
    """The streamed C=32 kernel takes the call: no workspace is asked for."""
    pk = md.packed("bf16", DEV)
    return _lib.load().nca_rollout_workspace_bytes(ctypes.byref(pk.desc), B, H, W) == 0


def test_hard_maze_30x30_rollout_matches_oracle():
    _say("stream32 30x30 rollout")
    m, md, x, g4, cl = _maze(3, 30, k=2)
    B, _, H, W = x.shape
    assert _takes_stream(md, B, H, W)
    cell = oracle_cell(m)
    n = 24
    xr, fr = O.rollout(cell, x, g4, cl, n, "bf16", seed=3, row0=5, step0=2, p_fire=0.8)
    xd, gd, cd = x.to(DEV), g4.to(DEV), cl.to(DEV)
    with torch.no_grad():
        y, conf, f = rollout_steps(md, xd, gd, cd, n, seed=3, row0=5, step0=2, p_fire=0.8,
                                   precision="bf16", want_fired=True)
        cur = xd
        for t in range(n):
            cur, _, _ = rollout_steps(md, cur, gd, cd, 1, seed=3, row0=5, step0=2 + t, p_fire=0.8,
                                      precision="bf16", want_conf=False)
    err = (y.cpu() - xr).abs().max().item()
    _say("max-abs", err)
    assert err <= TOL
    assert torch.equal(f.cpu().long(), fr)
    assert torch.equal(y, cur), "fused rollout differs from chained single steps"
    _, rb, _ = O.readout(cell, y.cpu())
    assert np.array_equal(conf.cpu().numpy().view(np.int32), rb.view(np.int32))


@pytest.mark.parametrize("tau_kind", ["configured", "median"])
def test_gated_firing_fused_equals_chained_and_oracle_steps(tau_kind):
    """Gated firing (p_low = 0.25 p): 10 fused steps == 10 chained single-step launches, bit for
    bit (states and fired counts), and every chained step matches the oracle's step."""
    _say("stream32 gated", tau_kind)
    m, md, x, g4, cl = _maze(3, 30, k=2, seed=1)
    cell = oracle_cell(m)
    p = 0.8
    cc0, _, _ = O.readout(cell, x)
    tau = 0.9 if tau_kind == "configured" else float(np.median(cc0))
    xd, gd, cd = x.to(DEV), g4.to(DEV), cl.to(DEV)
    kw = dict(seed=4, p_fire=p, p_low=0.25 * p, tau=tau, precision="bf16")
    with torch.no_grad():
        y, _, f = rollout_steps(md, xd, gd, cd, 10, want_fired=True, **kw)
    cur = x.clone()
    fired = torch.zeros(x.shape[0], dtype=torch.int64)
    for t in range(10):
        with torch.no_grad():
            yt, _, ft = rollout_steps(md, cur.to(DEV), gd, cd, 1, step0=t, want_fired=True, **kw)
        yr, fr = O.rollout(cell, cur, g4, cl, 1, "bf16", seed=4, step0=t, p_fire=p, p_low=0.25 * p,
                           tau=tau)
        assert torch.equal(ft.cpu().long(), fr), t
        assert (yt.cpu() - yr).abs().max().item() <= TOL, t
        fired += ft.cpu().long()
        cur = yt.cpu()
    assert torch.equal(y.cpu(), cur)
    assert torch.equal(f.cpu().long(), fired)


@pytest.mark.parametrize("padding", ["zero", "wall"])
@pytest.mark.parametrize("H,W,n", [(30, 31, 7), (10, 10, 5), (5, 24, 3), (16, 6, 9)])
def test_grids_paddings_and_partial_tiles(H, W, n, padding):
    """Random states and clamps (the caller's state does not hold the clamp values: the first
    step's update takes them from the clamp tensor), step counts whose last tile is partial."""
    _say("stream32 grid", H, W, n, padding)
    kw = {"padding": padding}
    if padding != "wall":
        kw["wall_token"] = None
    m, md, x, g4, cl = _random(H, W, **kw)
    B = x.shape[0]
    assert _takes_stream(md, B, H, W)
    xr, fr = O.rollout(oracle_cell(m), x, g4, cl, n, "bf16", seed=6, p_fire=0.7)
    with torch.no_grad():
        y, _, f = rollout_steps(md, x.to(DEV), g4.to(DEV), cl.to(DEV), n, seed=6, p_fire=0.7,
                                precision="bf16", want_fired=True)
    err = (y.cpu() - xr).abs().max().item()
    _say("max-abs", err)
    assert err <= TOL
    assert torch.equal(f.cpu().long(), fr)


def test_injected_masks_and_zero_steps():
    _say("stream32 masks")
    m, md, x, g4, cl = _maze(2, 30, k=2, seed=2)
    B, _, H, W = x.shape
    g = torch.Generator().manual_seed(3)
    masks = (torch.rand((9, B, 1, H, W), generator=g) < 0.4).float()
    xr, _ = O.rollout(oracle_cell(m), x, g4, cl, 9, "bf16", masks=masks)
    with torch.no_grad():
        y, _, _ = rollout_steps(md, x.to(DEV), g4.to(DEV), cl.to(DEV), 9, masks=masks.to(DEV),
                                precision="bf16")
        y0, _, f0 = rollout_steps(md, x.to(DEV), g4.to(DEV), cl.to(DEV), 0, precision="bf16",
                                  want_fired=True)
    assert (y.cpu() - xr).abs().max().item() <= TOL
    assert torch.equal(y0.cpu(), x) and int(f0.abs().sum()) == 0


def test_streamed_and_tiled_paths_agree():
    """The same 16-step rollout on the streamed kernel and on the halo-tiled path (one launch per
    step): the same masks (fired counts exact) and states within the bf16 tolerance."""
    _say("stream32 vs tiled")
    m, md, x, g4, cl = _maze(2, 30, k=3, seed=3)
    L = _lib.load()
    pk = md.packed("bf16", DEV)
    B, C, H, W = x.shape
    xd, gd, cd = x.to(DEV), g4.to(DEV), cl.to(DEV)
    with torch.no_grad():
        ys, _, fs = rollout_steps(md, xd, gd, cd, 16, seed=8, p_fire=0.6, precision="bf16",
                                  want_fired=True)
        assert L.nca_set_kernel_path(2) == 0
        try:
            assert L.nca_rollout_workspace_bytes(ctypes.byref(pk.desc), B, H, W) == 2 * B * C * H * W * 4
            yt, _, ft = rollout_steps(md, xd, gd, cd, 16, seed=8, p_fire=0.6, precision="bf16",
                                      want_fired=True)
        finally:
            L.nca_set_kernel_path(0)
    assert torch.equal(fs, ft)
    assert (ys - yt).abs().max().item() <= TOL
