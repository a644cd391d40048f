"""The temporally blocked kernel (rollout_window16: bf16 cells with C = 16 on LDS-resident windows,
T steps per launch), on the GPU through the C ABI.

* Its results equal the per-step path's (one launch of the wave-per-tile kernel per step,
  nca_set_kernel_path(2)) bit for bit: states, fired counts and board confidences, on the 201x201
  maze boards and on ragged grids (windows ending mid-row, grids narrower than a tile, grids of
  one cell's width) x wall / zero / wrap padding x T = 2, 3, 4, 8 steps per launch, for step
  counts that leave a partial last launch, with Philox masks, per-step keys and injected masks,
  caller states that do not hold the clamp values yet, and in place (x_in == x_out).
* The 201x201 C=16 maze cell against the oracle: each of 16 steps within the bf16 bar of the
  oracle's step from the GPU's previous state, fired counts exact.
"""

from __future__ import annotations

import copy
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
DEV = torch.device("cuda:0")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    clib.build()
    yield
    L = _lib.load()
    L.nca_set_kernel_path(0)
    L.nca_set_window_steps(0)


def _say(*a):
    print(*a, flush=True)


def _random_case(H, W, B=3, padding="wall", seed=0):
    m = perturbed_model("maze_c16", seed, *DYN["maze_c16"], padding=padding)
    g = torch.Generator().manual_seed(H * 1000 + W + seed)
    x = torch.randn((B, 16, H, W), generator=g) * 0.3  # not clamped: the first step clamps
    g4 = torch.rand((B, 1, H, W), generator=g) < 0.3
    cl = torch.randn((B, m.cfg.c_in, H, W), generator=g)
    return m, copy.deepcopy(m).to(DEV), x.to(DEV), g4.to(DEV), cl.to(DEV)


def _run(md, x, g4, cl, n, path, T=0, out=None, **kw):
    L = _lib.load()
    assert L.nca_set_kernel_path(path) == 0
    assert L.nca_set_window_steps(T) == 0
    try:
        with torch.no_grad():
            return rollout_steps(md, x, g4, cl, n, precision="bf16", want_fired=True, out=out, **kw)
    finally:
        L.nca_set_kernel_path(0)
        L.nca_set_window_steps(0)


def _equal(a, b, what):
    for u, v, name in zip(a, b, ("state", "conf", "fired")):
        assert torch.equal(u, v), (what, name, (u.float() - v.float()).abs().max().item())


@pytest.mark.parametrize("padding", ["wall", "zero", "wrap"])
@pytest.mark.parametrize("H,W", [(201, 201), (37, 45), (5, 70), (33, 1), (3, 2), (13, 13), (31, 17)])
def test_window_kernel_equals_the_per_step_path(H, W, padding):
    _say("window vs per-step", H, W, padding)
    B = 2 if H * W > 10000 else 3
    m, md, x, g4, cl = _random_case(H, W, B=B, padding=padding)
    for T, n in ((2, 7), (3, 5), (4, 9), (8, 8)):
        kw = dict(seed=11, row0=5, step0=3, p_fire=0.6)
        ref = _run(md, x, g4, cl, n, path=2, **kw)
        got = _run(md, x, g4, cl, n, path=4, T=T, **kw)
        _equal(got, ref, (T, n))


def test_window_kernel_per_step_keys_and_injected_masks():
    m, md, x, g4, cl = _random_case(37, 45, B=3)
    B, C, H, W = x.shape
    seeds = np.arange(70, 76, dtype=np.int64)
    ref = _run(md, x, g4, cl, 6, path=2, step_seeds=seeds, p_fire=0.5)
    got = _run(md, x, g4, cl, 6, path=4, T=3, step_seeds=seeds, p_fire=0.5)
    _equal(got, ref, "step keys")
    masks = (torch.rand((6, B, 1, H, W), generator=torch.Generator().manual_seed(2)) < 0.4).float().to(DEV)
    ref = _run(md, x, g4, cl, 6, path=2, masks=masks)
    got = _run(md, x, g4, cl, 6, path=4, T=4, masks=masks)
    _equal(got, ref, "injected masks")


def test_window_kernel_in_place_and_automatic_choice():
    """x_in == x_out; and the automatic path on 201x201 with two steps per launch set (the
    temporally blocked kernel) equals the per-step path."""
    m, md, x, g4, cl = _random_case(201, 201, B=2)
    ref = _run(md, x, g4, cl, 5, path=2, seed=3, p_fire=0.5)
    y = x.clone()
    got = _run(md, y, g4, cl, 5, path=4, T=2, out=y, seed=3, p_fire=0.5)
    _equal(got, ref, "in place")
    got = _run(md, x, g4, cl, 6, path=0, T=2, seed=3, p_fire=0.5)
    ref = _run(md, x, g4, cl, 6, path=2, seed=3, p_fire=0.5)
    _equal(got, ref, "automatic")


def test_window_kernel_maze201_against_the_oracle():
    """The 201x201 C=16 maze cell, 16 steps in 8 launches: every step within the bf16 bar of the
    oracle's step from the GPU's previous state, fired counts exact."""
    m = perturbed_model("maze_c16", 0, *DYN["maze_c16"])
    md = copy.deepcopy(m).to(DEV)
    b = maze_boards(2, 201, 0)
    x, g4, cl = initial_state(m, b, k=1, sigma=0.15)
    B, C, H, W = x.shape
    xd, gd, cd = x.to(DEV), g4.to(DEV), cl.to(DEV)
    states, fired = [], torch.zeros(B, dtype=torch.int64)
    cur = xd
    for t in range(0, 16, 2):  # two steps per call, one launch each
        cur, _, f = _run(md, cur, gd, cd, 2, path=0, T=2, seed=7, row0=1, step0=t, p_fire=0.5)
        fired += f.cpu().long()
        states.append(cur.cpu())
    _, fr = O.rollout(oracle_cell(m), x, g4, cl, 16, "bf16", seed=7, row0=1, p_fire=0.5)
    assert torch.equal(fired, fr)
    # one-step check of every second step from the GPU state two steps earlier
    masks = [O.fire_masks_np(7, 1, B, t, H, W, 0.5) for t in range(16)]
    prev = x
    worst = 0.0
    for i, s in enumerate(states):
        mid = O.step(oracle_cell(m), prev, g4, cl, masks[2 * i], "bf16").float()
        ref = O.step(oracle_cell(m), mid, g4, cl, masks[2 * i + 1], "bf16").float()
        worst = max(worst, (s - ref).abs().max().item())
        prev = s
    _say("worst two-step error", worst)
    assert worst <= 2e-2
