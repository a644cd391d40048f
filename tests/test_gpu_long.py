"""64-step parity on the kernels that carry the large configurations, and the BPTT chunk at its
training shape, on the GPU through the C ABI.

* The streamed C=32 kernel on 30x30 hard mazes (the hard-maze conf@K rollout), bf16: every one
  of 64 steps within max-abs 2e-2 of the oracle's step from the GPU's previous state, with
  uniform firing and with confidence-gated firing (tau 0.9 as configured, and tau at the median
  confidence). For gated firing the oracle's own gating decision from the GPU's state equals the
  GPU's mask bit for bit at every step. The drift of the whole trajectory from the oracle's is
  held within 1.5x the oracle's own drift when only its fp32 summation order changes
  (cells.BF16_SELF_DRIFT, measured by tests/test_oracle_drift.py): bf16 rounding flips amplify
  along a trajectory the same way for any correct summation order.
* The 201x201 maze cell (C=16) on the per-step path: the wave-per-tile kernel in bf16 (the same
  per-step bar; the trajectory within 1.5x the oracle's own 64-step drift, 0.20) and the
  halo-window kernel in fp32 (every one of 64 trajectory
  states within 1e-4), 2 boards, fired counts exact, fused == chained.
* The BPTT chunk at its training shape: 30x30 hard mazes, C=32, bf16, a 32-step chunk (2
  boards): loss and every parameter gradient within a relative norm error of 2e-2 of the fp64
  straight-through oracle; the gradient of the initial state, which passes 32 bf16-rounded
  Jacobians, within 1.5x the relative difference between the oracle's own fp32 and fp64 sums.
"""

from __future__ import annotations

import copy
import sys

import numpy as np
import pytest
import torch

sys.path.insert(0, __file__.rsplit("/", 1)[0])
from cells import (DYN, drift_guard, initial_state, one_step_errors, oracle_cell,  # noqa: E402
                   perturbed_model)

from ncas_amd import _lib  # noqa: E402
from ncas_amd.inference import rollout_steps  # noqa: E402
from ncas_amd.readout import readout  # noqa: E402
from ncas_amd.rng import fire_mask  # noqa: E402
from ncas_amd.tasks import maze_boards  # noqa: E402
from ncas_amd.train import bptt_chunk  # noqa: E402
from oracle import clib  # noqa: E402
from oracle import nca_oracle as O  # noqa: E402

pytestmark = pytest.mark.gpu
TOL = {"fp32": 1e-4, "bf16": 2e-2}
DEV = torch.device("cuda:0")
NAMES = ("kernels", "w1", "b1", "w2", "b2", "head_w", "head_b")
STEPS = 64


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    clib.build()
    yield
    _lib.load().nca_set_kernel_path(0)


def _say(*a):
    print(*a, flush=True)


def _maze(preset, n, size, k=1, seed=0, sigma=0.15, extra=0.0):
    m = perturbed_model(preset, seed, *DYN[preset])
    b = maze_boards(n, size, seed, extra_openings=extra)
    x, g4, cl = initial_state(m, b, k=k, sigma=sigma, seed=seed)
    return m, copy.deepcopy(m).to(DEV), x, g4, cl, b


def _per_step(md, x, g4, cl, n, precision, **kw):
    """n chained one-step launches: the states after every step (on the GPU) and the fired
    counts."""
    states, fired = [], torch.zeros(x.shape[0], dtype=torch.int64)
    cur = x
    step0 = kw.pop("step0", 0)
    with torch.no_grad():
        for t in range(n):
            cur, _, f = rollout_steps(md, cur, g4, cl, 1, step0=step0 + t, precision=precision,
                                      want_fired=True, want_conf=False, **kw)
            states.append(cur)
            fired += f.cpu().long()
    return states, fired


def test_stream32_30x30_uniform_64_steps():
    _say("stream32 30x30 uniform, 64 per-step states")
    m, md, x, g4, cl, _ = _maze("maze_hard_c32", 3, 30, k=2, extra=0.10)
    cell = oracle_cell(m)
    kw = dict(seed=13, row0=7, p_fire=0.8)
    ref = []
    _, fr = O.rollout(cell, x, g4, cl, STEPS, "bf16", step0=5, trace=lambda t, s: ref.append(s.clone()),
                      **kw)
    xd, gd, cd = x.to(DEV), g4.to(DEV), cl.to(DEV)
    states, fired = _per_step(md, xd, gd, cd, STEPS, "bf16", step0=5, **kw)
    B, C, H, W = x.shape
    host = [s.cpu() for s in states]
    masks = [O.fire_masks_np(13, 7, B, 5 + t, H, W, 0.8) for t in range(STEPS)]
    step_errs = one_step_errors(cell, x, host, g4, cl, masks, "bf16")
    drift = [(s - r).abs().max().item() for s, r in zip(host, ref)]
    _say(f"worst one-step error {max(step_errs):.3g}, trajectory drift {max(drift):.3g} "
         f"(at step {int(np.argmax(drift))}, guard {drift_guard('stream32_uniform'):.3g})")
    assert max(step_errs) <= TOL["bf16"]
    assert max(drift) <= drift_guard("stream32_uniform")
    assert torch.equal(fired, fr)
    with torch.no_grad():
        fused, _, ff = rollout_steps(md, xd, gd, cd, STEPS, step0=5, precision="bf16",
                                     want_fired=True, **kw)
    assert torch.equal(fused, states[-1]) and torch.equal(ff.cpu().long(), fr)


@pytest.mark.parametrize("tau_kind", ["configured", "median"])
def test_stream32_30x30_gated_64_steps(tau_kind):
    _say("stream32 30x30 gated, 64 per-step states", tau_kind)
    m, md, x, g4, cl, _ = _maze("maze_hard_c32", 3, 30, k=2, seed=1, extra=0.10)
    cell = oracle_cell(m)
    p = 0.8
    cc0, _, _ = O.readout(cell, x)
    tau = 0.9 if tau_kind == "configured" else float(np.median(cc0))
    B, C, H, W = x.shape
    kw = dict(seed=4, p_fire=p, p_low=0.25 * p, tau=tau)
    xd, gd, cd = x.to(DEV), g4.to(DEV), cl.to(DEV)
    states, fired = _per_step(md, xd, gd, cd, STEPS, "bf16", **kw)
    # the GPU's mask of every step, from the GPU's state before it (the readout is bit-exact)
    masks, n_low, prev = [], 0, xd
    for t in range(STEPS):
        with torch.no_grad():
            conf_cell, _, _ = readout(md, prev)
        mk = fire_mask(B, H, W, 4, t, p, p_low=0.25 * p, tau=tau, conf_cell=conf_cell, given=gd[:, 0])
        # the oracle's own gating decision from the same state
        g_np = g4.reshape(B, H * W).numpy().astype(np.uint8)
        oc, _, _ = O.readout(cell, prev.cpu())
        om = clib.fire_mask(4, 0, B, t, H * W, p, 0.25 * p, tau, oc, g_np)
        assert np.array_equal(mk.cpu().numpy().reshape(B, H * W), om), t
        n_low += int((torch.from_numpy(oc) > tau).sum())
        masks.append(mk.cpu())
        prev = states[t]
    assert torch.equal(fired, torch.stack(masks).sum(dim=(0, 2, 3, 4)).long())
    _say("confident cell-steps", n_low, "of", STEPS * B * H * W)
    assert 0 < n_low < STEPS * B * H * W or tau_kind == "configured"
    ref = []
    O.rollout(cell, x, g4, cl, STEPS, "bf16", masks=torch.stack(masks),
              trace=lambda t, s: ref.append(s.clone()))
    host = [s.cpu() for s in states]
    step_errs = one_step_errors(cell, x, host, g4, cl, masks, "bf16")
    drift = [(s - r).abs().max().item() for s, r in zip(host, ref)]
    guard = drift_guard(f"stream32_gated/{tau_kind}")
    _say(f"worst one-step error {max(step_errs):.3g}, trajectory drift {max(drift):.3g} "
         f"(at step {int(np.argmax(drift))}, guard {guard:.3g})")
    assert max(step_errs) <= TOL["bf16"]
    assert max(drift) <= guard
    with torch.no_grad():
        fused, _, ff = rollout_steps(md, xd, gd, cd, STEPS, precision="bf16", want_fired=True, **kw)
    assert torch.equal(fused, states[-1]) and torch.equal(ff.cpu().long(), fired)


@pytest.mark.parametrize("precision,path", [("bf16", 0), ("fp32", 3)])
def test_maze201_per_step_path_64_steps(precision, path):
    """bf16: the wave-per-tile kernel (automatic choice); fp32: the halo-window kernel."""
    _say("201x201, 64 per-step states", precision, "path", path)
    m, md, x, g4, cl, _ = _maze("maze_c16", 2, 201)
    cell = oracle_cell(m)
    kw = dict(seed=3, row0=1, p_fire=0.5)
    ref = []
    _, fr = O.rollout(cell, x, g4, cl, STEPS, precision, trace=lambda t, s: ref.append(s.clone()), **kw)
    L = _lib.load()
    xd, gd, cd = x.to(DEV), g4.to(DEV), cl.to(DEV)
    try:
        assert L.nca_set_kernel_path(path) == 0
        states, fired = _per_step(md, xd, gd, cd, STEPS, precision, **kw)
        with torch.no_grad():
            fused, _, ff = rollout_steps(md, xd, gd, cd, STEPS, precision=precision,
                                         want_fired=True, **kw)
    finally:
        L.nca_set_kernel_path(0)
    B, C, H, W = x.shape
    host = [s.cpu() for s in states]
    drift = [(s - r).abs().max().item() for s, r in zip(host, ref)]
    if precision == "fp32":
        _say(f"worst per-step error {max(drift):.3g} at step {int(np.argmax(drift))}")
        assert max(drift) <= TOL["fp32"]
    else:
        masks = [O.fire_masks_np(3, 1, B, t, H, W, 0.5) for t in range(STEPS)]
        step_errs = one_step_errors(cell, x, host, g4, cl, masks, "bf16")
        _say(f"worst one-step error {max(step_errs):.3g}, trajectory drift {max(drift):.3g} "
             f"(at step {int(np.argmax(drift))}, guard {drift_guard('maze201'):.3g})")
        assert max(step_errs) <= TOL["bf16"]
        assert max(drift) <= drift_guard("maze201")
    assert torch.equal(fired, fr)
    assert torch.equal(fused, states[-1]) and torch.equal(ff.cpu().long(), fr)


def test_bptt_bf16_30x30_32_step_chunk():
    """The training chunk's shape: 30x30 hard mazes, C=32, bf16, 32 steps (2 boards), every step
    supervised, Philox masks from per-step keys, against the fp64 straight-through oracle."""
    _say("bptt bf16 30x30 32-step chunk")
    m, md, x, g4, cl, b = _maze("maze_hard_c32", 2, 30, extra=0.10)
    B, C, H, W = x.shape
    n = 32
    seeds = [1000 + 7 * t for t in range(n)]
    masks = torch.stack([O.fire_masks_np(s, 0, B, t, H, W, 0.8) for t, s in enumerate(seeds)])
    targets = md.output_index(torch.from_numpy(b.targets))
    weights = [1.0] * n
    with torch.no_grad():
        res = bptt_chunk(md, x.to(DEV), g4.to(DEV), cl.to(DEV), targets.to(DEV), weights,
                         step_seeds=seeds, p_fire=0.8, precision="bf16", want_grad_x0=True)
    loss, ref = O.bptt_chunk(oracle_cell(m), x, g4, cl, masks.double(), targets, weights, "bf16",
                             grad_x0=True, grad_round=True)

    def rel(a, r):
        a, r = a.detach().double().cpu().reshape(-1), r.detach().double().cpu().reshape(-1)
        return float((a - r).norm() / r.norm().clamp_min(1e-30))

    errs = {k: rel(res.grads[k], ref[k]) for k in NAMES}
    errs["x0"] = rel(res.grad_x0, ref["x0"])
    _say("loss", float(res.loss), loss, "relative gradient errors", errs)
    assert abs(float(res.loss) - loss) <= 2e-2 * abs(loss)
    assert max(errs[k] for k in NAMES) <= 2e-2
    assert errs["x0"] <= drift_guard("bptt_x0")
