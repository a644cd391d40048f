"""The evidence behind the GPU tests' bf16 trajectory guards: the oracle's own bf16 trajectories,
run with only the fp32 summation order changed (oracle.nca_oracle.SUM_ORDERS), drift apart by
the amounts in cells.BF16_SELF_DRIFT, for the exact configuration of every GPU trajectory test
(same cells, boards, initial states, Philox keys and steps). The GPU's trajectories are held
within DRIFT_MARGIN (1.5) times these. A value in the table above what is measured here fails.

The reference holds its own bf16 backends to 2e-2 on the state (src/nca/engine/bench.py:
500-509); for the cells whose dynamics amplify bf16 rounding flips the oracle cannot meet that
bar against itself over 64 steps (201x201: 0.20), which is why the bar is applied per step from
the GPU's own state and the trajectory is held to the measured self-drift instead.
"""

from __future__ import annotations

import itertools
import sys

import numpy as np
import pytest
import torch

sys.path.insert(0, __file__.rsplit("/", 1)[0])
from cells import (BF16_SELF_DRIFT, CELLS, DYN, boards_for, initial_state, make_model,  # noqa: E402
                   oracle_cell, perturbed_model)

from ncas_amd.tasks import maze_boards  # noqa: E402
from oracle import clib  # noqa: E402
from oracle import nca_oracle as O  # noqa: E402


@pytest.fixture(scope="module", autouse=True)
def _threads():
    clib.build()
    n = torch.get_num_threads()
    torch.set_num_threads(max(1, min(8, torch.get_num_threads())))
    yield
    torch.set_num_threads(n)


def _self_drift(cell, x, g4, cl, n, last_only=False, **kw) -> float:
    trs = {}
    for order in O.SUM_ORDERS:
        states = []
        O.rollout(cell, x, g4, cl, n, "bf16", order=order,
                  trace=lambda t, s: states.append(s.clone()), **kw)
        trs[order] = states[-1:] if last_only else states
    return max(max((p - q).abs().max().item() for p, q in zip(trs[a], trs[b]))
               for a, b in itertools.combinations(trs, 2))


def _check(key, measured):
    print(f"{key}: self-drift {measured:.5f} (table {BF16_SELF_DRIFT[key]})", flush=True)
    assert BF16_SELF_DRIFT[key] <= measured * (1 + 1e-6), (key, measured)


@pytest.mark.parametrize("name", list(CELLS))
def test_rollout64_self_drift(name):
    # tests/test_gpu_parity.py::test_rollout_64_steps_matches_oracle
    preset, size = CELLS[name]
    m = make_model(name, 0)
    x, g4, cl = initial_state(m, boards_for(preset, 2, size, 0), k=3, sigma=0.15, seed=0)
    _check(f"rollout64/{name}", _self_drift(oracle_cell(m), x, g4, cl, 64, seed=5, row0=11,
                                            step0=3, p_fire=m.cfg.fire_rate))


@pytest.mark.parametrize("name", ["maze_c16", "sudoku_c64", "maze_hard_c32", "ref_maze_ood"])
@pytest.mark.parametrize("n_boards,k", [(5, 3), (1, 1), (33, 2)])
def test_ws24_self_drift(name, n_boards, k):
    # tests/test_gpu_parity.py::test_wave_specialised_and_generic_kernels_agree
    preset, size = CELLS[name]
    m = make_model(name, 0)
    x, g4, cl = initial_state(m, boards_for(preset, n_boards, size, 0), k=k, sigma=0.15, seed=0)
    _check(f"ws24/{name}/{n_boards}x{k}",
           _self_drift(oracle_cell(m), x, g4, cl, 24, last_only=True, seed=4, p_fire=0.6))


def _maze(preset, n, size, k=1, seed=0, extra=0.0):
    m = perturbed_model(preset, seed, *DYN[preset])
    x, g4, cl = initial_state(m, maze_boards(n, size, seed, extra_openings=extra), k=k,
                              sigma=0.15, seed=seed)
    return m, x, g4, cl


def test_stream32_uniform_self_drift():
    # tests/test_gpu_long.py::test_stream32_30x30_uniform_64_steps
    m, x, g4, cl = _maze("maze_hard_c32", 3, 30, k=2, extra=0.10)
    _check("stream32_uniform", _self_drift(oracle_cell(m), x, g4, cl, 64, seed=13, row0=7,
                                           step0=5, p_fire=0.8))


@pytest.mark.parametrize("tau_kind", ["configured", "median"])
def test_stream32_gated_self_drift(tau_kind):
    # tests/test_gpu_long.py::test_stream32_30x30_gated_64_steps: the gating decisions of the
    # torch-order trajectory are injected into every order
    m, x, g4, cl = _maze("maze_hard_c32", 3, 30, k=2, seed=1, extra=0.10)
    cell = oracle_cell(m)
    cc0, _, _ = O.readout(cell, x)
    tau = 0.9 if tau_kind == "configured" else float(np.median(cc0))
    B, C, H, W = x.shape
    g_np = g4.reshape(B, H * W).numpy().astype(np.uint8)
    masks, cur = [], x
    for t in range(64):
        oc, _, _ = O.readout(cell, cur)
        mk = torch.from_numpy(clib.fire_mask(4, 0, B, t, H * W, 0.8, 0.2, tau, oc, g_np)
                              .astype(np.float32)).reshape(B, 1, H, W)
        masks.append(mk)
        cur = O.step(cell, cur, g4, cl, mk, "bf16").float()
    _check(f"stream32_gated/{tau_kind}",
           _self_drift(cell, x, g4, cl, 64, masks=torch.stack(masks)))


def test_maze201_self_drift():
    # tests/test_gpu_long.py::test_maze201_per_step_path_64_steps (bf16)
    m, x, g4, cl = _maze("maze_c16", 2, 201)
    _check("maze201", _self_drift(oracle_cell(m), x, g4, cl, 64, seed=3, row0=1, p_fire=0.5))


def test_bptt_x0_gradient_self_drift():
    # tests/test_gpu_long.py::test_bptt_bf16_30x30_32_step_chunk
    m, x, g4, cl = _maze("maze_hard_c32", 2, 30, extra=0.10)
    b = maze_boards(2, 30, 0, extra_openings=0.10)
    B, C, H, W = x.shape
    seeds = [1000 + 7 * t for t in range(32)]
    masks = torch.stack([O.fire_masks_np(s, 0, B, t, H, W, 0.8) for t, s in enumerate(seeds)])
    targets = m.output_index(torch.from_numpy(b.targets))
    cell = oracle_cell(m)
    kw = dict(grad_x0=True, grad_round=True)
    _, g64 = O.bptt_chunk(cell, x, g4, cl, masks.double(), targets, [1.0] * 32, "bf16", **kw)
    _, g32 = O.bptt_chunk(cell, x, g4, cl, masks.float(), targets, [1.0] * 32, "bf16",
                          dtype=torch.float32, **kw)
    a, r = g32["x0"].double(), g64["x0"].double()
    _check("bptt_x0", float((a - r).norm() / r.norm()))
