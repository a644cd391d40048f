"""Shared test fixtures: cells with non-trivial synthetic weights, boards, and the oracle view of
a product model (tests may import both the product and the oracle)."""

from __future__ import annotations

import numpy as np
import torch

from ncas_amd.model import build_model
from ncas_amd.tasks import maze_boards, sudoku_boards
from oracle.nca_oracle import OracleCell

import json
import os

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

# name -> (preset, grid) of the cells the parity tests run
CELLS = {
    "maze_c16": ("maze_c16", 13),  # C=16, MLP 64 -> 128 -> 16, wall padding, mlp head
    "sudoku_c64": ("sudoku_c64", 9),  # C=64, MLP 256 -> 256 -> 64, wrap padding, mlp head
    "maze_hard_c32": ("maze_hard_c32", 9),  # C=32, MLP 128 -> 256 -> 32
    "ref_maze_ood": ("maze_ood", 9),  # the reference's trained C=16 maze cell (l2 head)
    "ref_maze_hard": ("maze_hard", 9),  # the reference's trained C=32 maze cell (l2 head)
}
# (scale, decay) of perturbed_model per preset: bounded dynamics that keep moving
DYN = {"maze_c16": (2.0, 1.0), "sudoku_c64": (1.3, 0.3), "maze_hard_c32": (1.8, 0.8)}


def reference_trained_model(name: str):
    """The reference's trained maze_ood / maze_hard weights (tests/golden/ref_<name>.npz)."""
    from ncas_amd.model import NCA, NCAConfig

    with open(os.path.join(GOLDEN, f"ref_{name}.json")) as f:
        cfg = json.load(f)
    m = NCA(NCAConfig.from_dict(cfg))
    sd = {k: torch.from_numpy(v) for k, v in np.load(os.path.join(GOLDEN, f"ref_{name}.npz")).items()}
    m.load_state_dict(sd)
    return m


def make_model(name: str, seed: int = 0):
    preset, _ = CELLS[name]
    if name.startswith("ref_"):
        return reference_trained_model(preset)
    scale, decay = DYN[preset]
    return perturbed_model(preset, seed, scale=scale, decay=decay)


def perturbed_model(preset: str, seed: int = 0, scale: float = 1.0, decay: float = 0.5,
                    **overrides):
    """A cell whose dynamics move but stay bounded: fc1 ~ N(0, 1/F), fc2 ~ N(0, 0.25/hidden),
    biases ~ N(0, 0.01), head ~ N(0, 1/c_out), all drawn from torch.Generator(seed); then the
    first 2C hidden units are wired as a leak dx_c -= decay * x_c through the identity kernel
    (relu(x) - relu(-x) = x), which keeps the random part of the update from diverging."""
    m = build_model(preset, **overrides)
    g = torch.Generator().manual_seed(seed)
    C = m.cfg.channels
    F = m.perceive.out_dim
    hid = m.cfg.hidden
    with torch.no_grad():
        w1 = torch.randn(hid, F, generator=g) * (scale / F**0.5)
        b1 = torch.randn(hid, generator=g) * 0.01
        w2 = torch.randn(C, hid, generator=g) * (0.5 * scale / hid**0.5)
        b2 = torch.randn(C, generator=g) * 0.01
        if decay:
            ident = torch.zeros(3, 3)
            ident[1, 1] = 1.0
            m.perceive.weight[0, 0] = ident  # kernel 0 = identity (as in the fixed kernels)
            for c in range(C):
                w1[2 * c], w1[2 * c + 1] = 0.0, 0.0
                w1[2 * c, c], w1[2 * c + 1, c] = 1.0, -1.0
                b1[2 * c], b1[2 * c + 1] = 0.0, 0.0
                w2[:, 2 * c], w2[:, 2 * c + 1] = 0.0, 0.0
                w2[c, 2 * c], w2[c, 2 * c + 1] = -decay, decay
        m.update.fc1.weight.copy_(w1.reshape(m.update.fc1.weight.shape))
        m.update.fc1.bias.copy_(b1)
        m.update.fc2.weight.copy_(w2.reshape(m.update.fc2.weight.shape))
        m.update.fc2.bias.copy_(b2)
        if m.cfg.head == "mlp":
            m.head.weight.copy_(torch.randn(m.head.weight.shape, generator=g) * (1.0 / m.cfg.c_out**0.5))
            m.head.bias.copy_(torch.randn(m.head.bias.shape, generator=g) * 0.1)
    return m


def boards_for(preset: str, n: int, size: int, seed: int = 0):
    if preset.startswith("sudoku"):
        return sudoku_boards(n, seed)
    if preset in ("maze_ood", "maze_hard"):
        # the reference's maze vocabularies: empty 0, path 1, wall 2, endpoint 3 (maze_ood) or
        # start 3 / goal 4 (maze_hard); our generator's tokens are open 0, wall 1, start 2,
        # goal 3, path 4
        from ncas_amd.tasks import Boards

        b = maze_boards(n, size, seed)
        remap = np.array([0, 2, 3, 3, 1]) if preset == "maze_ood" else np.array([0, 2, 3, 4, 1])
        inputs, targets = remap[b.inputs], remap[b.targets]
        return Boards(inputs, targets, inputs >= 2)
    return maze_boards(n, size, seed)


def initial_state(model, boards, k: int = 1, sigma: float = 0.0, seed: int = 0):
    """(x, given4, clamp) on CPU for boards repeated k times; x ~ N(0, sigma) then clamped."""
    inputs = torch.from_numpy(np.repeat(boards.inputs, k, 0))
    given = torch.from_numpy(np.repeat(boards.given, k, 0))
    B, H, W = inputs.shape
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((B, model.cfg.channels, H, W), generator=g) * sigma
    given4 = given[:, None]
    clamp = model.clamp_values(inputs)
    return model.apply_clamp(x, given4, clamp).contiguous(), given4, clamp


def oracle_cell(model) -> OracleCell:
    cfg = model.cfg
    if cfg.head == "mlp":
        hw, hb = model.head.weight.detach().reshape(len(cfg.output_tokens), -1), model.head.bias.detach()
    else:
        hw, hb = model.out_embed.detach(), None
    return OracleCell(
        channels=cfg.channels, heads=cfg.heads, hidden=cfg.hidden, c_in=cfg.c_in,
        in_offset=cfg.in_offset, c_out=cfg.c_out, out_offset=cfg.out_offset,
        padding=cfg.padding, head=cfg.head,
        kernels=model.perceive.weight.detach().clone(),
        w1=model.update.fc1.weight.detach().reshape(cfg.hidden, -1).clone(),
        b1=model.update.fc1.bias.detach().clone(),
        w2=model.update.fc2.weight.detach().reshape(cfg.channels, -1).clone(),
        b2=model.update.fc2.bias.detach().clone(),
        head_w=hw.clone().float(), head_b=None if hb is None else hb.clone().float(),
        pad_vec=model.pad_vec.detach().clone(),
    )


def one_step_errors(cell, x0, states, given4, clamp, masks, precision):
    """Max-abs error of every step of a GPU trajectory against the oracle's step from the GPU's
    own previous state: states[t] (CPU) vs O.step(states[t - 1], masks[t]) (states[-1] = x0).
    In bf16 this is the per-step bar: a trajectory comparison also counts the amplification of
    bf16 rounding flips (fp32 sums in another order landing on the other side of a bf16 rounding
    boundary), which grows with the number of steps for cells whose dynamics amplify them."""
    from oracle import nca_oracle as O

    errs, prev = [], x0
    for t, s in enumerate(states):
        ref = O.step(cell, prev, given4, clamp, masks[t], precision).float()
        errs.append((s - ref).abs().max().item())
        prev = s
    return errs


# ------------------------------------------------------------------------------ bf16 drift
# How far the oracle's own bf16 trajectory moves when only the fp32 summation order of its sums
# changes: the largest max-abs state difference, over the trajectory's steps and over every pair
# of the oracle's orders (oracle.nca_oracle.SUM_ORDERS: torch's conv / GEMM, one rounding of the
# exact sum, blocks of 32 or 8 products ascending, blocks of 32 descending), for the exact
# configuration of each GPU trajectory test. A bf16 step rounds z, h and dx after fp32 sums, so
# two correct implementations that sum in different orders land on different sides of a bf16
# rounding boundary now and then, and the cell's dynamics amplify those flips along a trajectory.
# The GPU kernels are one more summation order: their trajectories are held within
# DRIFT_MARGIN times these values. tests/test_oracle_drift.py recomputes every value and fails
# when one here is above what it measures (values are rounded down). "bptt_x0": the relative
# norm difference of the chunk's initial-state gradient between fp32 and fp64 sums.
BF16_SELF_DRIFT = {
    "rollout64/maze_c16": 0.0301, "rollout64/sudoku_c64": 0.0024,
    "rollout64/maze_hard_c32": 0.0153, "rollout64/ref_maze_ood": 0.0401,
    "rollout64/ref_maze_hard": 0.0266,
    "stream32_uniform": 0.0136, "stream32_gated/configured": 0.0046,
    "stream32_gated/median": 0.0046, "maze201": 0.2047,
    "ws24/maze_c16/5x3": 0.0131, "ws24/maze_c16/1x1": 0.0083, "ws24/maze_c16/33x2": 0.0148,
    "ws24/sudoku_c64/5x3": 0.0016, "ws24/sudoku_c64/1x1": 0.0010,
    "ws24/sudoku_c64/33x2": 0.0017, "ws24/maze_hard_c32/5x3": 0.0080,
    "ws24/maze_hard_c32/1x1": 0.0073, "ws24/maze_hard_c32/33x2": 0.0089,
    "ws24/ref_maze_ood/5x3": 0.0092, "ws24/ref_maze_ood/1x1": 0.00006,
    "ws24/ref_maze_ood/33x2": 0.0265,
    "bptt_x0": 0.0284,
}
DRIFT_MARGIN = 1.5


def drift_guard(key: str) -> float:
    """The GPU's bf16 trajectory guard for configuration `key`."""
    return DRIFT_MARGIN * BF16_SELF_DRIFT[key]
