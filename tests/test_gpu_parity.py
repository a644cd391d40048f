"""Parity of the HIP path (through the C ABI) with the CPU oracle, on the GPU.

Bars (north star): fire masks, readout, decoded argmax and conf@K indices bit-exact; per-step
states within max-abs 1e-4 (fp32) / 2e-2 (bf16) of the oracle over the first 64 steps, with
the same Philox masks.
"""

from __future__ import annotations

import copy
import sys

import numpy as np
import pytest
import torch

sys.path.insert(0, __file__.rsplit("/", 1)[0])
from cells import (CELLS, boards_for, drift_guard, initial_state, make_model,  # noqa: E402
                   one_step_errors, oracle_cell)

from ncas_amd.inference import rollout_steps  # noqa: E402
from ncas_amd.readout import conf_select, readout  # noqa: E402
from ncas_amd.rng import fire_mask  # noqa: E402
from ncas_amd.step import make_step  # noqa: E402
from oracle import clib  # noqa: E402
from oracle import nca_oracle as O  # noqa: E402

pytestmark = pytest.mark.gpu
TOL = {"fp32": 1e-4, "bf16": 2e-2}
DEV = torch.device("cuda:0")


def state_error(name, precision, y, ref):
    """Max-abs state error as a fraction of the north-star bar (<= 1 passes): 1e-4 (fp32) or
    2e-2 (bf16), absolute for every cell, the reference's trained cells included (the reference
    compares states absolutely, src/nca/engine/bench.py:500-509)."""
    del name
    return (y - ref).abs().max().item() / TOL[precision]


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    clib.build()


def _say(*a):
    print(*a, flush=True)


def _case(name, n_boards=2, k=3, sigma=0.15, seed=0):
    preset, size = CELLS[name]
    m = make_model(name, seed)
    b = boards_for(preset, n_boards, size, seed)
    x, g4, cl = initial_state(m, b, k=k, sigma=sigma, seed=seed)
    return m, copy.deepcopy(m).to(DEV), x, g4, cl


# ------------------------------------------------------------------------------ fire masks
@pytest.mark.parametrize("rows,H,W", [(7, 9, 9), (3, 13, 13), (2, 30, 30), (5, 1, 3), (1, 201, 201)])
def test_fire_mask_bit_exact(rows, H, W):
    _say("fire mask", rows, H, W)
    for seed, row0, step in ((0, 0, 0), (2**62 + 12345, 77, 1234), (99, 2**31 - 5, 2**32 - 1)):
        got = fire_mask(rows, H, W, seed, step, 0.5, row0=row0, device=DEV)
        ref = clib.fire_mask(seed, row0, rows, step, H * W, 0.5)
        assert np.array_equal(got.cpu().numpy().reshape(rows, H * W), ref)
    rng = np.random.default_rng(0)
    conf = rng.random((rows, H * W)).astype(np.float32)
    given = rng.random((rows, H * W)) < 0.3
    got = fire_mask(rows, H, W, 5, 9, 0.8, row0=3, p_low=0.2, tau=0.6,
                    conf_cell=torch.from_numpy(conf).to(DEV),
                    given=torch.from_numpy(given).to(DEV))
    ref = clib.fire_mask(5, 3, rows, 9, H * W, 0.8, 0.2, 0.6, conf, given)
    assert np.array_equal(got.cpu().numpy().reshape(rows, H * W), ref)


# ------------------------------------------------------------------------------ readout
@pytest.mark.parametrize("name", list(CELLS))
def test_readout_bit_exact(name):
    _say("readout", name)
    m, md, x, _, _ = _case(name, n_boards=4, k=5, sigma=0.7)
    x[0, :, :3, :3] = 0.0  # cells whose logits are the head bias only
    cc, cb, am = readout(md, x.to(DEV))
    rc, rb, ra = O.readout(oracle_cell(m), x)
    assert np.array_equal(cc.cpu().numpy().view(np.int32), rc.view(np.int32))
    assert np.array_equal(cb.cpu().numpy().view(np.int32), rb.view(np.int32))
    assert np.array_equal(am.cpu().numpy(), ra)


def test_readout_ties_take_the_first_maximum():
    m, md, x, _, _ = _case("sudoku_c64", n_boards=2, k=1)
    with torch.no_grad():
        md.head.bias.fill_(0.25)
        m.head.bias.fill_(0.25)
    x[:, m.cfg.out_slice] = 0.0  # all logits equal
    cc, cb, am = readout(md, x.to(DEV))
    assert int(am.abs().sum()) == 0
    assert torch.allclose(cc.cpu(), torch.full_like(cc.cpu(), 1 / 9), atol=1e-7)


# ------------------------------------------------------------------------------ conf@K
@pytest.mark.parametrize("N,K", [(300, 128), (5, 1), (64, 65), (1000, 64)])
def test_conf_select_bit_exact(N, K):
    _say("conf select", N, K)
    rng = np.random.default_rng(N * 1000 + K)
    conf = rng.random((N, K)).astype(np.float32)
    conf[:, K // 2] = conf[:, 0]  # planted ties with trial 0
    conf[rng.random((N, K)) < 0.05] = 1.0  # many equal maxima
    conf[rng.random((N, K)) < 0.02] = -np.inf
    alive = rng.random((N, K)) < 0.9
    alive[0] = False  # a board with no alive trial -> index 0
    for k in sorted({1, 7, K // 2 or 1, K}):
        for al in (None, alive):
            got = conf_select(torch.from_numpy(conf).to(DEV),
                              None if al is None else torch.from_numpy(al).to(DEV), k)
            ref = clib.conf_select(conf, al, k)
            assert np.array_equal(got.cpu().numpy(), ref), (k, al is None)
            # and the reference's numpy rule (rollout.py:331-333)
            c = np.where(al[:, :k] if al is not None else True, conf[:, :k], -np.inf)
            assert np.array_equal(ref, c.argmax(axis=1))


# ------------------------------------------------------------------------------ one step
@pytest.mark.parametrize("precision", ["fp32", "bf16"])
@pytest.mark.parametrize("name", list(CELLS))
def test_step_matches_oracle(name, precision):
    _say("step", name, precision)
    m, md, x, g4, cl = _case(name)
    cell = oracle_cell(m)
    B, C, H, W = x.shape
    fires = {
        "philox": O.fire_masks_np(3, 0, B, 0, H, W, 0.5),
        "zeros": torch.zeros(B, 1, H, W),
        "ones": torch.ones(B, 1, H, W),
        "half": torch.full((B, 1, H, W), 0.5),
    }
    noise = torch.randn(x.shape, generator=torch.Generator().manual_seed(1)) * 0.2
    step = make_step(md, precision=precision)
    for fname, fire in fires.items():
        for nz in (None, noise):
            with torch.no_grad():
                y = step(x.to(DEV), g4.to(DEV), cl.to(DEV), fire.to(DEV),
                         None if nz is None else nz.to(DEV)).cpu()
            ref = O.step(cell, x, g4, cl, fire, precision, nz)
            err = state_error(name, precision, y, ref)
            assert err <= 1.0, (fname, nz is None, err)
            if fname == "zeros" and nz is None:
                assert torch.equal(y, x)  # a zero mask is the identity (x is clamped already)


def test_step_under_bf16_autocast_is_the_bf16_path():
    m, md, x, g4, cl = _case("sudoku_c64")
    fire = O.fire_masks_np(3, 0, x.shape[0], 0, 9, 9, 0.5).to(DEV)
    step = make_step(md)
    with torch.no_grad():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            a = step(x.to(DEV), g4.to(DEV), cl.to(DEV), fire)
        b = make_step(md, precision="bf16")(x.to(DEV), g4.to(DEV), cl.to(DEV), fire)
    assert a.dtype == torch.float32 and torch.equal(a, b)


# ------------------------------------------------------------------------------ rollouts
@pytest.mark.parametrize("precision", ["fp32", "bf16"])
@pytest.mark.parametrize("name", list(CELLS))
def test_rollout_64_steps_matches_oracle(name, precision):
    """Every one of the first 64 states within tolerance; fused == chained single steps."""
    _say("rollout64", name, precision)
    m, md, x, g4, cl = _case(name)
    cell = oracle_cell(m)
    p = m.cfg.fire_rate
    ref_states = []
    xr, fired_ref = O.rollout(cell, x, g4, cl, 64, precision, seed=5, row0=11, step0=3, p_fire=p,
                              trace=lambda t, s: ref_states.append(s.clone()))
    xd, gd, cd = x.to(DEV), g4.to(DEV), cl.to(DEV)
    B, C, H, W = x.shape
    states = []
    with torch.no_grad():
        cur = xd.clone()
        fired = torch.zeros(x.shape[0], dtype=torch.int64)
        for t in range(64):
            cur, _, f = rollout_steps(md, cur, gd, cd, 1, seed=5, row0=11, step0=3 + t, p_fire=p,
                                      precision=precision, want_fired=True)
            fired += f.cpu().long()
            states.append(cur.cpu())
        fused, conf, ff = rollout_steps(md, xd, gd, cd, 64, seed=5, row0=11, step0=3, p_fire=p,
                                        precision=precision, want_fired=True)
    traj = [(s - r).abs().max().item() for s, r in zip(states, ref_states)]
    masks = [O.fire_masks_np(5, 11, B, 3 + t, H, W, p) for t in range(64)]
    step_errs = one_step_errors(cell, x, states, g4, cl, masks, precision)
    _say(f"worst one-step error {max(step_errs):.3g}, trajectory drift {max(traj):.3g} "
         f"(bar {TOL[precision]})")
    assert max(step_errs) <= TOL[precision]
    if precision == "fp32":
        assert max(traj) <= TOL["fp32"]
    else:  # bf16: within 1.5x the oracle's own drift under another fp32 summation order
        assert max(traj) <= drift_guard(f"rollout64/{name}"), drift_guard(f"rollout64/{name}")
    assert torch.equal(fused, cur), "fused rollout differs from chained single steps"
    assert torch.equal(fired, fired_ref) and torch.equal(ff.cpu().long(), fired_ref)
    # the in-kernel board confidence is the readout of the final state, bit for bit
    _, rb, _ = O.readout(cell, fused.cpu())
    assert np.array_equal(conf.cpu().numpy().view(np.int32), rb.view(np.int32))


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_rollout_is_segment_and_row_invariant(precision):
    _say("segments", precision)
    m, md, x, g4, cl = _case("sudoku_c64", n_boards=3, k=4)
    xd, gd, cd = x.to(DEV), g4.to(DEV), cl.to(DEV)
    with torch.no_grad():
        full, _, _ = rollout_steps(md, xd, gd, cd, 40, seed=7, precision=precision)
        a, _, _ = rollout_steps(md, xd, gd, cd, 10, seed=7, precision=precision)
        b, _, _ = rollout_steps(md, a, gd, cd, 30, seed=7, step0=10, precision=precision)
        part, _, _ = rollout_steps(md, xd[5:9], gd[5:9], cd[5:9], 40, seed=7, row0=5,
                                   precision=precision)
    assert torch.equal(full, b)
    assert torch.equal(full[5:9], part)


def test_injected_masks_match_oracle():
    m, md, x, g4, cl = _case("maze_c16")
    B, C, H, W = x.shape
    g = torch.Generator().manual_seed(3)
    masks = (torch.rand((12, B, 1, H, W), generator=g) < 0.3).float()
    xr, _ = O.rollout(oracle_cell(m), x, g4, cl, 12, "fp32", masks=masks)
    with torch.no_grad():
        y, _, _ = rollout_steps(md, x.to(DEV), g4.to(DEV), cl.to(DEV), 12, masks=masks.to(DEV))
    assert (y.cpu() - xr).abs().max().item() <= TOL["fp32"]


@pytest.mark.parametrize("name", ["maze_c16", "sudoku_c64"])
def test_adaptive_firing_step_by_step(name):
    """Confidence-gated firing: from the same state the GPU draws the oracle's mask bit for bit
    (its readout is bit-exact), so each gated step matches the oracle's step."""
    _say("adaptive", name)
    m, md, x, g4, cl = _case(name)
    cell = oracle_cell(m)
    p, p_low = 0.8, 0.2
    _, _, _ = O.readout(cell, x)
    cc0, _, _ = O.readout(cell, x)
    tau = float(np.median(cc0))  # half the cells confident
    cur = x.clone()
    xd_g, cd = g4.to(DEV), cl.to(DEV)
    for t in range(12):
        with torch.no_grad():
            y, _, f = rollout_steps(md, cur.to(DEV), xd_g, cd, 1, seed=2, step0=t, p_fire=p,
                                    p_low=p_low, tau=tau, precision="fp32", want_fired=True)
        yr, fr = O.rollout(cell, cur, g4, cl, 1, "fp32", seed=2, step0=t, p_fire=p, p_low=p_low,
                           tau=tau)
        assert torch.equal(f.cpu().long(), fr), t
        assert (y.cpu() - yr).abs().max().item() <= TOL["fp32"]
        cur = y.cpu()


def test_full_c3_batch_rows_match_oracle():
    """32,768 rows of the 9x9 C=64 cell (256 boards x K=128): 8 steps on the GPU, rows sampled
    from the start, middle and end checked against the oracle."""
    _say("c3 full batch")
    from ncas_amd.tasks import sudoku_boards
    from cells import perturbed_model, DYN

    m = perturbed_model("sudoku_c64", 0, *DYN["sudoku_c64"])
    md = copy.deepcopy(m).to(DEV)
    b = sudoku_boards(256, 0)
    x, g4, cl = initial_state(m, b, k=128, sigma=0.15)
    cell = oracle_cell(m)
    for precision in ("fp32", "bf16"):
        with torch.no_grad():
            y, conf, _ = rollout_steps(md, x.to(DEV), g4.to(DEV), cl.to(DEV), 8, seed=11,
                                       precision=precision)
        y = y.cpu()
        for lo in (0, 16_384 - 8, 32_768 - 16):
            sl = slice(lo, lo + 16)
            yr, _ = O.rollout(cell, x[sl], g4[sl], cl[sl], 8, precision, seed=11, row0=lo)
            assert (y[sl] - yr).abs().max().item() <= TOL[precision], (precision, lo)
        assert torch.isfinite(conf).all()


@pytest.mark.parametrize("weights,n_boards,k,depth", [
    ("perturbed", 32, 8, 64),
    ("perturbed", 4, 128, 256),  # the Sudoku conf@K workload's K and D
    ("benchmark", 4, 128, 256),  # ... with its synthetic N(0, 0.02) weights and zero state
])
def test_decode_and_selection_bit_exact_fp32(weights, n_boards, k, depth):
    """fp32 trajectories of n_boards x k rows over `depth` steps: every decoded argmax and every
    conf@K index (k' = 1, 8, 32, k) equals the oracle trajectory's, with no exception for
    near-ties; the smallest top-2 logit gap and the smallest conf@K gap are printed (the margins
    that fp32 summation-order differences would have to cross)."""
    _say("decode + conf@K", weights, n_boards, k, depth)
    if weights == "perturbed":
        m, md, x, g4, cl = _case("sudoku_c64", n_boards=n_boards, k=k)
    else:
        from ncas_amd.model import build_model, init_weights

        m = init_weights(build_model("sudoku_c64"), seed=0, std=0.02, zero_last=False)
        md = copy.deepcopy(m).to(DEV)
        x, g4, cl = initial_state(m, boards_for("sudoku_c64", n_boards, 9, 0), k=k)
    cell = oracle_cell(m)
    xr, _ = O.rollout(cell, x, g4, cl, depth, "fp32", seed=21)
    with torch.no_grad():
        y, conf, _ = rollout_steps(md, x.to(DEV), g4.to(DEV), cl.to(DEV), depth, seed=21)
        cc, cb, am = readout(md, y)
    rc, rb, ra = O.readout(cell, xr)
    # decode of the same state is bit-exact
    gc, gb, ga = O.readout(cell, y.cpu())
    assert np.array_equal(am.cpu().numpy(), ga) and np.array_equal(cb.cpu().numpy(), gb)
    # trajectory level: every cell's argmax
    logits = torch.einsum("vc,bchw->bvhw", cell.head_w,
                          xr[:, cell.out_offset:cell.out_offset + cell.c_out]) \
        + cell.head_b[None, :, None, None]
    top2 = logits.topk(2, dim=1).values
    margin = float((top2[:, 0] - top2[:, 1]).min())
    mism = int((am.cpu().numpy() != ra).sum())
    _say(f"argmax mismatches {mism} of {ra.size}, smallest top-2 logit gap {margin:.3g}, "
         f"largest state difference {(y.cpu() - xr).abs().max().item():.3g}")
    assert mism == 0
    # conf@K selection, for several k'
    srt = np.sort(rb.reshape(n_boards, k), axis=1)
    _say(f"smallest conf@K gap {float((srt[:, -1] - srt[:, -2]).min()):.3g}")
    for kk in sorted({1, 8, 32, k}):
        if kk > k:
            continue
        sel = conf_select(conf.view(n_boards, k), None, kk).cpu().numpy()
        ref = clib.conf_select(rb.reshape(n_boards, k), None, kk)
        assert np.array_equal(sel, ref), kk


def test_conf_at_k_and_pass_at_k_on_the_gpu():
    """The GPU conf@K / pass@K: the reference's inline known answers
    (tests/test_rollout.py:63-68, tests/test_regressions_evaluation.py:68-73), then random
    metrics with ties, dead trials and board weights against the oracle's numpy rule."""
    from ncas_amd.rollout import conf_at_k, pass_at_k

    metric = np.array([[True, False, False], [False, False, True]])
    conf = np.array([[0.1, 0.9, 0.5], [0.2, 0.3, 0.9]])
    alive = np.ones((2, 3), dtype=bool)
    assert conf_at_k(metric, conf, alive, [1, 2, 3]) == {1: 0.5, 2: 0.0, 3: 0.5}
    assert pass_at_k(metric, alive, [1, 3]) == {1: 0.5, 3: 1.0}
    m1, c1, a1 = np.array([[1.0], [0.0]]), np.ones((2, 1)), np.ones((2, 1), bool)
    assert conf_at_k(m1, c1, a1, [1])[1] == 0.5
    assert conf_at_k(m1, c1, a1, [1], weights=np.array([0.9, 0.1]))[1] == 0.9
    rng = np.random.default_rng(3)
    N, K = 300, 16
    metric = rng.random((N, K)) < 0.4
    conf = (rng.integers(0, 6, (N, K)) / 6).astype(np.float32)  # many ties
    alive = rng.random((N, K)) < 0.8
    w = rng.random(N)
    ks = [1, 2, 5, 16, 40]
    for weights in (None, w):
        got, ref = conf_at_k(metric, conf, alive, ks, weights), O.conf_at_k(metric, conf, alive, ks, weights)
        assert got.keys() == ref.keys() and all(abs(got[k] - ref[k]) <= 1e-12 for k in ref)
        got, ref = pass_at_k(metric, alive, ks, weights), O.pass_at_k(metric, alive, ks, weights)
        assert got.keys() == ref.keys() and all(abs(got[k] - ref[k]) <= 1e-12 for k in ref)


def test_rollout_api_end_to_end():
    """rollout() on Sudoku boards: shapes, given cells show their inputs, fired counts."""
    from ncas_amd.rollout import RolloutConfig, conf_at_k, pass_at_k, rollout
    from ncas_amd.tasks import sudoku_boards

    m = make_model("sudoku_c64").to(DEV)
    b = sudoku_boards(6, 3)
    rc = RolloutConfig(depth=20, k=4, record_every=8, max_cells=4 * 81 * 4, fire_rate=0.5)
    res = rollout(m, None, b, rc, seed=0)
    assert res.pred.shape == (6, 4, 9, 9) and res.conf.shape == (6, 4)
    assert list(res.steps) == [8, 16, 20]
    given = np.repeat(b.given[:, None], 4, 1)
    assert np.array_equal(res.pred[given], np.repeat(b.inputs[:, None], 4, 1)[given])
    assert 0.4 * 81 * 20 < res.cell_updates.mean() < 0.6 * 81 * 20
    # independent of chunking: one pass gives the same result
    res2 = rollout(m, None, b, RolloutConfig(depth=20, k=4, fire_rate=0.5), seed=0)
    assert np.array_equal(res.pred, res2.pred) and np.array_equal(res.conf, res2.conf)
    exact = (res.pred == b.targets[:, None]).all(axis=(2, 3))
    assert set(conf_at_k(exact, res.conf, res.alive, [1, 4])) == {1, 4}
    assert set(pass_at_k(exact, res.alive, [1, 4])) == {1, 4}


@pytest.mark.parametrize("name", ["maze_c16", "sudoku_c64", "maze_hard_c32", "ref_maze_ood"])
@pytest.mark.parametrize("n_boards,k", [(5, 3), (1, 1), (33, 2)])
def test_wave_specialised_and_generic_kernels_agree(name, n_boards, k):
    """bf16 rollouts run by the wave-specialised kernel (default) and by the generic kernel,
    for odd row counts (a partial last workgroup, an empty row group): one step from the same
    state (the 24-step state of each) matches the oracle's step within 2e-2, fired counts are
    exact, the 24-step states stay within 1.5x the oracle's own drift under another summation
    order, and the two kernels agree bit for bit where they sum in the same order."""
    from ncas_amd import _lib

    _say("ws vs generic", name, n_boards, k)
    m, md, x, g4, cl = _case(name, n_boards=n_boards, k=k)
    cell = oracle_cell(m)
    B, C, H, W = x.shape
    xr, fr = O.rollout(cell, x, g4, cl, 24, "bf16", seed=4, p_fire=0.6)
    out = {}
    L = _lib.load()
    try:
        for path in (0, 1):
            assert L.nca_set_kernel_path(path) == 0
            with torch.no_grad():
                y, conf, f = rollout_steps(md, x.to(DEV), g4.to(DEV), cl.to(DEV), 24, seed=4,
                                           p_fire=0.6, precision="bf16", want_fired=True)
                y1, _, _ = rollout_steps(md, y, g4.to(DEV), cl.to(DEV), 1, seed=4, step0=24,
                                         p_fire=0.6, precision="bf16")
            out[path] = (y.cpu(), conf.cpu(), f.cpu())
            ref1 = O.step(cell, y.cpu(), g4, cl, O.fire_masks_np(4, 0, B, 24, H, W, 0.6), "bf16")
            assert (y1.cpu() - ref1).abs().max().item() <= TOL["bf16"], path
    finally:
        L.nca_set_kernel_path(0)
    guard = drift_guard(f"ws24/{name}/{n_boards}x{k}")
    _say("drift per path", [(out[p][0] - xr).abs().max().item() for p in (0, 1)], "guard",
         guard, "between paths", (out[0][0] - out[1][0]).abs().max().item())
    for path in (0, 1):
        # 24 bf16 steps from the same state: within 1.5x the oracle's own drift under another fp32
        # summation order
        assert (out[path][0] - xr).abs().max().item() <= guard, path
        assert torch.equal(out[path][2].long(), fr), path
    if name == "sudoku_c64":  # the C=64 kernels sum fc1 / fc2 in different orders
        assert (out[0][0] - out[1][0]).abs().max().item() <= guard
    else:  # the C=16 / C=32 wave-specialised and generic kernels sum in the same order
        assert torch.equal(out[0][0], out[1][0])
