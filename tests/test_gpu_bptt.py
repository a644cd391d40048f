"""The BPTT chunk on the GPU (nca_bptt_forward / nca_bptt_backward through the C ABI) against the
fp64 autograd oracle (the engine around it is tested in test_gpu_train.py).

* fp32 cells: loss and every parameter gradient (and d L / d x0) within a relative norm error
  of 1e-4 of the oracle over multi-step chunks with sparse step weights, a loss mask, wall /
  wrap padding and injected or Philox fire masks.
* bf16 cells: the single-step vector-Jacobian product from the GPU's own state (so that both
  sides differentiate the same rounded operands) within 1e-3; multi-step chunks within 1e-2
  of the oracle (a bf16 rounding flip in the forward moves a state by up to 2e-2). The oracle
  rounds the gradients of dx, h and z to bf16 (`grad_round`) as the reference's bf16 backward
  does (src/nca/engine/triton_mlp.py:46-78), like the kernels.
* The chunk's saved states are the rollout kernels' states bit for bit; gradients are
  bitwise reproducible; chaining two chunks through grad_final / grad_x0 equals one chunk.
"""

from __future__ import annotations

import copy
import ctypes
import sys

import numpy as np
import pytest
import torch

sys.path.insert(0, __file__.rsplit("/", 1)[0])
from cells import CELLS, DYN, boards_for, initial_state, make_model, oracle_cell, perturbed_model  # noqa: E402

from ncas_amd import _lib  # noqa: E402
from ncas_amd.inference import rollout_steps  # noqa: E402
from ncas_amd.tasks import maze_boards  # noqa: E402
from ncas_amd.train import bptt_chunk  # noqa: E402
from oracle import nca_oracle as O  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
NAMES = ("kernels", "w1", "b1", "w2", "b2", "head_w", "head_b")


def _say(*a):
    print(*a, flush=True)


def _rel(a, b):
    a = a.detach().double().cpu().reshape(-1)
    b = b.detach().double().cpu().reshape(-1)
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def _case(name, n_boards=2, k=2, steps=5, seed=0):
    preset, size = CELLS[name]
    m = make_model(name, seed)
    b = boards_for(preset, n_boards, size, seed)
    x, g4, cl = initial_state(m, b, k=k, sigma=0.15, seed=seed)
    B, C, H, W = x.shape
    g = torch.Generator().manual_seed(seed + 3)
    masks = (torch.rand((steps, B, 1, H, W), generator=g) < 0.6).float()
    targets = torch.randint(0, len(m.cfg.output_tokens), (B, H, W), generator=g)
    return m, copy.deepcopy(m).to(DEV), x, g4, cl, masks, targets


def _gpu_chunk(md, x, g4, cl, targets, weights, precision, **kw):
    with torch.no_grad():
        return bptt_chunk(md, x.to(DEV), g4.to(DEV), cl.to(DEV), targets.to(DEV), weights,
                          precision=precision, want_grad_x0=True, **kw)


@pytest.mark.parametrize("name", ["maze_hard_c32", "maze_c16", "sudoku_c64"])
def test_bptt_fp32_matches_oracle(name):
    _say("bptt fp32", name)
    m, md, x, g4, cl, masks, targets = _case(name)
    weights = [1.0, 0.0, 0.5, 0.0, 1.0]
    lm = (torch.rand(targets.shape, generator=torch.Generator().manual_seed(9)) < 0.8).float()
    for mask in (None, lm):
        res = _gpu_chunk(md, x, g4, cl, targets, weights, "fp32", masks=masks.to(DEV),
                         loss_mask=None if mask is None else mask.to(DEV))
        loss, ref = O.bptt_chunk(oracle_cell(m), x, g4, cl, masks.double(), targets, weights,
                                 "fp32", loss_mask=mask, grad_x0=True)
        assert abs(float(res.loss) - loss) <= 1e-5 * abs(loss), (float(res.loss), loss)
        for k in NAMES:
            assert _rel(res.grads[k], ref[k]) <= 1e-4, (k, _rel(res.grads[k], ref[k]))
        assert _rel(res.grad_x0, ref["x0"]) <= 1e-4


def test_bptt_philox_masks_and_step_seeds():
    """Fire masks drawn in-kernel from per-step keys are the oracle's Philox masks."""
    m, md, x, g4, cl, _, targets = _case("maze_hard_c32", steps=4)
    B, C, H, W = x.shape
    seeds = [11, 2**40 + 3, 7, 99]
    masks = torch.stack([O.fire_masks_np(s, 5, B, 20 + t, H, W, 0.7) for t, s in enumerate(seeds)])
    res = _gpu_chunk(md, x, g4, cl, targets, [1, 1, 1, 1], "fp32", step_seeds=seeds, p_fire=0.7,
                     row0=5, step0=20)
    loss, ref = O.bptt_chunk(oracle_cell(m), x, g4, cl, masks.double(), targets, [1, 1, 1, 1],
                             "fp32", grad_x0=True)
    assert abs(float(res.loss) - loss) <= 1e-5 * abs(loss)
    for k in NAMES:
        assert _rel(res.grads[k], ref[k]) <= 1e-4, k


@pytest.mark.parametrize("name", ["maze_hard_c32", "sudoku_c64"])
def test_bptt_bf16_single_step_vjp_from_the_gpu_state(name):
    _say("bptt bf16 vjp", name)
    m, md, x, g4, cl, masks, targets = _case(name, steps=4)
    with torch.no_grad():
        xs, _, _ = rollout_steps(md, x.to(DEV), g4.to(DEV), cl.to(DEV), 6, seed=3, precision="bf16")
    xs = xs.cpu()
    cot = torch.randn(xs.shape, generator=torch.Generator().manual_seed(4)) * 0.01
    res = _gpu_chunk(md, xs, g4, cl, targets, [1.0], "bf16", masks=masks[:1].to(DEV),
                     grad_final=cot.to(DEV))
    loss, ref = O.bptt_chunk(oracle_cell(m), xs, g4, cl, masks[:1].double(), targets, [1.0],
                             "bf16", grad_x0=True, final_cotangent=cot.double(), grad_round=True)
    worst = max(_rel(res.grads[k], ref[k]) for k in NAMES)
    _say("bf16 vjp worst rel", worst, "x0", _rel(res.grad_x0, ref["x0"]))
    assert worst <= 1e-3
    assert _rel(res.grad_x0, ref["x0"]) <= 1e-3


@pytest.mark.parametrize("name", ["maze_hard_c32", "maze_c16"])
def test_bptt_bf16_chunk_near_oracle(name):
    m, md, x, g4, cl, masks, targets = _case(name, steps=5)
    weights = [0.5, 0.0, 1.0, 0.0, 1.0]
    res = _gpu_chunk(md, x, g4, cl, targets, weights, "bf16", masks=masks.to(DEV))
    loss, ref = O.bptt_chunk(oracle_cell(m), x, g4, cl, masks.double(), targets, weights, "bf16",
                             grad_x0=True, grad_round=True)
    worst = max(_rel(res.grads[k], ref[k]) for k in NAMES)
    _say("bf16 chunk worst rel", worst, "loss", float(res.loss), loss)
    assert abs(float(res.loss) - loss) <= 1e-4 * abs(loss)
    assert worst <= 1e-2


@pytest.mark.parametrize("fire", ["seed", "step_seeds", "masks"])
@pytest.mark.parametrize("size", [30, 13])
def test_bptt_forward_records_every_rollout_state(fire, size):
    """nca_bptt_forward runs a bf16 C=32 chunk as one fused launch of the streamed kernel that
    writes the state after every step: state t equals a t-step rollout bit for bit, with Philox
    keys, per-step keys or injected masks, on a 30x30 maze and on a 13x13 grid."""
    from ncas_amd.rng import fire_desc
    _say("bptt forward states", fire, size)
    m = perturbed_model("maze_hard_c32", 2, *DYN["maze_hard_c32"])
    b = maze_boards(3, size, 2, extra_openings=0.1)
    x, g4, cl = initial_state(m, b, k=2, sigma=0.15, seed=2)
    md = copy.deepcopy(m).to(DEV)
    B, C, H, W = x.shape
    n = 7
    xd, gd, cd = x.to(DEV), g4.to(DEV), cl.to(DEV)
    kw = dict(seed=5, p_fire=0.7, row0=3, step0=4)
    ss = m8 = None
    if fire == "step_seeds":
        kw["step_seeds"] = [9, 2**41 + 1, 3, 4, 5, 6, 7]
        ss = torch.as_tensor(np.asarray(kw["step_seeds"], dtype=np.int64)).to(DEV)
    if fire == "masks":
        g = torch.Generator().manual_seed(7)
        masks = (torch.rand((n, B, 1, H, W), generator=g) < 0.5).float().to(DEV)
        m8 = (masks != 0).to(torch.uint8).contiguous()
    fd = fire_desc(kw["seed"], kw["p_fire"], None, None, True, kw["row0"], kw["step0"], ss, m8)
    pk = md.packed("bf16", DEV)
    states = torch.full((n + 1, B, C, H, W), float("nan"), device=DEV)
    g8 = gd.to(torch.uint8).contiguous()
    L = _lib.load()
    _lib.check(L.nca_bptt_forward(ctypes.byref(pk.desc), pk.buf.data_ptr(), B, H, W, xd.data_ptr(),
                                  g8.data_ptr(), cd.data_ptr(), ctypes.byref(fd), n,
                                  states.data_ptr(), _lib.stream_of(DEV)), "nca_bptt_forward")
    torch.cuda.synchronize()
    assert torch.equal(states[0], xd)
    with torch.no_grad():
        for t in range(1, n + 1):
            if fire == "masks":
                y, _, _ = rollout_steps(md, xd, gd, cd, t, masks=masks[:t], precision="bf16")
            else:
                kwt = dict(kw)
                if "step_seeds" in kwt:
                    kwt["step_seeds"] = kwt["step_seeds"][:t]
                y, _, _ = rollout_steps(md, xd, gd, cd, t, precision="bf16", **kwt)
            assert torch.equal(states[t], y), t


@pytest.mark.parametrize("fire", ["seed", "step_seeds", "masks"])
@pytest.mark.parametrize("hw", [(30, 30), (20, 30), (25, 30), (30, 20)])
def test_bptt_forward_in_pieces_equals_whole_boards(fire, hw):
    """nca_bptt_forward_ws with a workspace runs each board in pieces of rows on two or three
    workgroups (30x30: three pieces of 10 rows; 20x30 and 30x20: two equal pieces; 25x30: pieces
    of 13 and 12 rows) that exchange their boundary rows every step: every recorded state equals
    the whole-board forward's bit for bit, with Philox keys, per-step keys or injected masks."""
    from ncas_amd.rng import fire_desc
    H, W = hw
    _say("bptt forward pieces", fire, H, W)
    m = perturbed_model("maze_hard_c32", 3, *DYN["maze_hard_c32"])
    b = maze_boards(4, 30, 3, extra_openings=0.1)
    x, g4, cl = initial_state(m, b, k=2, sigma=0.15, seed=3)
    x, g4, cl = (t[:, :, :H, :W].contiguous() for t in (x, g4, cl))
    md = copy.deepcopy(m).to(DEV)
    B, C = x.shape[:2]
    n = 9
    xd, cd = x.to(DEV), cl.to(DEV)
    g8 = g4.to(DEV).to(torch.uint8).contiguous()
    ss = m8 = None
    if fire == "step_seeds":
        ss = torch.as_tensor(np.arange(11, 11 + n, dtype=np.int64) * (2**33 + 7)).to(DEV)
    if fire == "masks":
        g = torch.Generator().manual_seed(8)
        m8 = (torch.rand((n, B, 1, H, W), generator=g) < 0.6).to(torch.uint8).to(DEV).contiguous()
    fd = fire_desc(6, 0.7, None, None, True, 2, 5, ss, m8)
    pk = md.packed("bf16", DEV)
    L = _lib.load()
    ws_bytes = L.nca_bptt_workspace_bytes(ctypes.byref(pk.desc), B, H, W, n)
    assert ws_bytes > 0
    ws = torch.full((ws_bytes // 4,), float("nan"), device=DEV)
    # two calls on the same workspace: the second, from another state, finds the first one's
    # exchange words there (tagged with the same steps) unless the call clears them
    for x0 in (xd, (xd * 0.5 + 0.25).contiguous()):
        whole = torch.full((n + 1, B, C, H, W), float("nan"), device=DEV)
        _lib.check(L.nca_bptt_forward(ctypes.byref(pk.desc), pk.buf.data_ptr(), B, H, W,
                                      x0.data_ptr(), g8.data_ptr(), cd.data_ptr(), ctypes.byref(fd),
                                      n, whole.data_ptr(), _lib.stream_of(DEV)), "nca_bptt_forward")
        pieces = torch.full((n + 1, B, C, H, W), float("nan"), device=DEV)
        _lib.check(L.nca_bptt_forward_ws(ctypes.byref(pk.desc), pk.buf.data_ptr(), B, H, W,
                                         x0.data_ptr(), g8.data_ptr(), cd.data_ptr(),
                                         ctypes.byref(fd), n, pieces.data_ptr(), ws.data_ptr(),
                                         ws_bytes, _lib.stream_of(DEV)), "nca_bptt_forward_ws")
        torch.cuda.synchronize()
        assert not torch.isnan(whole).any()
        for t in range(n + 1):
            assert torch.equal(pieces[t], whole[t]), t


@pytest.mark.parametrize("padding,n,rows", [("zero", 1, 8), ("zero", 2, 8), ("wall", 3, 100), ("wall", 2, 130)])
def test_bptt_forward_in_pieces_edges(padding, n, rows):
    """Random 30x30 states: chunks of 1 step (no exchange) and 2 (one exchange) with zero
    padding; 100 rows (three pieces would need 300 CUs, so fewer) and 130 rows (whole boards on a
    256-CU device). nca_bptt_forward_ws records the whole-board forward's states bit for bit."""
    from ncas_amd.rng import fire_desc
    _say("bptt forward pieces edges", padding, n, rows)
    kw = {"padding": padding}
    if padding != "wall":
        kw["wall_token"] = None
    m = perturbed_model("maze_hard_c32", 5, *DYN["maze_hard_c32"], **kw)
    md = copy.deepcopy(m).to(DEV)
    g = torch.Generator().manual_seed(rows * 10 + n)
    H = W = 30
    x = (torch.randn((rows, 32, H, W), generator=g) * 0.3).to(DEV)
    g8 = (torch.rand((rows, 1, H, W), generator=g) < 0.3).to(torch.uint8).to(DEV).contiguous()
    cl = torch.randn((rows, m.cfg.c_in, H, W), generator=g).to(DEV)
    fd = fire_desc(9, 0.7, None, None, True, 0, 3, None, None)
    pk = md.packed("bf16", DEV)
    L = _lib.load()
    whole = torch.full((n + 1, rows, 32, H, W), float("nan"), device=DEV)
    _lib.check(L.nca_bptt_forward(ctypes.byref(pk.desc), pk.buf.data_ptr(), rows, H, W, x.data_ptr(),
                                  g8.data_ptr(), cl.data_ptr(), ctypes.byref(fd), n, whole.data_ptr(),
                                  _lib.stream_of(DEV)), "nca_bptt_forward")
    ws_bytes = L.nca_bptt_workspace_bytes(ctypes.byref(pk.desc), rows, H, W, n)
    ws = torch.full((ws_bytes // 4,), float("nan"), device=DEV)
    pieces = torch.full_like(whole, float("nan"))
    _lib.check(L.nca_bptt_forward_ws(ctypes.byref(pk.desc), pk.buf.data_ptr(), rows, H, W, x.data_ptr(),
                                     g8.data_ptr(), cl.data_ptr(), ctypes.byref(fd), n, pieces.data_ptr(),
                                     ws.data_ptr(), ws_bytes, _lib.stream_of(DEV)), "nca_bptt_forward_ws")
    torch.cuda.synchronize()
    assert not torch.isnan(whole).any()
    for t in range(n + 1):
        assert torch.equal(pieces[t], whole[t]), t


def test_bptt_bf16_odd_cell_count_13x13():
    """bf16 C=32 on 13x13 boards, 3 rows (507 cells: the fused MLP backward's unaligned path, the
    streamed forward): the single-step VJP from the GPU's state within 1e-3 of the oracle and a
    4-step chunk within 1e-2."""
    _say("bptt bf16 13x13")
    m = perturbed_model("maze_hard_c32", 4, *DYN["maze_hard_c32"])
    md = copy.deepcopy(m).to(DEV)
    b = maze_boards(3, 13, 4, extra_openings=0.1)
    x, g4, cl = initial_state(m, b, k=1, sigma=0.15, seed=4)
    targets = m.output_index(torch.from_numpy(b.targets))
    g = torch.Generator().manual_seed(5)
    masks = (torch.rand((4, 3, 1, 13, 13), generator=g) < 0.7).float()
    with torch.no_grad():
        xs, _, _ = rollout_steps(md, x.to(DEV), g4.to(DEV), cl.to(DEV), 5, seed=3, precision="bf16")
    xs = xs.cpu()
    cot = torch.randn(xs.shape, generator=torch.Generator().manual_seed(6)) * 0.01
    res = _gpu_chunk(md, xs, g4, cl, targets, [1.0], "bf16", masks=masks[:1].to(DEV),
                     grad_final=cot.to(DEV))
    loss, ref = O.bptt_chunk(oracle_cell(m), xs, g4, cl, masks[:1].double(), targets, [1.0],
                             "bf16", grad_x0=True, final_cotangent=cot.double(), grad_round=True)
    worst = max(_rel(res.grads[k], ref[k]) for k in NAMES)
    _say("vjp worst rel", worst)
    assert worst <= 1e-3 and _rel(res.grad_x0, ref["x0"]) <= 1e-3
    w = [1.0, 0.0, 0.5, 1.0]
    res = _gpu_chunk(md, x, g4, cl, targets, w, "bf16", masks=masks.to(DEV))
    loss, ref = O.bptt_chunk(oracle_cell(m), x, g4, cl, masks.double(), targets, w, "bf16",
                             grad_x0=True, grad_round=True)
    worst = max(_rel(res.grads[k], ref[k]) for k in NAMES)
    _say("chunk worst rel", worst)
    assert abs(float(res.loss) - loss) <= 1e-4 * abs(loss)
    assert worst <= 1e-2


def test_bptt_states_are_the_rollout_states_and_gradients_are_reproducible():
    m, md, x, g4, cl, masks, targets = _case("maze_hard_c32", steps=6)
    a = _gpu_chunk(md, x, g4, cl, targets, [1] * 6, "bf16", seed=8)
    b = _gpu_chunk(md, x, g4, cl, targets, [1] * 6, "bf16", seed=8)
    with torch.no_grad():
        y, _, _ = rollout_steps(md, x.to(DEV), g4.to(DEV), cl.to(DEV), 6, seed=8, precision="bf16")
    assert torch.equal(a.x, y)
    assert torch.equal(a.loss, b.loss) and torch.equal(a.grad_x0, b.grad_x0)
    for k in NAMES:
        assert torch.equal(a.grads[k], b.grads[k]), k


def test_bptt_chunks_chain_through_grad_final():
    """Steps [0, 6) in one chunk == steps [3, 6) then [0, 3) with the later chunk's d L / d x3
    as grad_final; parameter gradients add up."""
    m, md, x, g4, cl, masks, targets = _case("maze_c16", steps=6)
    w = [1.0, 0.0, 0.5, 1.0, 0.0, 1.0]
    full = _gpu_chunk(md, x, g4, cl, targets, w, "fp32", masks=masks.to(DEV))
    with torch.no_grad():
        x3, _, _ = rollout_steps(md, x.to(DEV), g4.to(DEV), cl.to(DEV), 3, masks=masks[:3].to(DEV))
    s = sum(w)
    late = _gpu_chunk(md, x3, g4, cl, targets, [v / s for v in w[3:]] + [0.0] * 0, "fp32",
                      masks=masks[3:].to(DEV))
    # the later chunk normalises by max(sum(w[3:] / s), 1) = 1: its loss is sum w_t L_t / s
    early = _gpu_chunk(md, x, g4, cl, targets, [v / s for v in w[:3]], "fp32",
                       masks=masks[:3].to(DEV), grad_final=late.grad_x0)
    for k in NAMES:
        assert _rel(early.grads[k] + late.grads[k], full.grads[k]) <= 1e-5, k
    assert _rel(early.grad_x0, full.grad_x0) <= 1e-5
    assert abs(float(early.loss + late.loss) - float(full.loss)) <= 1e-6 * abs(float(full.loss))


def test_bptt_30x30_hard_maze_chunk_matches_oracle():
    """The training configuration's cell and grid (30x30 hard mazes, C=32, halo-tiled forward)
    on 6 boards x 6 steps, fp32, and the memory of the full chunk (64 boards x 32 steps)."""
    _say("bptt 30x30")
    m = perturbed_model("maze_hard_c32", 0, *DYN["maze_hard_c32"])
    md = copy.deepcopy(m).to(DEV)
    b = maze_boards(6, 30, 0, extra_openings=0.1)
    x, g4, cl = initial_state(m, b, k=1, sigma=0.15)
    targets = m.output_index(torch.from_numpy(b.targets))
    g = torch.Generator().manual_seed(1)
    masks = (torch.rand((6, 6, 1, 30, 30), generator=g) < 0.8).float()
    w = [0, 0, 1, 0, 0, 1]
    res = _gpu_chunk(md, x, g4, cl, targets, w, "fp32", masks=masks.to(DEV))
    loss, ref = O.bptt_chunk(oracle_cell(m), x, g4, cl, masks.double(), targets, w, "fp32",
                             grad_x0=True)
    assert abs(float(res.loss) - loss) <= 1e-5 * abs(loss)
    for k in NAMES:
        assert _rel(res.grads[k], ref[k]) <= 1e-4, k
    pk = md.packed("bf16", DEV)
    ws = _lib.load().nca_bptt_workspace_bytes(ctypes.byref(pk.desc), 64, 30, 30, 32)
    states = 33 * 64 * 32 * 900 * 4
    _say(f"full chunk: states {states / 2**20:.1f} MiB + workspace {ws / 2**20:.1f} MiB")
    assert 0 < ws < 512 * 2**20


def _pieces_case(rows, n=4, seed=7):
    from ncas_amd.rng import fire_desc
    m = perturbed_model("maze_hard_c32", seed, *DYN["maze_hard_c32"])
    md = copy.deepcopy(m).to(DEV)
    g = torch.Generator().manual_seed(seed)
    H = W = 30
    x = (torch.randn((rows, 32, H, W), generator=g) * 0.3).to(DEV)
    g8 = (torch.rand((rows, 1, H, W), generator=g) < 0.3).to(torch.uint8).to(DEV).contiguous()
    cl = torch.randn((rows, m.cfg.c_in, H, W), generator=g).to(DEV)
    fd = fire_desc(9, 0.7, None, None, True, 0, 3, None, None)
    return md, md.packed("bf16", DEV), x, g8, cl, fd, n


def _forward(L, pk, x, g8, cl, fd, n, ws=None):
    rows, C, H, W = x.shape
    out = torch.full((n + 1, rows, C, H, W), float("nan"), device=DEV)
    nbytes = 0 if ws is None else ws.numel() * 4
    _lib.check(L.nca_bptt_forward_ws(ctypes.byref(pk.desc), pk.buf.data_ptr(), rows, H, W,
                                     x.data_ptr(), g8.data_ptr(), cl.data_ptr(), ctypes.byref(fd),
                                     n, out.data_ptr(), None if ws is None else ws.data_ptr(),
                                     nbytes, _lib.stream_of(DEV)), "nca_bptt_forward_ws")
    return out


def test_bptt_pieces_status_word():
    """The forward in pieces (64 boards of 30x30: three pieces each) leaves the workspace's status
    word at 0; with the pieces' waits forced to run out (a host setting: every wait looks for a
    tag that never comes and gives up after 4 re-reads) every kernel still ends, the word is 1,
    and the repair launch has recomputed the boards whole: the states still equal the whole-board
    forward's bit for bit. bptt_chunk reports the word as ChunkResult.halo_failed. The one-launch
    backward's pieces give up the same way and its repair launch recomputes the gradients on
    whole boards (ChunkResult.back_repaired): equal to the whole-board path bit for bit."""
    _say("bptt pieces status")
    L = _lib.load()
    md, pk, x, g8, cl, fd, n = _pieces_case(64)
    assert L.nca_bptt_forward_pieces(ctypes.byref(pk.desc), 64, 30, 30, 0) == 3
    ws_bytes = L.nca_bptt_workspace_bytes(ctypes.byref(pk.desc), 64, 30, 30, n)
    ws = torch.full((ws_bytes // 4,), float("nan"), device=DEV)
    whole = _forward(L, pk, x, g8, cl, fd, n)
    good = _forward(L, pk, x, g8, cl, fd, n, ws)
    torch.cuda.synchronize()
    assert int(ws[:1].view(torch.int32).item()) == 0
    assert torch.equal(good, whole)
    targets = torch.zeros((64, 30, 30), dtype=torch.int64, device=DEV)
    ref = bptt_chunk(md, x, g8.bool(), cl, targets, [1.0] * n, seed=9, p_fire=0.7,
                     precision="bf16", want_grad_x0=True)
    try:
        # the one-launch backward on whole boards: what the backward's repair launch computes
        assert L.nca_set_bptt_backward_path(2) == 0
        ref_whole = bptt_chunk(md, x, g8.bool(), cl, targets, [1.0] * n, seed=9, p_fire=0.7,
                               precision="bf16", want_grad_x0=True)
        assert L.nca_set_bptt_backward_path(0) == 0
        assert L.nca_set_piece_debug(4, 1, 0) == 0
        forced = _forward(L, pk, x, g8, cl, fd, n, ws)
        torch.cuda.synchronize()
        assert int(ws[:1].view(torch.int32).item()) == 1
        assert torch.equal(forced, whole)
        # the forward's and the backward's pieces give up; both repair launches run
        res = bptt_chunk(md, x, g8.bool(), cl, targets, [1.0] * n, seed=9, p_fire=0.7,
                         precision="bf16", want_grad_x0=True)
        assert bool(res.halo_failed.all()) and bool(res.back_repaired.all())
        assert torch.equal(res.x, ref.x) and torch.equal(res.grad_x0, ref.grad_x0)
        assert torch.equal(res.loss, ref_whole.loss) and torch.equal(res.grad_x0, ref_whole.grad_x0)
        assert all(torch.equal(res.grads[k], ref_whole.grads[k]) for k in ref.grads)
        for k in NAMES:
            assert _rel(res.grads[k], ref.grads[k]) <= 1e-5, k
    finally:
        L.nca_set_piece_debug(0, 0, 0)
        L.nca_set_bptt_backward_path(0)
    again = _forward(L, pk, x, g8, cl, fd, n, ws)
    torch.cuda.synchronize()
    assert int(ws[:1].view(torch.int32).item()) == 0 and torch.equal(again, whole)
    assert not bool(ref.halo_failed.any()) and not bool(ref.back_repaired.any())


def test_bptt_pieces_not_resident_together():
    """Planned as for a device of 10,000 CUs, 200 boards take three pieces each: 600 workgroups of
    which at most one fits a CU, more than the device holds at once, so the pieces of some boards
    are not resident together. With the waits bounded to 64 re-reads, a piece whose neighbour is
    not resident gives up (the status word is then 1 and the repair recomputes the boards whole);
    either way the states equal the whole-board forward's bit for bit."""
    _say("bptt pieces not resident together")
    L = _lib.load()
    md, pk, x, g8, cl, fd, n = _pieces_case(200, n=3, seed=8)
    whole = _forward(L, pk, x, g8, cl, fd, n)
    try:
        assert L.nca_set_piece_debug(64, 0, 10_000) == 0
        assert L.nca_bptt_forward_pieces(ctypes.byref(pk.desc), 200, 30, 30, 0) == 3
        ws_bytes = L.nca_bptt_workspace_bytes(ctypes.byref(pk.desc), 200, 30, 30, n)
        ws = torch.full((ws_bytes // 4,), float("nan"), device=DEV)
        got = _forward(L, pk, x, g8, cl, fd, n, ws)
        torch.cuda.synchronize()
    finally:
        L.nca_set_piece_debug(0, 0, 0)
    _say("status word", int(ws[:1].view(torch.int32).item()))
    assert torch.equal(got, whole)


def _with_padding(m, padding):
    from dataclasses import replace

    from ncas_amd.model import NCA

    m2 = NCA(replace(m.cfg, padding=padding))
    m2.load_state_dict(m.state_dict())
    return m2


@pytest.mark.parametrize("padding,size,rows,fire", [
    ("wall", 30, 8, "seed"),     # four pieces of 8, 8, 8, 6 rows
    ("wrap", 30, 8, "masks"),    # the top and bottom pieces exchange across the wrap
    ("wall", 13, 6, "masks"),    # pieces of 4, 4, 4 and 1 rows
    ("wrap", 13, 100, "seed"),   # two pieces of 7 and 6 rows (200 workgroups)
    ("wrap", 30, 100, "masks"),  # too many boards for pieces that fit the LDS: whole boards
    ("wall", 30, 300, "seed"),   # more boards than slots: three launches per step
])
def test_bptt_one_launch_backward_equals_per_step_launches(padding, size, rows, fire):
    """The chunk's backward as one launch (bf16 C=32 cells; on pieces of boards exchanging g_z
    rows, or on whole boards) against the same backward as three launches per step: each step's
    per-cell arithmetic is the same in both, so d L / d x0 agrees bit for bit; the parameter
    gradients and the loss are the same sums over cells in another fixed order (fp32 rounding).
    With a loss mask, sparse step weights and grad_final."""
    _say("bptt one-launch backward", padding, size, rows, fire)
    L = _lib.load()
    m = perturbed_model("maze_hard_c32", 3, *DYN["maze_hard_c32"])
    if padding != m.cfg.padding:
        m = _with_padding(m, padding)
    md = copy.deepcopy(m).to(DEV)
    b = maze_boards(rows, size, 0, extra_openings=0.1)
    x, g4, cl = initial_state(m, b, k=1, sigma=0.15, seed=1)
    targets = m.output_index(torch.from_numpy(b.targets))
    n, w = 6, [1.0, 0.0, 0.5, 1.0, 0.0, 1.0]
    g = torch.Generator().manual_seed(5)
    kw = {"grad_final": (torch.randn(x.shape, generator=g) * 1e-3).to(DEV),
          "loss_mask": (torch.rand((rows, size, size), generator=g) < 0.8).float().to(DEV)}
    if fire == "masks":
        kw["masks"] = (torch.rand((n, rows, 1, size, size), generator=g) < 0.7).float().to(DEV)
    else:
        kw["seed"] = 11
    out = {}
    try:
        for path in (1, 0, 2):
            assert L.nca_set_bptt_backward_path(path) == 0
            out[path] = _gpu_chunk(md, x, g4, cl, targets, w, "bf16", **kw)
    finally:
        L.nca_set_bptt_backward_path(0)
    per = out[1]
    for path in (0, 2):
        res = out[path]
        assert torch.equal(res.x, per.x)
        assert torch.equal(res.grad_x0, per.grad_x0), path
        worst = max(_rel(res.grads[k], per.grads[k]) for k in NAMES)
        _say("path", path, "worst rel", worst, "loss", float(res.loss), float(per.loss))
        for k in NAMES:
            assert _rel(res.grads[k], per.grads[k]) <= 1e-5, (path, k)
        assert abs(float(res.loss) - float(per.loss)) <= 1e-6 * abs(float(per.loss))
