"""Parity of the halo-tiled per-step kernel (grids whose rows do not fit one workgroup's LDS), on
the GPU through the C ABI.

* On grids the resident kernel also takes, the tiled path (nca_set_kernel_path(2)) gives the
  generic resident kernel's results bit for bit: same states, fired counts and confidences.
* On the configurations that need it - 201x201 mazes with the C=16 cell, 30x30 hard mazes with
  the C=32 cell and confidence-gated firing - and on ragged grids whose windows end mid-row,
  states stay within max-abs 1e-4 (fp32) / 2e-2 (bf16) of the CPU oracle with the same Philox
  masks, and fired counts are exact.
* bf16 cells with 16 channels run the per-step path on the wave-per-tile kernel; it gives the
  halo-window kernel's results (nca_set_kernel_path(3)) bit for bit on every padding and on grids
  whose last tile ends mid-row, with Philox, per-step-key and injected masks.
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
from ncas_amd.rng import fire_desc  # noqa: E402
from ncas_amd.step import make_step  # noqa: E402
from ncas_amd.tasks import maze_boards  # noqa: E402
from oracle import clib  # noqa: E402
from oracle import nca_oracle as O  # noqa: E402

pytestmark = pytest.mark.gpu
TOL = {"fp32": 1e-4, "bf16": 2e-2}
DEV = torch.device("cuda:0")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    clib.build()
    yield
    _lib.load().nca_set_kernel_path(0)


def _say(*a):
    print(*a, flush=True)


class _path:
    """Kernel selection for the duration of a block (restored to automatic afterwards)."""

    def __init__(self, path):
        self.path = path

    def __enter__(self):
        assert _lib.load().nca_set_kernel_path(self.path) == 0

    def __exit__(self, *exc):
        _lib.load().nca_set_kernel_path(0)


def _maze_case(preset, n, size, k=1, seed=0, sigma=0.15, extra=0.0, **overrides):
    m = perturbed_model(preset, seed, *DYN[preset], **overrides)
    b = maze_boards(n, size, seed, extra_openings=extra)
    x, g4, cl = initial_state(m, b, k=k, sigma=sigma, seed=seed)
    return m, copy.deepcopy(m).to(DEV), x, g4, cl


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
@pytest.mark.parametrize("name", ["maze_c16", "sudoku_c64", "maze_hard_c32", "ref_maze_ood"])
def test_tiled_equals_generic_resident_bitwise(name, precision):
    _say("tiled vs generic", name, precision)
    preset, size = CELLS[name]
    m = make_model(name)
    md = copy.deepcopy(m).to(DEV)
    x, g4, cl = initial_state(m, boards_for(preset, 3, size, 1), k=5, sigma=0.15, seed=1)
    xd, gd, cd = x.to(DEV), g4.to(DEV), cl.to(DEV)
    out = {}
    for path in (1, 2):
        with _path(path), torch.no_grad():
            out[path] = rollout_steps(md, xd, gd, cd, 17, seed=9, row0=4, step0=2, p_fire=0.6,
                                      precision=precision, want_fired=True)
    for a, b in zip(out[1], out[2]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_tiled_201x201_maze_matches_oracle(precision):
    """The 201x201 C=16 maze cell (windows 16x32 with halos from the neighbouring windows):
    8 fused steps against the oracle, and fused == chained single steps."""
    _say("201x201", precision)
    m, md, x, g4, cl = _maze_case("maze_c16", 2, 201)
    cell = oracle_cell(m)
    xr, fr = O.rollout(cell, x, g4, cl, 8, precision, seed=3, row0=1, p_fire=0.5)
    xd, gd, cd = x.to(DEV), g4.to(DEV), cl.to(DEV)
    with torch.no_grad():
        y, conf, f = rollout_steps(md, xd, gd, cd, 8, seed=3, row0=1, p_fire=0.5,
                                   precision=precision, want_fired=True)
        cur = xd
        for t in range(8):
            cur, _, _ = rollout_steps(md, cur, gd, cd, 1, seed=3, row0=1, step0=t, p_fire=0.5,
                                      precision=precision, want_conf=False)
    err = (y.cpu() - xr).abs().max().item()
    _say("max-abs", err)
    assert err <= TOL[precision]
    assert torch.equal(f.cpu().long(), fr)
    assert torch.equal(y, cur)
    _, rb, _ = O.readout(cell, y.cpu())
    assert np.array_equal(conf.cpu().numpy().view(np.int32), rb.view(np.int32))


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_tiled_hard_maze_30x30_gated_firing_step_by_step(precision):
    """The 30x30 C=32 hard-maze cell with confidence-gated firing (p_low = 0.25 p, tau = 0.9 as
    configured, and a tau at the median confidence so that both branches occur): from the same
    state the GPU draws the oracle's mask bit for bit and each step matches the oracle's."""
    _say("30x30 gated", precision)
    m, md, x, g4, cl = _maze_case("maze_hard_c32", 3, 30, k=2, extra=0.10)
    cell = oracle_cell(m)
    p = 0.8
    cc0, _, _ = O.readout(cell, x)
    for tau in (0.9, float(np.median(cc0))):
        cur = x.clone()
        for t in range(6):
            with torch.no_grad():
                y, _, f = rollout_steps(md, cur.to(DEV), g4.to(DEV), cl.to(DEV), 1, seed=2, step0=t,
                                        p_fire=p, p_low=0.25 * p, tau=tau, precision=precision,
                                        want_fired=True)
            yr, fr = O.rollout(cell, cur, g4, cl, 1, precision, seed=2, step0=t, p_fire=p,
                               p_low=0.25 * p, tau=tau)
            assert torch.equal(f.cpu().long(), fr), (tau, t)
            assert (y.cpu() - yr).abs().max().item() <= TOL[precision], (tau, t)
            cur = y.cpu()


@pytest.mark.parametrize("padding", ["zero", "wall", "wrap"])
@pytest.mark.parametrize("H,W", [(37, 45), (5, 70), (33, 1)])
def test_tiled_ragged_grids_and_paddings(H, W, padding):
    """Windows that end mid-row and mid-column, every padding rule; 5 fp32 steps + the given
    cells' clamp, against the oracle."""
    _say("ragged", H, W, padding)
    kw = {"padding": padding}
    if padding != "wall":
        kw["wall_token"] = None
    m = perturbed_model("maze_hard_c32", 1, *DYN["maze_hard_c32"], **kw)
    md = copy.deepcopy(m).to(DEV)
    g = torch.Generator().manual_seed(H * 100 + W)
    B = 3
    x = torch.randn((B, 32, H, W), generator=g) * 0.3
    g4 = torch.rand((B, 1, H, W), generator=g) < 0.3
    cl = torch.randn((B, m.cfg.c_in, H, W), generator=g)
    xr, fr = O.rollout(oracle_cell(m), x, g4, cl, 5, "fp32", seed=6, p_fire=0.7)
    with _path(2), torch.no_grad():
        y, _, f = rollout_steps(md, x.to(DEV), g4.to(DEV), cl.to(DEV), 5, seed=6, p_fire=0.7,
                                want_fired=True)
    assert (y.cpu() - xr).abs().max().item() <= TOL["fp32"]
    assert torch.equal(f.cpu().long(), fr)


def test_tiled_single_step_with_noise_and_injected_mask():
    _say("tiled step + noise")
    m, md, x, g4, cl = _maze_case("maze_c16", 2, 41)
    B, C, H, W = x.shape
    g = torch.Generator().manual_seed(5)
    fire = (torch.rand((B, 1, H, W), generator=g) < 0.5).float()
    noise = torch.randn(x.shape, generator=g) * 0.2
    step = make_step(md, precision="fp32")
    with _path(2), torch.no_grad():
        y = step(x.to(DEV), g4.to(DEV), cl.to(DEV), fire.to(DEV), noise.to(DEV)).cpu()
    ref = O.step(oracle_cell(m), x, g4, cl, fire, "fp32", noise)
    assert (y - ref).abs().max().item() <= TOL["fp32"]


def test_tiled_workspace_alias_and_errors():
    """Through the raw ABI: in-place rollouts (odd and even step counts) equal out-of-place
    ones, a missing workspace is refused with NCA_ERR_UNSUPPORTED, a zero-step call copies."""
    _say("workspace")
    m, md, x, g4, cl = _maze_case("maze_c16", 2, 61)
    L = _lib.load()
    pk = md.packed("fp32", DEV)
    B, C, H, W = x.shape
    xd, g8, cd = x.to(DEV), g4.to(torch.uint8).to(DEV), cl.to(DEV)
    ws_bytes = L.nca_rollout_workspace_bytes(ctypes.byref(pk.desc), B, H, W)
    assert ws_bytes == 2 * B * C * H * W * 4
    ws = torch.empty(ws_bytes // 4, device=DEV)
    st = _lib.stream_of(DEV)
    fd = fire_desc(4, 0.5)

    def run(src, dst, n, work=ws, nbytes=ws_bytes):
        return L.nca_rollout_ws(ctypes.byref(pk.desc), pk.buf.data_ptr(), B, H, W, src.data_ptr(),
                                g8.data_ptr(), cd.data_ptr(), dst.data_ptr(), ctypes.byref(fd), n,
                                None, None, None, None if work is None else work.data_ptr(),
                                nbytes, st)

    refs = {0: xd}
    for n in (1, 2, 3, 4, 5):
        ref = torch.empty_like(xd)
        assert run(xd, ref, n) == 0
        inplace = xd.clone()
        assert run(inplace, inplace, n) == 0
        torch.cuda.synchronize()
        assert torch.equal(ref, inplace), n
        assert not torch.equal(ref, refs[n - 1]), n
        refs[n] = ref
    half = torch.empty_like(xd)
    assert run(xd, half, 2, ws, ws_bytes // 2) == 0  # two steps need one buffer
    torch.cuda.synchronize()
    assert torch.equal(half, refs[2])
    out = torch.empty_like(xd)
    assert run(xd, out, 3, ws, ws_bytes // 2) == _lib.NCA_ERR_UNSUPPORTED
    assert run(xd, out, 3, None, 0) == _lib.NCA_ERR_UNSUPPORTED
    assert b"workspace" in L.nca_last_error()
    assert run(xd, out, 1, None, 0) == 0  # one out-of-place step needs none
    assert run(xd, out, 0, None, 0) == 0
    torch.cuda.synchronize()
    assert torch.equal(out, xd)
    # the resident kernels need no workspace
    pk9 = copy.deepcopy(make_model("sudoku_c64")).to(DEV).packed("bf16", DEV)
    assert L.nca_rollout_workspace_bytes(ctypes.byref(pk9.desc), 32768, 9, 9) == 0


@pytest.mark.parametrize("padding", ["zero", "wall", "wrap"])
@pytest.mark.parametrize("H,W,B", [(201, 201, 2), (37, 45, 3), (5, 70, 3), (33, 1, 3), (3, 2, 5)])
def test_wave_tile_kernel_equals_window_kernel_bitwise(H, W, B, padding):
    """bf16 C=16: 6 steps (first and last in the caller's layout, the ones between cell-major) and
    single steps, on the wave-per-tile kernel (path 2) and the halo-window kernel (path 3): the
    same states and fired counts bit for bit."""
    _say("wave tiles vs windows", H, W, padding)
    kw = {"padding": padding}
    if padding != "wall":
        kw["wall_token"] = None
    m = perturbed_model("maze_c16", 2, *DYN["maze_c16"], **kw)
    md = copy.deepcopy(m).to(DEV)
    g = torch.Generator().manual_seed(H * 1000 + W)
    x = (torch.randn((B, 16, H, W), generator=g) * 0.3).to(DEV)
    g4 = (torch.rand((B, 1, H, W), generator=g) < 0.3).to(DEV)
    cl = torch.randn((B, m.cfg.c_in, H, W), generator=g).to(DEV)
    masks = (torch.rand((6, B, 1, H, W), generator=g) < 0.5).float().to(DEV)
    runs = [dict(seed=4, row0=2, step0=3, p_fire=0.6), dict(step_seeds=[5, 6, 7, 8, 9, 10], p_fire=0.5),
            dict(masks=masks)]
    for kwr in runs:
        out = {}
        for path in (2, 3):
            with _path(path), torch.no_grad():
                y, _, f = rollout_steps(md, x, g4, cl, 6, precision="bf16", want_fired=True, **kwr)
                y1, _, f1 = rollout_steps(md, x, g4, cl, 1, precision="bf16", want_fired=True,
                                          **{k: (v[:1] if k in ("masks", "step_seeds") else v)
                                             for k, v in kwr.items()})
            out[path] = (y, f, y1, f1)
        for a, b in zip(out[2], out[3]):
            assert torch.equal(a, b), kwr


def test_wave_tile_kernel_guard_for_more_than_2_to_26_cells():
    """The wave-per-tile kernel addresses the cell-major state with 32-bit byte offsets; calls
    with rows * H * W * 64 >= 2^32 (1,664 boards of 201x201, 4.3 GB per state) take the
    halo-window kernel instead. The last boards of such a call equal the same boards run alone
    (on the wave-per-tile kernel) bit for bit, over two steps (the second reads the cell-major
    workspace)."""
    B, H, W = 1664, 201, 201
    assert B * H * W * 64 >= 2**32
    _say("offset guard", B, H, W)
    m = perturbed_model("maze_c16", 2, *DYN["maze_c16"])
    md = copy.deepcopy(m).to(DEV)
    g = torch.Generator(device=DEV).manual_seed(11)
    with torch.no_grad():
        x = torch.randn((B, 16, H, W), generator=g, device=DEV) * 0.3
        g4 = torch.rand((B, 1, H, W), generator=g, device=DEV) < 0.3
        cl = torch.randn((B, m.cfg.c_in, H, W), generator=g, device=DEV)
        y, _, _ = rollout_steps(md, x, g4, cl, 2, seed=5, row0=3, p_fire=0.5, precision="bf16",
                                want_conf=False)
        tail = slice(B - 2, B)
        y2, _, _ = rollout_steps(md, x[tail].contiguous(), g4[tail].contiguous(), cl[tail].contiguous(), 2,
                                 seed=5, row0=3 + B - 2, p_fire=0.5, precision="bf16", want_conf=False)
        assert torch.equal(y[tail], y2)
        del x, y
        torch.cuda.empty_cache()
