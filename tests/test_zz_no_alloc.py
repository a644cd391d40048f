"""The allocation-free entry point nca_rollout_noalloc, through the C ABI, on the GPU: its results
equal nca_rollout_ws's (the same call with a caller workspace) bit for bit - states, board
confidences and fired counts - on two calls in a row, the second with a smaller input, on the
per-step path (201x201 mazes, bf16 wave-per-tile kernel and fp32 halo-window kernel, an
in-place single step) and on a resident-kernel grid; a call whose workspace would exceed the
scratch is refused with NCA_ERR_UNSUPPORTED before anything runs."""

from __future__ import annotations

import copy
import ctypes
import sys

import numpy as np
import pytest
import torch

sys.path.insert(0, __file__.rsplit("/", 1)[0])
from cells import DYN, initial_state, perturbed_model  # noqa: E402

from ncas_amd import _lib  # noqa: E402
from ncas_amd.rng import fire_desc  # noqa: E402
from ncas_amd.tasks import maze_boards, sudoku_boards  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _say(*a):
    print(*a, flush=True)


def _inputs(preset, n, size):
    m = perturbed_model(preset, 0, *DYN[preset])
    b = sudoku_boards(n, 0) if preset.startswith("sudoku") else maze_boards(n, size, 0)
    x, g4, cl = initial_state(m, b, k=1, sigma=0.15)
    return copy.deepcopy(m).to(DEV), x.to(DEV), g4.to(DEV).to(torch.uint8).contiguous(), cl.to(DEV)


def _call(md, precision, x, g8, cl, n_steps, noalloc, out=None, seed=5):
    """One rollout through the C ABI; returns (x_out, conf, fired)."""
    L = _lib.load()
    pk = md.packed(precision, DEV)
    B, C, H, W = x.shape
    y = torch.empty_like(x) if out is None else out
    conf = torch.empty(B, dtype=torch.float32, device=DEV)
    fired = torch.empty(B, dtype=torch.int32, device=DEV)
    fd = fire_desc(seed, 0.5, None, None, True, 3, 7)
    stream = _lib.stream_of(DEV)
    args = (ctypes.byref(pk.desc), pk.buf.data_ptr(), B, H, W, x.data_ptr(), g8.data_ptr(),
            cl.data_ptr(), y.data_ptr(), ctypes.byref(fd), n_steps, None, conf.data_ptr(),
            fired.data_ptr())
    if noalloc:
        rc = L.nca_rollout_noalloc(*args, stream)
    else:
        nb = L.nca_rollout_workspace_bytes(ctypes.byref(pk.desc), B, H, W)
        ws = torch.empty(max(nb, 4) // 4, dtype=torch.float32, device=DEV)
        rc = L.nca_rollout_ws(*args, ws.data_ptr(), nb, stream)
    _lib.check(rc, "nca_rollout_noalloc" if noalloc else "nca_rollout_ws")
    return y, conf, fired


@pytest.mark.parametrize("preset,precision,size", [("maze_c16", "bf16", 201),
                                                    ("maze_c16", "fp32", 201),
                                                    ("sudoku_c64", "bf16", 9)])
def test_noalloc_equals_the_workspace_call_twice(preset, precision, size):
    _say("noalloc", preset, precision, size)
    md, x, g8, cl = _inputs(preset, 3, size)
    for rows, n_steps in ((3, 6), (1, 4)):  # the second call is smaller
        xs, gs, cs = x[:rows].contiguous(), g8[:rows].contiguous(), cl[:rows].contiguous()
        ref = _call(md, precision, xs, gs, cs, n_steps, noalloc=False)
        got = _call(md, precision, xs, gs, cs, n_steps, noalloc=True)
        torch.cuda.synchronize()
        for a, b in zip(got, ref):
            assert torch.equal(a, b), (rows, n_steps)
        _say("rows", rows, "steps", n_steps, "equal")


def test_noalloc_in_place_single_step():
    md, x, g8, cl = _inputs("maze_c16", 2, 201)
    ref = _call(md, "bf16", x, g8, cl, 1, noalloc=False)
    y = x.clone()
    got = _call(md, "bf16", y, g8, cl, 1, noalloc=True, out=y)
    torch.cuda.synchronize()
    assert torch.equal(got[0], ref[0]) and torch.equal(got[2], ref[2])


def test_noalloc_refuses_calls_beyond_the_scratch():
    """32 boards of 201 x 201 x 16 fp32 need two 83 MB state buffers: refused before any work
    (the pointers are never read), and the message names the limit."""
    md, x, g8, cl = _inputs("maze_c16", 1, 201)
    L = _lib.load()
    pk = md.packed("bf16", DEV)
    rows = 32
    need = 2 * rows * 16 * 201 * 201 * 4
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    fd = fire_desc(1, 0.5)
    rc = L.nca_rollout_noalloc(ctypes.byref(pk.desc), pk.buf.data_ptr(), rows, 201, 201,
                               x.data_ptr(), g8.data_ptr(), cl.data_ptr(), x.data_ptr(),
                               ctypes.byref(fd), 5, None, None, None, _lib.stream_of(DEV))
    assert rc == _lib.NCA_ERR_UNSUPPORTED
    msg = L.nca_last_error().decode()
    assert "scratch" in msg and str(_lib.NOALLOC_SCRATCH_BYTES) in msg, msg
    # the largest call that fits still runs on the same scratch
    assert 2 * 20 * 16 * 201 * 201 * 4 <= _lib.NOALLOC_SCRATCH_BYTES
